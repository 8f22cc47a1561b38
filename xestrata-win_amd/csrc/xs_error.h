// xestrata-win_amd/csrc/xs_error.h - the calling thread's error message (xs_last_error), shared by the C ABI's
// translation units.
#pragma once

#include <string>

namespace xs {
// Sets this thread's message and returns `code`.
int set_error(int code, const std::string& message);
}  // namespace xs
