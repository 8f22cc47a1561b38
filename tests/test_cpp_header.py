"""The engine-facing C++ header (include/xs_strata_kernels.hpp) compiles where the engine would include it, on the CPU:

- stand-alone (no engine headers on the path: its own DeviceError);
- in a translation unit that declares the engine's `class strata::core::DeviceError` itself first (the declaration
  of include/strata/core/device.hpp:66) and says so with XS_STRATA_HAVE_DEVICE_ERROR;
- beside the reference's real include/strata/core/device.hpp, where the reference tree is present (this container);

and a program built against it links with libxsmoe.so and runs a host-only entry point (no GPU call)."""
import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
REF_INCLUDE = pathlib.Path("/root/reference/include")
CXX = shutil.which("g++")

USE = r"""
#include "xs_strata_kernels.hpp"
#include <cstdio>
// every wrapper of the prompt and layer surface, compiled and linked; main calls it only with a stream, never here
void surface(void* stream) {
    namespace k = strata::kernels;
    namespace m = strata::prefill::mmq;
    const k::NativeExpertLayout L = k::native_expert_layout(12, 14, 2048, 768);
    k::iq_dequant_f16(12, nullptr, 256, nullptr, stream);
    k::iq_mmq_quantize(stream, nullptr, nullptr, nullptr, 256, 256, 1, k::iq_mmq_type_sums(12), k::iq_mmq_type_dup(12));
    k::iq_mmq_quantize_scatter(stream, nullptr, nullptr, nullptr, 256, 256, 1, 8, true);
    m::quantize(nullptr, nullptr, nullptr, 12, 256, 256, 1, stream);
    m::quantize_scatter(nullptr, nullptr, nullptr, nullptr, 12, 256, 256, 1, 8, stream);
    m::swiglu(nullptr, nullptr, 1, 768, false, stream);
    m::iota(nullptr, 16, stream);
    k::iq_mmq_grouped(stream, 12, nullptr, 0, 256, 256, 1, nullptr, 1, nullptr, 1, nullptr, nullptr, 256);
    k::f32_gemv_fp32_mmvf(nullptr, nullptr, nullptr, 2048, 128, stream);
    k::bf16_gemv_fp32_mmvf(nullptr, nullptr, nullptr, 2048, 128, stream);
    k::f32_gemv_fp32_mmvf_multi(nullptr, 2048, nullptr, nullptr, 128, 2048, 128, 4, stream);
    k::bf16_gemv_fp32_mmvf_multi(nullptr, 2048, nullptr, nullptr, 128, 2048, 128, 4, stream);
    k::f32_gemm_rows(nullptr, 2048, nullptr, nullptr, 128, 2048, 128, 64, stream);
    k::bf16_gemv(nullptr, nullptr, nullptr, 2048, 128, stream);
    k::bf16_gemv_split(nullptr, nullptr, nullptr, 2048, 128, 32, stream);
    k::f32_to_bf16_bulk(nullptr, nullptr, 2048, stream);
    m::Product prod;
    m::Context().run(prod, stream);
    k::native_moe_combine_multi_hits(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 2048, 8, 1, stream);
    const size_t ws = k::moe_layer_decode_workspace_bytes(L, 128, 8, 1);
    k::moe_layer_decode(L, nullptr, L.bytes, 128, 8, nullptr, nullptr, nullptr, nullptr, 1, nullptr, ws, stream);
    k::moe_layer_check(nullptr, stream);
    k::moe_layer_prefill(L, nullptr, L.bytes, 128, 8, nullptr, nullptr, nullptr, nullptr, 64, nullptr,
                         k::moe_layer_prefill_workspace_bytes(L, 128, 8, 64), stream);
    std::printf("%zu %d\n", m::q8_bytes(4, 256), (int)k::native_moe_fuse_hits());
}

int main(int argc, char** argv) {
    namespace k = strata::kernels;
    if (argc > 1) surface(argv[1]);
    const k::NativeExpertLayout L = k::native_expert_layout(12, 14, 2048, 768);
    std::printf("%zu %d\n", L.bytes, (int)k::native_expert_supported(12, 14, 2048, 768));
    try {
        k::native_expert_layout(12, 14, 2000, 768);
    } catch (const std::invalid_argument&) {
        std::printf("invalid\n");
    }
    try {
        throw strata::core::DeviceError("device");
    } catch (const std::runtime_error& e) {
        std::printf("%s\n", e.what());
    }
    return 0;
}
"""

ENGINE_DECL = r"""
#include <stdexcept>
namespace strata::core {
class DeviceError : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};
}  // namespace strata::core
#define XS_STRATA_HAVE_DEVICE_ERROR 1
"""

ENGINE_HEADER = r"""
#include "strata/core/device.hpp"
"""

pytestmark = pytest.mark.skipif(CXX is None, reason="g++ is not installed")


def compile_only(tmp_path, prefix, extra=()):
    src = tmp_path / "tu.cpp"
    src.write_text(prefix + USE)
    r = subprocess.run([CXX, "-std=c++17", "-fsyntax-only", "-Wall", "-Werror", "-I", str(ROOT / "include"), *extra,
                        str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_header_stand_alone(tmp_path):
    compile_only(tmp_path, "")


def test_header_after_engine_declaration(tmp_path):
    compile_only(tmp_path, ENGINE_DECL)


def test_header_beside_engine_device_hpp(tmp_path):
    if not (REF_INCLUDE / "strata" / "core" / "device.hpp").exists():
        pytest.skip("the reference tree is not present here")
    compile_only(tmp_path, ENGINE_HEADER, ["-std=c++20", "-I", str(REF_INCLUDE)])
    compile_only(tmp_path, "", ["-std=c++20", "-I", str(REF_INCLUDE)])   # device.hpp found by __has_include


def test_links_and_runs_host_entry_points(tmp_path):
    lib = ROOT / "xestrata-win_amd" / "libxsmoe.so"
    if not lib.exists():
        pytest.skip("libxsmoe.so is not built")
    src = tmp_path / "prog.cpp"
    src.write_text(USE)
    exe = tmp_path / "prog"
    r = subprocess.run([CXX, "-std=c++17", "-I", str(ROOT / "include"), str(src), "-o", str(exe), str(lib),
                        f"-Wl,-rpath,{lib.parent}"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    assert out.stdout.split() == ["3059712", "1", "invalid", "device"]
