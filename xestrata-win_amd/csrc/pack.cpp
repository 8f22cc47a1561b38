// xestrata-win_amd/csrc/pack.cpp - the expert arena of a native pack (include/xs_pack.h): the layout table from
// native_experts.txt or from a GGUF model's expert tensors, its check against the model's shards, and the arena
// filled in HBM from those shards in place.
//
// Host code.  The GGUF reader parses the header and tensor directory only (GGUF v3: magic, version, tensor and
// key counts, typed key/values, then name / n_dims / dims / type / offset per tensor; the data section starts at the
// next multiple of general.alignment, 32 by default).  Loading streams each tensor through pinned host buffers: a
// worker reads a chunk of whole experts with pread, then one hipMemcpy2DAsync lays the chunk's slices into their
// blobs (source pitch the slice, destination pitch the blob), while the worker reads the next chunk into its other
// buffer.  The copy engine does the scatter; no kernel touches the bytes.
#include "../../include/xs_pack.h"
#include "../../include/xs_moe.h"
#include "xs_error.h"

#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cctype>
#include <charconv>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <sstream>
#include <string>
#include <string_view>
#include <thread>
#include <vector>

struct xs_pack {
    struct Layer {
        int gu = 0, d = 0, up = 0;
        int64_t block = 0;
        uint64_t offset = ~0ull, bytes = 0, up_off = 0, down_off = 0;
    };
    int version = 0;
    int64_t n_layers = 0, n_expert = 0, n_embd = 0, n_ff = 0;
    uint64_t max_blob = 0, total = 0;
    std::vector<Layer> layer;
    std::vector<uint64_t> gguf_off;       // 3 per layer (gate, up, down), or empty: no offsets in the table
    std::vector<std::string> gguf_file;   // 3 per layer, "" = the native shard; or empty

    uint64_t per(int64_t l, int r) const {   // bytes of one expert's slice of role r
        const Layer& L = layer[(size_t)l];
        return r == 0 ? L.up_off : r == 1 ? L.down_off - L.up_off : L.bytes - L.down_off;
    }
    uint64_t at(int64_t l, int r) const {    // the slice's offset inside the blob
        const Layer& L = layer[(size_t)l];
        return r == 0 ? 0 : r == 1 ? L.up_off : L.down_off;
    }
};

namespace {

const char* const kRole[3] = {"gate", "up", "down"};

// ggml type ids with a block geometry: values and bytes per block, and the name; 42 is Strata's Q2_0 (64 values in
// 18 bytes).  The set the reference's GGUF reader knows (gguf_reader.hpp:124-260): a tensor of another type has no
// payload size there, so a table naming one is refused here too.
struct TypeInfo {
    int id, qk, bytes;
    const char* name;
};
constexpr TypeInfo kTypes[] = {
    {0, 1, 4, "F32"},         {1, 1, 2, "F16"},         {2, 32, 18, "Q4_0"},      {3, 32, 20, "Q4_1"},
    {6, 32, 22, "Q5_0"},      {7, 32, 24, "Q5_1"},      {8, 32, 34, "Q8_0"},      {9, 32, 36, "Q8_1"},
    {10, 256, 84, "Q2_K"},    {11, 256, 110, "Q3_K"},   {12, 256, 144, "Q4_K"},   {13, 256, 176, "Q5_K"},
    {14, 256, 210, "Q6_K"},   {16, 256, 66, "IQ2_XXS"}, {17, 256, 74, "IQ2_XS"},  {18, 256, 98, "IQ3_XXS"},
    {20, 32, 18, "IQ4_NL"},   {21, 256, 110, "IQ3_S"},  {22, 256, 82, "IQ2_S"},   {23, 256, 136, "IQ4_XS"},
    {24, 1, 1, "I8"},         {29, 256, 56, "IQ1_M"},   {30, 1, 2, "BF16"},       {42, 64, 18, "Q2_0"},
};

const TypeInfo* type_info(int64_t id) {
    for (const TypeInfo& t : kTypes)
        if (t.id == id) return &t;
    return nullptr;
}

std::string type_name(int64_t id) {
    const TypeInfo* t = type_info(id);
    return t ? t->name : "type " + std::to_string(id);
}

// bytes of a row of n values (0: unknown type, or not whole blocks)
uint64_t row_bytes(int64_t type, int64_t n) {
    const TypeInfo* t = type_info(type);
    if (!t || n <= 0 || n % t->qk) return 0;
    return (uint64_t)(n / t->qk) * (uint64_t)t->bytes;
}

// a tensor's payload bytes from its shape (dim 0 the row); 0 when unknown or not whole blocks
uint64_t payload_bytes(int64_t type, const std::vector<uint64_t>& shape) {
    const TypeInfo* t = type_info(type);
    if (!t || shape.empty() || shape[0] % (uint64_t)t->qk) return 0;
    uint64_t n = 1;
    for (uint64_t d : shape) {
        if (d == 0 || n > ~0ull / d) return 0;
        n *= d;
    }
    const uint64_t blocks = n / (uint64_t)t->qk;
    if (blocks > ~0ull / (uint64_t)t->bytes) return 0;
    return blocks * (uint64_t)t->bytes;
}

// one blob's offsets from the three types: [n_ff gate rows | n_ff up rows | n_embd down rows]
bool blob_format(int gu, int d, int up, int64_t n_embd, int64_t n_ff, xs_pack::Layer& L, std::string& err) {
    const uint64_t gr = row_bytes(gu, n_embd), ur = row_bytes(up, n_embd), dr = row_bytes(d, n_ff);
    if (!gr || !ur || !dr) {
        const int bad = !gr ? gu : !ur ? up : d;
        err = "expert types: " + type_name(bad) + " has no block geometry here or its rows (" +
              std::to_string(bad == d && !dr ? n_ff : n_embd) + " values) are not whole blocks";
        return false;
    }
    L.gu = gu;
    L.d = d;
    L.up = up;
    L.up_off = (uint64_t)n_ff * gr;
    L.down_off = L.up_off + (uint64_t)n_ff * ur;
    L.bytes = L.down_off + (uint64_t)n_embd * dr;
    return true;
}

int fail(int code, const std::string& m) { return xs::set_error(code, m); }

// ---- GGUF: the header and tensor directory
struct GTensor {
    std::vector<uint64_t> shape;
    int64_t type = -1;
    uint64_t offset = 0;
};

struct Gguf {
    std::string path;
    uint64_t size = 0, data_start = 0;
    std::map<std::string, GTensor> tensors;
};

class Reader {
public:
    explicit Reader(FILE* f) : f_(f) {}
    void bytes(void* p, size_t n) {
        if (n && std::fread(p, 1, n, f_) != n) throw std::runtime_error("the header runs past the end of the file");
        pos_ += n;
    }
    template <class T>
    T get() {
        T v;
        bytes(&v, sizeof v);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (n > (1ull << 30)) throw std::runtime_error("a string of " + std::to_string(n) + " bytes in the header");
        std::string s((size_t)n, '\0');
        bytes(&s[0], (size_t)n);
        return s;
    }
    void skip(uint64_t n) {
        if (n == 0) return;
        if (fseeko(f_, (off_t)n, SEEK_CUR) != 0) throw std::runtime_error("the header runs past the end of the file");
        pos_ += n;
    }
    uint64_t pos() const { return pos_; }

private:
    FILE* f_;
    uint64_t pos_ = 0;
};

size_t scalar_size(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;    // u8, i8, bool
        case 2: case 3: return 2;            // u16, i16
        case 4: case 5: case 6: return 4;    // u32, i32, f32
        case 10: case 11: case 12: return 8; // u64, i64, f64
        default: return 0;
    }
}

// a key's value: an unsigned integer when it is one (general.alignment), else skipped
bool read_value(Reader& r, uint32_t t, uint64_t& u) {
    if (t == 8) { (void)r.str(); return false; }
    if (t == 9) {
        const uint32_t et = r.get<uint32_t>();
        const uint64_t n = r.get<uint64_t>();
        if (et == 8) {
            for (uint64_t i = 0; i < n; ++i) (void)r.str();
        } else if (et == 9) {
            throw std::runtime_error("nested metadata arrays");
        } else {
            const size_t es = scalar_size(et);
            if (!es) throw std::runtime_error("metadata array of type " + std::to_string(et));
            r.skip(n * es);
        }
        return false;
    }
    const size_t s = scalar_size(t);
    if (!s) throw std::runtime_error("metadata value of type " + std::to_string(t));
    uint64_t v = 0;
    r.bytes(&v, s);
    u = v;
    return t == 0 || t == 2 || t == 4 || t == 10;
}

bool gguf_open(const std::string& path, Gguf& g, std::string& err) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) {
        err = "cannot open " + path;
        return false;
    }
    std::unique_ptr<FILE, int (*)(FILE*)> hold(f, std::fclose);
    try {
        struct stat st {};
        if (fstat(fileno(f), &st) != 0) throw std::runtime_error("fstat failed");
        g.path = path;
        g.size = (uint64_t)st.st_size;
        Reader r(f);
        if (r.get<uint32_t>() != 0x46554747u) throw std::runtime_error("not a GGUF file (bad magic)");
        const uint32_t version = r.get<uint32_t>();
        if (version != 3) throw std::runtime_error("GGUF v" + std::to_string(version) + ", this reader handles v3");
        const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
        uint64_t align = 32;
        for (uint64_t i = 0; i < n_kv; ++i) {
            const std::string key = r.str();
            const uint32_t t = r.get<uint32_t>();
            uint64_t u = 0;
            if (read_value(r, t, u) && key == "general.alignment" && u) align = u;
        }
        for (uint64_t i = 0; i < n_tensors; ++i) {
            std::string name = r.str();
            GTensor t;
            const uint32_t nd = r.get<uint32_t>();
            if (nd == 0 || nd > 4) throw std::runtime_error("bad n_dims for " + name);
            t.shape.resize(nd);
            for (uint32_t d = 0; d < nd; ++d) t.shape[d] = r.get<uint64_t>();
            t.type = r.get<uint32_t>();
            t.offset = r.get<uint64_t>();
            if (!g.tensors.emplace(name, std::move(t)).second)
                throw std::runtime_error("duplicate tensor name '" + name + "'");
        }
        g.data_start = (r.pos() + align - 1) / align * align;
        if (g.data_start > g.size) {
            // a metadata-only shard may end inside the alignment padding: nothing is read there
            if (n_tensors) throw std::runtime_error("the data section starts past the end of the file");
            g.data_start = g.size;
        }
        return true;
    } catch (const std::exception& e) {
        err = "GGUF " + path + ": " + e.what();
        return false;
    }
}

// the shards of the model `any` belongs to: <stem>-NNNNN-of-MMMMM.gguf, 1..M in order; else `any` alone
bool split_paths(const std::string& any, std::vector<std::string>& out, std::string& err) {
    out.clear();
    const size_t at = any.rfind("-of-");
    bool split = at != std::string::npos && at >= 6 && any[at - 6] == '-' && any.size() == at + 4 + 5 + 5 &&
                 any.compare(at + 9, 5, ".gguf") == 0;
    int no = 0, n = 0;
    for (size_t i = 0; split && i < 5; ++i) {
        const char a = any[at - 5 + i], b = any[at + 4 + i];
        if (a < '0' || a > '9' || b < '0' || b > '9') split = false;
        no = no * 10 + (a - '0');
        n = n * 10 + (b - '0');
    }
    if (!split || n < 1 || no < 1 || no > n) {
        out.push_back(any);
        return true;
    }
    for (int i = 1; i <= n; ++i) {
        char num[8];
        std::snprintf(num, sizeof num, "%05d", i);
        std::string p = any;
        p.replace(at - 5, 5, num);
        if (access(p.c_str(), R_OK) != 0) {
            err = "missing model shard " + p + " (shard " + std::to_string(i) + " of " + std::to_string(n) + ")";
            return false;
        }
        out.push_back(std::move(p));
    }
    return true;
}

std::string dir_of(const std::string& path) {
    const size_t cut = path.find_last_of('/');
    return cut == std::string::npos ? std::string() : path.substr(0, cut + 1);
}

std::string base_of(const std::string& path) {
    const size_t cut = path.find_last_of('/');
    return cut == std::string::npos ? path : path.substr(cut + 1);
}

// the file that holds role r of layer l: a name beside the native shard, or the native shard itself
std::string file_of(const xs_pack& P, const std::string& native, int64_t l, int r) {
    const size_t i = (size_t)(3 * l + r);
    if (P.gguf_file.size() <= i || P.gguf_file[i].empty()) return native;
    return dir_of(native) + P.gguf_file[i];
}

std::string tensor_name(int64_t block, int r) {
    return "blk." + std::to_string(block) + ".ffn_" + kRole[r] + "_exps.weight";
}

std::string dims(uint64_t a, uint64_t b, uint64_t c) {
    return "[" + std::to_string(a) + ", " + std::to_string(b) + ", " + std::to_string(c) + "]";
}

bool check(const xs_pack& P, const std::string& native, std::string& err) {
    if (P.gguf_off.size() != (size_t)(3 * P.n_layers)) {
        err = "native_experts.txt has no GGUF offsets (a pack older than v2): repack it with iq_pack.py";
        return false;
    }
    std::map<std::string, Gguf> files;
    for (int64_t l = 0; l < P.n_layers; ++l) {
        const xs_pack::Layer& L = P.layer[(size_t)l];
        for (int r = 0; r < 3; ++r) {
            const std::string path = file_of(P, native, l, r);
            auto it = files.find(path);
            if (it == files.end()) {
                Gguf g;
                std::string e;
                if (!gguf_open(path, g, e)) {
                    err = "native experts from the GGUF: " + e;
                    return false;
                }
                it = files.emplace(path, std::move(g)).first;
            }
            const Gguf& g = it->second;
            const std::string name = tensor_name(L.block, r);
            const auto t = g.tensors.find(name);
            const int64_t want_type = r == 0 ? L.gu : r == 1 ? L.up : L.d;
            const uint64_t cols = (uint64_t)(r < 2 ? P.n_embd : P.n_ff), rows = (uint64_t)(r < 2 ? P.n_ff : P.n_embd);
            const uint64_t bytes = P.per(l, r) * (uint64_t)P.n_expert;
            const uint64_t payload = g.size - g.data_start;
            std::string why;
            if (t == g.tensors.end())
                why = "is not in it";
            else if (t->second.type != want_type)
                why = "is " + type_name(t->second.type) + ", the pack says type " + std::to_string(want_type);
            else if (t->second.shape.size() != 3 || t->second.shape[0] != cols || t->second.shape[1] != rows ||
                     t->second.shape[2] != (uint64_t)P.n_expert)
                why = "is not " + dims(cols, rows, (uint64_t)P.n_expert);
            else if (payload_bytes(t->second.type, t->second.shape) != bytes)
                why = "is not " + std::to_string(P.per(l, r)) + " B per expert";
            else if (g.data_start + t->second.offset != P.gguf_off[(size_t)(3 * l + r)])
                why = "starts at byte " + std::to_string(g.data_start + t->second.offset) + ", the pack says " +
                      std::to_string(P.gguf_off[(size_t)(3 * l + r)]);
            else if (t->second.offset > payload || bytes > payload - t->second.offset)
                why = "runs past the end of the file (a truncated shard?)";
            if (!why.empty()) {
                err = "the pack's native_experts.txt does not match the model: " + name + " in " + path + " " + why +
                      " - repack with iq_pack.py from this model's shards";
                return false;
            }
        }
    }
    return true;
}

// ---- loading: workers over (layer, role) tensors, chunks of whole experts through two pinned buffers each
struct Loader {
    const xs_pack& P;
    std::string native;
    uint8_t* const* dst;
    size_t chunk_cap;
    std::atomic<int64_t> next{0};
    std::atomic<bool> bad{false};
    std::mutex mu;
    std::string err;

    void set_bad(const std::string& m) {
        std::lock_guard<std::mutex> g(mu);
        if (!bad.exchange(true)) err = m;
    }

    void worker() {
        hipStream_t s = nullptr;
        uint8_t* buf[2] = {nullptr, nullptr};
        hipEvent_t ev[2] = {nullptr, nullptr};
        bool pending[2] = {false, false};
        std::map<std::string, int> fds;
        auto hip_ok = [&](hipError_t e, const char* what) {
            if (e == hipSuccess) return true;
            set_bad(std::string(what) + ": " + hipGetErrorString(e));
            return false;
        };
        bool ready = hip_ok(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
        for (int b = 0; ready && b < 2; ++b)
            ready = hip_ok(hipHostMalloc((void**)&buf[b], chunk_cap, hipHostMallocDefault), "hipHostMalloc") &&
                    hip_ok(hipEventCreateWithFlags(&ev[b], hipEventDisableTiming), "hipEventCreateWithFlags");
        int cur = 0;
        while (ready && !bad) {
            const int64_t item = next.fetch_add(1);
            if (item >= 3 * P.n_layers) break;
            const int64_t l = item / 3;
            const int r = (int)(item % 3);
            const std::string path = file_of(P, native, l, r);
            auto it = fds.find(path);
            if (it == fds.end()) {
                const int fd = ::open(path.c_str(), O_RDONLY);
                if (fd < 0) {
                    set_bad("cannot open " + path);
                    break;
                }
                posix_fadvise(fd, 0, 0, POSIX_FADV_SEQUENTIAL);
                it = fds.emplace(path, fd).first;
            }
            const int fd = it->second;
            const uint64_t per = P.per(l, r), blob = P.layer[(size_t)l].bytes, at = P.at(l, r);
            const uint64_t src = P.gguf_off[(size_t)(3 * l + r)];
            const int64_t step = std::max<int64_t>(1, (int64_t)(chunk_cap / per));
            for (int64_t e0 = 0; e0 < P.n_expert && !bad; e0 += step) {
                const int64_t n = std::min<int64_t>(step, P.n_expert - e0);
                if (pending[cur] && !hip_ok(hipEventSynchronize(ev[cur]), "hipEventSynchronize")) break;
                pending[cur] = false;
                const uint64_t want = (uint64_t)n * per;
                uint64_t got = 0;
                while (got < want) {
                    const ssize_t k = ::pread(fd, buf[cur] + got, (size_t)(want - got), (off_t)(src + (uint64_t)e0 * per + got));
                    if (k <= 0) break;
                    got += (uint64_t)k;
                }
                if (got != want) {
                    set_bad("short read or unreadable shard while reading the experts from " + path);
                    break;
                }
                uint8_t* d = dst[l] + (uint64_t)e0 * blob + at;
                if (!hip_ok(hipMemcpy2DAsync(d, blob, buf[cur], per, per, (size_t)n, hipMemcpyDefault, s),
                            "hipMemcpy2DAsync") ||
                    !hip_ok(hipEventRecord(ev[cur], s), "hipEventRecord"))
                    break;
                pending[cur] = true;
                cur ^= 1;
            }
        }
        if (s) hip_ok(hipStreamSynchronize(s), "hipStreamSynchronize");
        for (int b = 0; b < 2; ++b) {
            if (ev[b]) (void)hipEventDestroy(ev[b]);
            if (buf[b]) (void)hipHostFree(buf[b]);
        }
        if (s) (void)hipStreamDestroy(s);
        for (auto& f : fds) ::close(f.second);
    }
};

int load(const xs_pack* P, const char* native_shard, uint8_t* const* layer_dst, int threads,
         xs_pack_load_stats_t* stats) {
    const auto t0 = std::chrono::steady_clock::now();
    std::string err;
    if (!check(*P, native_shard, err)) return fail(XS_EINVAL, err);
    uint64_t max_per = 0;
    for (int64_t l = 0; l < P->n_layers; ++l)
        for (int r = 0; r < 3; ++r) max_per = std::max(max_per, P->per(l, r));
    Loader ld{*P, native_shard, layer_dst, (size_t)std::max<uint64_t>(64ull << 20, max_per)};
    const int n = std::max(1, std::min(threads > 0 ? threads : 4, 32));
    std::vector<std::thread> pool;
    for (int i = 1; i < n; ++i) pool.emplace_back([&ld] { ld.worker(); });
    ld.worker();
    for (auto& t : pool) t.join();
    if (ld.bad) return fail(XS_EDEVICE, "pack load: " + ld.err);
    if (stats) {
        stats->bytes = P->total;
        stats->layers = (uint64_t)P->n_layers;
        stats->seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    }
    return XS_OK;
}

// ---- native_experts.txt
//
// The file is lines of whitespace-separated fields.  A line starting with '#' is a comment; a comment can carry the
// format's version tag (upstream Strata's "# strata native experts vN", N = 2..4, or XeStrata's "# xestrata native
// experts xsN", N = 1, read as 4) and "(n_expert N" (the pack's expert count, which wins over the caller's: a pruned
// model ships fewer).  Every other non-empty line is one MoE layer: layer, gate/up type, down type, arena offset, blob
// bytes, then optionally the three tensors' absolute GGUF offsets (gate, up, down) and a shard column.  The reader
// first turns the text into header facts and rows (read_manifest), then checks the rows against the geometry and
// lays them into the table (xs_pack_layout_load).

struct VersionTag {
    const char* prefix;   // the comment's text up to the number
    const char* label;    // how a refused version is named ("v5", "xs2")
    int newest;           // the newest number this reader takes
    bool upstream;        // the number is the version itself (else it reads as 4)
};
constexpr VersionTag kVersionTags[] = {
    {"# strata native experts v", "v", 4, true},
    {"# xestrata native experts xs", "xs", 1, false},
};

struct ManifestRow {
    std::string text;               // the line, for messages
    int64_t layer = -1;
    int64_t gu = -1, d = -1;
    uint64_t offset = 0, blob = 0;
    bool has_gguf = false;
    uint64_t gguf_off[3] = {0, 0, 0};
    std::vector<std::string> shards;   // the shard column's fields as written (empty: no column)
};

struct Manifest {
    int version = 0;
    int64_t n_expert = 0;           // 0: no header gave it
    std::vector<ManifestRow> rows;
};

std::vector<std::string_view> fields_of(std::string_view line) {
    std::vector<std::string_view> f;
    size_t i = 0;
    while (i < line.size()) {
        while (i < line.size() && std::isspace((unsigned char)line[i])) ++i;
        size_t j = i;
        while (j < line.size() && !std::isspace((unsigned char)line[j])) ++j;
        if (j > i) f.push_back(line.substr(i, j - i));
        i = j;
    }
    return f;
}

template <typename T>
bool number_of(std::string_view s, T& v) {
    const char* end = s.data() + s.size();
    const auto r = std::from_chars(s.data(), end, v);
    return r.ec == std::errc() && r.ptr == end;
}

// a comment line's facts: the version tag (an error for a version past what this reader takes) and n_expert
bool read_comment(std::string_view line, Manifest& m, std::string& err) {
    for (const VersionTag& t : kVersionTags) {
        const std::string_view prefix(t.prefix);
        if (line.substr(0, prefix.size()) != prefix) continue;
        const std::string digits(line.substr(prefix.size()));
        const int n = (int)std::strtol(digits.c_str(), nullptr, 10);
        if (n > t.newest) {
            err = std::string("native_experts.txt is ") + t.label + std::to_string(n) + ", newer than this reader "
                  "knows (it takes upstream Strata's v2-v4 and XeStrata's xs1)";
            return false;
        }
        m.version = t.upstream ? n : 4;
    }
    static constexpr std::string_view kCount = "(n_expert ";
    const size_t at = line.find(kCount);
    if (at != std::string_view::npos) {
        m.n_expert = std::atoll(std::string(line.substr(at + kCount.size())).c_str());
        if (m.n_expert <= 0) {
            err = "native_experts.txt: a header with no experts: " + std::string(line);
            return false;
        }
    }
    return true;
}

// one layer line: five numbers, then either the three GGUF offsets and the shard column or nothing this reader uses
bool read_row(std::string_view line, ManifestRow& r, std::string& err) {
    const std::vector<std::string_view> f = fields_of(line);
    r.text = std::string(line);
    if (f.size() < 5 || !number_of(f[0], r.layer) || !number_of(f[1], r.gu) || !number_of(f[2], r.d) ||
        !number_of(f[3], r.offset) || !number_of(f[4], r.blob)) {
        err = "native_experts.txt: a malformed line: " + r.text;
        return false;
    }
    r.has_gguf = f.size() >= 8 && number_of(f[5], r.gguf_off[0]) && number_of(f[6], r.gguf_off[1]) &&
                 number_of(f[7], r.gguf_off[2]);
    if (r.has_gguf)
        for (size_t i = 8; i < f.size(); ++i) r.shards.emplace_back(f[i]);
    return true;
}

bool read_manifest(std::istream& in, Manifest& m, std::string& err) {
    for (std::string line; std::getline(in, line);) {
        std::string_view v(line);
        if (!v.empty() && v.back() == '\r') v.remove_suffix(1);
        if (v.empty()) continue;
        if (v.front() == '#') {
            if (!read_comment(v, m, err)) return false;
            continue;
        }
        m.rows.emplace_back();
        if (!read_row(v, m.rows.back(), err)) return false;
    }
    return true;
}

// The shard column as three file names (gate, up, down; "" = the native shard).  Written as one name for all three
// roles, as "gate,up,down" in one field (an empty field: the native shard), or as three fields ("-": the native
// shard).  No column: no names.
bool shard_names(const ManifestRow& r, std::vector<std::string>& names, std::string& err) {
    names.clear();
    if (r.shards.empty()) return true;
    std::vector<std::string> parts = r.shards;
    if (parts.size() == 1 && parts[0].find(',') != std::string::npos) {
        std::vector<std::string> split(1);
        for (const char c : parts[0]) {
            if (c == ',') split.emplace_back();
            else split.back() += c;
        }
        parts = std::move(split);
    }
    if (parts.size() == 1) parts = {parts[0], parts[0], parts[0]};
    if (parts.size() != 3) {
        err = "native_experts.txt: layer " + std::to_string(r.layer) + ": the shard column must be one name, "
              "gate,up,down or three names, not: " + r.text;
        return false;
    }
    for (std::string& s : parts)
        if (s == "-") s.clear();
    names = std::move(parts);
    return true;
}

}  // namespace

extern "C" {

int xs_pack_layout_load(const char* pack_dir, int64_t n_layers, int64_t n_expert, int64_t n_embd, int64_t n_ff,
                        xs_pack_t** out) {
    if (!out) return fail(XS_EINVAL, "pack layout: no output");
    *out = nullptr;
    if (!pack_dir || n_layers <= 0 || n_expert <= 0 || n_embd <= 0 || n_ff <= 0)
        return fail(XS_EINVAL, "pack layout: the geometry is empty");
    const std::string path = std::string(pack_dir) + "/native_experts.txt";
    std::ifstream in(path);
    if (!in)
        return fail(XS_EINVAL, "pack layout: " + path + " is missing: not a native pack (the Strata Q2_0 expert form "
                               "is not a format these kernels read)");
    Manifest m;
    std::string err;
    if (!read_manifest(in, m, err)) return fail(XS_EINVAL, err);

    auto P = std::make_unique<xs_pack>();
    P->version = m.version;
    P->n_layers = n_layers;
    P->n_expert = m.n_expert > 0 ? m.n_expert : n_expert;
    P->n_embd = n_embd;
    P->n_ff = n_ff;
    P->layer.assign((size_t)n_layers, xs_pack::Layer{});
    std::vector<char> seen((size_t)n_layers, 0);
    for (const ManifestRow& r : m.rows) {
        if (r.layer < 0 || r.layer >= n_layers)
            return fail(XS_EINVAL, "native_experts.txt: a malformed line (layer out of range): " + r.text);
        const std::string which = "native_experts.txt: layer " + std::to_string(r.layer);
        if (seen[(size_t)r.layer]++) return fail(XS_EINVAL, which + " is listed twice");
        xs_pack::Layer& L = P->layer[(size_t)r.layer];
        if (!blob_format((int)r.gu, (int)r.d, (int)r.gu, n_embd, n_ff, L, err))
            return fail(XS_EINVAL, which + ": " + err);
        if (L.bytes != r.blob)
            return fail(XS_EINVAL, which + " says " + std::to_string(r.blob) + " B a blob, but its formats make " +
                                       std::to_string(L.bytes));
        std::vector<std::string> names;
        if (!shard_names(r, names, err)) return fail(XS_EINVAL, err);
        if (r.has_gguf) {
            if (P->gguf_off.empty()) P->gguf_off.assign((size_t)(3 * n_layers), 0);
            std::copy(r.gguf_off, r.gguf_off + 3, P->gguf_off.begin() + 3 * r.layer);
        }
        if (!names.empty()) {
            if (P->gguf_file.empty()) P->gguf_file.assign((size_t)(3 * n_layers), std::string());
            std::copy(names.begin(), names.end(), P->gguf_file.begin() + 3 * r.layer);
        }
        L.block = r.layer;
        L.offset = r.offset;
        P->max_blob = std::max<uint64_t>(P->max_blob, r.blob);
    }
    // the layers tile the arena from offset 0 in order, each n_expert blobs long
    uint64_t next = 0;
    for (int64_t l = 0; l < n_layers; ++l) {
        const xs_pack::Layer& L = P->layer[(size_t)l];
        if (!seen[(size_t)l] || L.offset != next)
            return fail(XS_EINVAL, "native_experts.txt: layer " + std::to_string(l) + " is missing or not contiguous "
                                   "(expected at arena offset " + std::to_string(next) + ")");
        next += L.bytes * (uint64_t)P->n_expert;
    }
    P->total = next;
    *out = P.release();
    return XS_OK;
}

int xs_pack_layout_from_gguf(const char* gguf, const int64_t* moe_blocks, int64_t n_layers, int64_t n_expert,
                             int64_t n_embd, int64_t n_ff, xs_pack_t** out) {
    if (!out) return fail(XS_EINVAL, "experts from the GGUF: no output");
    *out = nullptr;
    if (!gguf || !moe_blocks || n_layers <= 0 || n_expert <= 0 || n_embd <= 0 || n_ff <= 0)
        return fail(XS_EINVAL, "experts from the GGUF: the geometry is empty");
    std::string err;
    std::vector<std::string> paths;
    if (!split_paths(gguf, paths, err)) return fail(XS_EINVAL, "experts from the GGUF: " + err);
    std::vector<Gguf> shards(paths.size());
    std::map<std::string, size_t> where;   // tensor name -> shard
    for (size_t i = 0; i < paths.size(); ++i) {
        if (!gguf_open(paths[i], shards[i], err)) return fail(XS_EINVAL, "experts from the GGUF: " + err);
        for (const auto& t : shards[i].tensors) {
            const auto ins = where.emplace(t.first, i);
            if (!ins.second)
                return fail(XS_EINVAL, "experts from the GGUF: tensor " + t.first + " is in two shards (" +
                                           paths[ins.first->second] + " and " + paths[i] + ")");
        }
    }
    auto P = std::make_unique<xs_pack>();
    P->version = 0;
    P->n_layers = n_layers;
    P->n_expert = n_expert;
    P->n_embd = n_embd;
    P->n_ff = n_ff;
    P->layer.assign((size_t)n_layers, xs_pack::Layer{});
    P->gguf_off.assign((size_t)(3 * n_layers), 0);
    P->gguf_file.assign((size_t)(3 * n_layers), std::string());
    uint64_t at = 0;
    for (int64_t l = 0; l < n_layers; ++l) {
        const GTensor* t[3] = {};
        size_t sh[3] = {};
        for (int r = 0; r < 3; ++r) {
            const std::string name = tensor_name(moe_blocks[l], r);
            const uint64_t cols = (uint64_t)(r < 2 ? n_embd : n_ff), rows = (uint64_t)(r < 2 ? n_ff : n_embd);
            const auto w = where.find(name);
            if (w != where.end()) {
                sh[r] = w->second;
                t[r] = &shards[sh[r]].tensors.at(name);
            }
            if (!t[r] || t[r]->shape.size() != 3 || t[r]->shape[0] != cols || t[r]->shape[1] != rows ||
                t[r]->shape[2] != (uint64_t)n_expert)
                return fail(XS_EINVAL, "experts from the GGUF: " + name + " is missing or not " +
                                           dims(cols, rows, (uint64_t)n_expert));
            const Gguf& g = shards[sh[r]];
            const uint64_t pb = payload_bytes(t[r]->type, t[r]->shape);
            if (t[r]->offset > g.size - g.data_start || pb > g.size - g.data_start - t[r]->offset)
                return fail(XS_EINVAL, "experts from the GGUF: " + name +
                                           " runs past the end of its file (a truncated shard?)");
        }
        xs_pack::Layer& L = P->layer[(size_t)l];
        if (!blob_format((int)t[0]->type, (int)t[2]->type, (int)t[1]->type, n_embd, n_ff, L, err))
            return fail(XS_EINVAL, "experts from the GGUF: block " + std::to_string(moe_blocks[l]) + ": " + err);
        for (int r = 0; r < 3; ++r) {
            if (payload_bytes(t[r]->type, t[r]->shape) != P->per(l, r) * (uint64_t)n_expert)
                return fail(XS_EINVAL, "experts from the GGUF: block " + std::to_string(moe_blocks[l]) + "'s " +
                                           kRole[r] + " tensor is not " + std::to_string(P->per(l, r)) +
                                           " B per expert");
            P->gguf_off[(size_t)(3 * l + r)] = shards[sh[r]].data_start + t[r]->offset;
            P->gguf_file[(size_t)(3 * l + r)] = base_of(shards[sh[r]].path);
        }
        L.block = moe_blocks[l];
        L.offset = at;
        P->max_blob = std::max<uint64_t>(P->max_blob, L.bytes);
        at += L.bytes * (uint64_t)n_expert;
    }
    P->total = at;
    *out = P.release();
    return XS_OK;
}

void xs_pack_free(xs_pack_t* pack) { delete pack; }

int xs_pack_info(const xs_pack_t* P, xs_pack_info_t* out) {
    if (!P || !out) return fail(XS_EINVAL, "pack info: no pack or no output");
    out->version = P->version;
    out->has_gguf_off = P->gguf_off.size() == (size_t)(3 * P->n_layers);
    out->n_layers = P->n_layers;
    out->n_expert = P->n_expert;
    out->max_blob = P->max_blob;
    out->total = P->total;
    return XS_OK;
}

int xs_pack_layer(const xs_pack_t* P, int64_t l, xs_pack_layer_t* out) {
    if (!P || !out) return fail(XS_EINVAL, "pack layer: no pack or no output");
    if (l < 0 || l >= P->n_layers)
        return fail(XS_EINVAL, "pack layer: layer " + std::to_string(l) + " of " + std::to_string(P->n_layers));
    const xs_pack::Layer& L = P->layer[(size_t)l];
    out->gu_type = L.gu;
    out->d_type = L.d;
    out->up_type = L.up;
    out->block = L.block;
    out->offset = L.offset;
    out->bytes = L.bytes;
    out->up_off = L.up_off;
    out->down_off = L.down_off;
    for (int r = 0; r < 3; ++r) {
        const size_t i = (size_t)(3 * l + r);
        out->gguf_off[r] = i < P->gguf_off.size() ? P->gguf_off[i] : 0;
        out->gguf_file[r] = i < P->gguf_file.size() ? P->gguf_file[i].c_str() : "";
    }
    return XS_OK;
}

uint64_t xs_pack_blob_offset(const xs_pack_t* P, int64_t l, int64_t e) {
    if (!P || l < 0 || l >= P->n_layers || e < 0 || e >= P->n_expert) return ~0ull;
    return P->layer[(size_t)l].offset + (uint64_t)e * P->layer[(size_t)l].bytes;
}

int xs_pack_check_gguf(const xs_pack_t* P, const char* native_shard) {
    if (!P || !native_shard) return fail(XS_EINVAL, "pack check: no pack or no shard");
    std::string err;
    return check(*P, native_shard, err) ? XS_OK : fail(XS_EINVAL, err);
}

int xs_pack_load_gguf(const xs_pack_t* P, const char* native_shard, void* arena, uint64_t arena_bytes, int threads,
                      xs_pack_load_stats_t* stats) {
    if (!P || !native_shard || !arena) return fail(XS_EINVAL, "pack load: no pack, shard or arena");
    if (arena_bytes < P->total)
        return fail(XS_EINVAL, "pack load: the arena is " + std::to_string(arena_bytes) + " B, the pack needs " +
                                   std::to_string(P->total));
    std::vector<uint8_t*> dst((size_t)P->n_layers);
    for (int64_t l = 0; l < P->n_layers; ++l) dst[(size_t)l] = (uint8_t*)arena + P->layer[(size_t)l].offset;
    return load(P, native_shard, dst.data(), threads, stats);
}

int xs_pack_load_gguf_layers(const xs_pack_t* P, const char* native_shard, void* const* layer_dst, int threads,
                             xs_pack_load_stats_t* stats) {
    if (!P || !native_shard || !layer_dst) return fail(XS_EINVAL, "pack load: no pack, shard or destinations");
    for (int64_t l = 0; l < P->n_layers; ++l)
        if (!layer_dst[l]) return fail(XS_EINVAL, "pack load: layer " + std::to_string(l) + " has no destination");
    return load(P, native_shard, (uint8_t* const*)layer_dst, threads, stats);
}

}  // extern "C"
