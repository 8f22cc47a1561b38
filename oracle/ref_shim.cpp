// oracle/ref_shim.cpp - C entry points over the reference's own header-only host code, compiled (by oracle/Makefile,
// into oracle/_ref/) from include/strata/artifact/dequant.hpp, include/strata/kernels/canon_math.hpp,
// include/strata/kernels/bf16_bits.hpp and include/strata/artifact/gguf_reader.hpp where they lie in the reference tree.  TEST INFRASTRUCTURE: it validates
// oracle/xs_oracle.c's restatement and writes tests/golden's vectors; it is never part of the product.
#include "strata/artifact/dequant.hpp"
#include "strata/kernels/canon_math.hpp"
#include "strata/kernels/bf16_bits.hpp"

#include <cmath>
#include <cstdint>

extern "C" {

float xsref_fp16_to_fp32(uint16_t h) { return strata::fp16_to_fp32(h); }

// type ids are ggml's: Q8_0 8, Q4_K 12, Q6_K 14, IQ4_XS 23
int xsref_dequant(int type, const uint8_t* src, int64_t n_blocks, float* dst) {
    for (int64_t i = 0; i < n_blocks; ++i) {
        switch (type) {
            case 8: strata::dequantize_q8_0(src + 34 * i, dst + 32 * i); break;
            case 12: strata::dequantize_q4_K(src + 144 * i, dst + 256 * i); break;
            case 14: strata::dequantize_q6_K(src + 210 * i, dst + 256 * i); break;
            case 23: strata::dequantize_iq4_xs(src + 136 * i, dst + 256 * i); break;
            default: return -1;
        }
    }
    return 0;
}

void xsref_canon_exp(const float* x, int64_t n, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = strata::kernels::canon::exp(x[i]);
}
void xsref_canon_rcp(const float* x, int64_t n, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = strata::kernels::canon::rcp(x[i]);
}
void xsref_canon_silu_mul(const float* g, const float* u, int64_t n, float* h) {
    for (int64_t i = 0; i < n; ++i) h[i] = strata::kernels::canon::silu_mul(g[i], u[i]);
}
void xsref_bf16_from_f32(const float* x, int64_t n, uint16_t* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = strata::kernels::bf16_from_f32(x[i]);
}
void xsref_canon_q8(const float* x, int64_t n, float* d, float* id, int8_t* q) {
    // n values as one block: the scale of their largest magnitude (fmax of fabs, as the kernels reduce it: a
    // negative zero counts as +0), its inverse, and each value's int8
    float amax = 0.0f;
    for (int64_t i = 0; i < n; ++i) amax = std::fmax(amax, std::fabs(x[i]));
    *d = strata::kernels::canon::q8_scale(amax);
    *id = strata::kernels::canon::q8_inv(*d);
    for (int64_t i = 0; i < n; ++i) q[i] = strata::kernels::canon::q8_value(x[i], *id);
}

}  // extern "C"

// ---- the reference's GGUF reader (include/strata/artifact/gguf_reader.hpp, gguf_split.hpp), for the pack loader's
// checks: block geometry, type names, a file's tensor directory, payload bytes and the shard names of a split model
#include "strata/artifact/gguf_reader.hpp"

#include <cstring>
#include <string>

extern "C" {

int xsref_block_geometry(uint32_t t, int* elems, int* bytes) { return strata::block_geometry(t, *elems, *bytes) ? 1 : 0; }

const char* xsref_type_name(uint32_t t) { return strata::ggml_type_name(t); }

// the tensor count of `path` (data start and file size through the pointers), or -1 with the reader's message
int64_t xsref_gguf_dir(const char* path, uint64_t* data_start, uint64_t* size, char* err, size_t errn) {
    try {
        strata::GgufFile f(path);
        *data_start = f.data_start();
        *size = f.file_size();
        return (int64_t)f.tensors().size();
    } catch (const std::exception& e) {
        std::snprintf(err, errn, "%s", e.what());
        return -1;
    }
}

// tensor i of `path` in directory order: name, type, dims, offset from the data start
int xsref_gguf_tensor(const char* path, int64_t i, char* name, size_t nn, uint32_t* type, uint32_t* nd,
                      uint64_t* shape, uint64_t* offset) {
    try {
        strata::GgufFile f(path);
        if (i < 0 || (size_t)i >= f.tensors().size()) return -1;
        const strata::TensorInfo& t = f.tensors()[(size_t)i];
        std::snprintf(name, nn, "%s", t.name.c_str());
        *type = t.type;
        *nd = (uint32_t)t.shape.size();
        for (size_t d = 0; d < t.shape.size() && d < 4; ++d) shape[d] = t.shape[d];
        *offset = t.offset;
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

uint64_t xsref_payload_bytes(uint32_t type, const uint64_t* shape, uint32_t nd) {
    strata::TensorInfo t;
    t.type = type;
    t.shape.assign(shape, shape + nd);
    return strata::tensor_payload_bytes(t);
}

// the model's shard paths for any one of them, newline-separated into out; -1 with the message when one is missing
int xsref_split_paths(const char* any, char* out, size_t n) {
    try {
        std::string s;
        for (const auto& p : strata::gguf_split_paths(any)) s += p + "\n";
        std::snprintf(out, n, "%s", s.c_str());
        return 0;
    } catch (const std::exception& e) {
        std::snprintf(out, n, "%s", e.what());
        return -1;
    }
}

}  // extern "C"
