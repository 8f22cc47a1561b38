// oracle/cpu_path.cpp - the reference's CPU/host MoE decode path restated for x86-64 AVX2, to time it on the GPU box's
// own host cores beside the GPU (bench.py's cpu_baseline).  TEST/BENCH INFRASTRUCTURE: never linked into the product.
//
// What the reference's CPU expert path does (src/kernels/cpu/native_expert.cpp:129-311 and the multi-token AVX2 rows
// of src/kernels/cpu/iq_avx2_rows.inl:220-327, 680-750), restated here in code of this repository's own:
//   - activations: for K-quant weights ggml's Q8_K (include/strata/kernels/quantize_act.hpp:37-55: a float scale a
//     256 values, d = 1 / (-127 / max) with max the signed value of the largest magnitude, codes nearest-even and
//     clamped to 127, sixteen 16-value sums); for Q8_0 weights Q8_0 as src/kernels/cpu/expert.cpp:79-110 (d =
//     amax / 127 kept as fp16, codes round-to-nearest-even of x * 127 / amax);
//   - gate/up rows with the weights unpacked once a block for every token of the expert (the reference's
//     multi-token kernels, from one token on), SwiGLU g / (1 + exp(-g)) * u (native_expert.cpp:277), h quantized
//     again for the down rows, down rows;
//   - Q8_0 rows as ggml's single-token dot (the reference takes ggml-cpu's vec_dot for Q8_0, kq_mt_min);
//   - the routed outputs weighted and summed in rank order, then the residual (plain_model.cpp:985-987).
// The integer parts of every block product are exact; the float accumulation (a scalar sum over blocks) is this
// file's and not ggml's 8-lane order - ggml is absent from this image, so those last bits are parity-unpinned; the
// bench reports the output's distance to the GPU's.
//
// Threads: the reference's pool pins one worker a physical core, every core but the first, and the host thread
// drains too (include/strata/kernels/cpu/pool.hpp:96-121): here OpenMP threads, each pinned once to its own physical
// core (the host thread to the first), the expert rows of a phase split into tasks taken dynamically.
// Timing: the best of 5 means of 10 (src/kernels/iq_mmq_parity.cpp:150-163), expert sets rotated so the weights
// come from DRAM.
#include <immintrin.h>
#include <omp.h>
#include <sched.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <set>
#include <utility>
#include <vector>

extern "C" void xso_router_top10(const float* logits, int n_tokens, int n_expert, int k, int32_t* ids, float* weights);

namespace {

constexpr int kQ8_0 = 8, kQ4_K = 12, kQ6_K = 14;
constexpr int kMaxTok = 8;

float h2f(const uint8_t* p) {
    uint16_t h;
    std::memcpy(&h, p, 2);
    return _cvtsh_ss(h);
}

// ---------------------------------------------------------------- activations
struct Q8K {   // ggml's block_q8_K
    float d;
    int8_t qs[256];
    int16_t bsums[16];
};
static_assert(sizeof(Q8K) == 292, "block_q8_K is 292 bytes");
struct Q80 {   // ggml's block_q8_0 (the fp16 scale widened here: the value is the fp16's)
    float d;
    int8_t qs[32];
};

int nearest_even(float f) {   // half to even through the 1.5 * 2^23 magic (|f| < 2^22)
    const float v = f + 12582912.0f;
    int32_t i;
    std::memcpy(&i, &v, 4);
    return (i & 0x007fffff) - 0x00400000;
}

void quantize_q8_k(const float* x, int64_t n, Q8K* y) {
    for (int64_t b = 0; b < n / 256; ++b) {
        const float* v = x + 256 * b;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 256; ++j) {
            const float a = std::fabs(v[j]);
            if (a > amax) {
                amax = a;
                max = v[j];
            }
        }
        Q8K& o = y[b];
        if (amax == 0.0f) {
            std::memset(&o, 0, sizeof o);
            continue;
        }
        const float iscale = -127.0f / max;
        for (int j = 0; j < 256; ++j) {
            const float p = iscale * v[j];
            o.qs[j] = (int8_t)std::min(127, nearest_even(p));
        }
        for (int j = 0; j < 16; ++j) {
            int s = 0;
            for (int i = 0; i < 16; ++i) s += o.qs[16 * j + i];
            o.bsums[j] = (int16_t)s;
        }
        o.d = 1.0f / iscale;
    }
}

void quantize_q8_0(const float* x, int64_t n, Q80* y) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* v = x + 32 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(v[j]));
        const float d = amax / 127.0f;
        const float inv = amax != 0.0f ? 127.0f / amax : 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float p = v[j] * inv;
            y[b].qs[j] = (int8_t)std::max(-128, std::min(127, (int)std::nearbyint(p)));   // nearest even
        }
        y[b].d = _cvtsh_ss(_cvtss_sh(d, 0));   // kept as fp16, nearest even
    }
}

// ---------------------------------------------------------------- AVX2 helpers
inline int hsum_i32(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
    return _mm_cvtsi128_si32(s);
}
// u8 x s8 products, pairs summed to s16, then times a per-16-bit-lane s16 factor and pairs summed to s32
inline __m256i dot_u8s8(__m256i u, __m256i s, __m256i factor) {
    return _mm256_madd_epi16(_mm256_maddubs_epi16(u, s), factor);
}

// ---------------------------------------------------------------- row dots, NT tokens, weights unpacked once a block
// Q4_K: value = d sc q - dmin m (q a nibble, sc / m six bits a 32 values): a block's integer sums then the two scales
template <int NT>
void row_q4_k(const uint8_t* row, int nb, const Q8K* const* y, float* res) {
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    float acc[NT] = {};
    for (int i = 0; i < nb; ++i) {
        const uint8_t* b = row + 144 * i;
        const uint8_t* s = b + 4;
        int sc[8], mn[8];
        for (int j = 0; j < 4; ++j) {
            sc[j] = s[j] & 63;
            mn[j] = s[j + 4] & 63;
            sc[j + 4] = (s[j + 8] & 0x0F) | ((s[j] >> 6) << 4);
            mn[j + 4] = (s[j + 8] >> 4) | ((s[j + 4] >> 6) << 4);
        }
        __m256i iq[NT];
        for (int t = 0; t < NT; ++t) iq[t] = _mm256_setzero_si256();
        for (int j = 0; j < 4; ++j) {   // 64 values: low nibbles sub-block 2j, high nibbles 2j + 1
            const __m256i q = _mm256_loadu_si256((const __m256i*)(b + 16 + 32 * j));
            const __m256i lo = _mm256_and_si256(q, m4), hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
            const __m256i f0 = _mm256_set1_epi16((int16_t)sc[2 * j]), f1 = _mm256_set1_epi16((int16_t)sc[2 * j + 1]);
            for (int t = 0; t < NT; ++t) {
                const __m256i y0 = _mm256_loadu_si256((const __m256i*)(y[t][i].qs + 64 * j));
                const __m256i y1 = _mm256_loadu_si256((const __m256i*)(y[t][i].qs + 64 * j + 32));
                iq[t] = _mm256_add_epi32(iq[t], _mm256_add_epi32(dot_u8s8(lo, y0, f0), dot_u8s8(hi, y1, f1)));
            }
        }
        const float d = h2f(b), dmin = h2f(b + 2);
        for (int t = 0; t < NT; ++t) {
            int msum = 0;
            for (int j = 0; j < 8; ++j) msum += mn[j] * (y[t][i].bsums[2 * j] + y[t][i].bsums[2 * j + 1]);
            acc[t] += d * y[t][i].d * (float)hsum_i32(iq[t]) - dmin * y[t][i].d * (float)msum;
        }
    }
    for (int t = 0; t < NT; ++t) res[t] = acc[t];
}

// Q6_K: value = d sc (q - 32), q six bits (a nibble of ql, two bits of qh), sc signed a 16 values
template <int NT>
void row_q6_k(const uint8_t* row, int nb, const Q8K* const* y, float* res) {
    const __m256i m4 = _mm256_set1_epi8(0x0F), m3 = _mm256_set1_epi8(0x03);
    float acc[NT] = {};
    for (int i = 0; i < nb; ++i) {
        const uint8_t* b = row + 210 * i;
        const int8_t* sc = (const int8_t*)(b + 192);
        __m256i iq[NT];
        for (int t = 0; t < NT; ++t) iq[t] = _mm256_setzero_si256();
        for (int n = 0; n < 2; ++n) {   // 128 values: ql[64n..], qh[32n..]
            const __m256i l0 = _mm256_loadu_si256((const __m256i*)(b + 64 * n));
            const __m256i l1 = _mm256_loadu_si256((const __m256i*)(b + 64 * n + 32));
            const __m256i h = _mm256_loadu_si256((const __m256i*)(b + 128 + 32 * n));
            __m256i q[4];
            q[0] = _mm256_or_si256(_mm256_and_si256(l0, m4), _mm256_slli_epi16(_mm256_and_si256(h, m3), 4));
            q[1] = _mm256_or_si256(_mm256_and_si256(l1, m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 2), m3), 4));
            q[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 4), m3), 4));
            q[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 6), m3), 4));
            for (int k = 0; k < 4; ++k) {   // values 128 n + 32 k ..: scales 8 n + 2 k (low 16), + 1 (high 16)
                const int s0 = sc[8 * n + 2 * k], s1 = sc[8 * n + 2 * k + 1];
                const __m256i f = _mm256_setr_epi16(s0, s0, s0, s0, s0, s0, s0, s0, s1, s1, s1, s1, s1, s1, s1, s1);
                for (int t = 0; t < NT; ++t) {
                    const __m256i yv = _mm256_loadu_si256((const __m256i*)(y[t][i].qs + 128 * n + 32 * k));
                    iq[t] = _mm256_add_epi32(iq[t], dot_u8s8(q[k], yv, f));
                }
            }
        }
        const float d = h2f(b + 208);
        for (int t = 0; t < NT; ++t) {
            int off = 0;
            for (int j = 0; j < 16; ++j) off += sc[j] * y[t][i].bsums[j];
            acc[t] += d * y[t][i].d * (float)(hsum_i32(iq[t]) - 32 * off);
        }
    }
    for (int t = 0; t < NT; ++t) res[t] = acc[t];
}

// Q8_0 against Q8_0: |w| and the sign moved onto the activation (maddubs takes an unsigned left operand)
template <int NT>
void row_q8_0(const uint8_t* row, int nb, const Q80* const* y, float* res) {
    const __m256i ones = _mm256_set1_epi16(1);
    float acc[NT] = {};
    for (int i = 0; i < nb; ++i) {
        const uint8_t* b = row + 34 * i;
        const __m256i w = _mm256_loadu_si256((const __m256i*)(b + 2));
        const __m256i aw = _mm256_sign_epi8(w, w);
        const float d = h2f(b);
        for (int t = 0; t < NT; ++t) {
            const __m256i yv = _mm256_loadu_si256((const __m256i*)y[t][i].qs);
            acc[t] += d * y[t][i].d * (float)hsum_i32(dot_u8s8(aw, _mm256_sign_epi8(yv, w), ones));
        }
    }
    for (int t = 0; t < NT; ++t) res[t] = acc[t];
}

// ---------------------------------------------------------------- the layer
struct Layout {
    int gu_type, d_type;
    int64_t n_embd, n_ff, gu_row, d_row, up_off, down_off, bytes;
};

float silu_mul(float g, float u) { return (g / (1.0f + std::exp(-g))) * u; }

template <int NT>
void gu_rows(const Layout& L, const uint8_t* blob, const void* const* act, float* const* ff, int r0, int r1) {
    float g[NT], u[NT];
    for (int r = r0; r < r1; ++r) {
        const uint8_t* gr = blob + r * L.gu_row;
        const uint8_t* ur = blob + L.up_off + r * L.gu_row;
        if (L.gu_type == kQ4_K) {
            row_q4_k<NT>(gr, (int)(L.n_embd / 256), (const Q8K* const*)act, g);
            row_q4_k<NT>(ur, (int)(L.n_embd / 256), (const Q8K* const*)act, u);
        } else {
            row_q8_0<NT>(gr, (int)(L.n_embd / 32), (const Q80* const*)act, g);
            row_q8_0<NT>(ur, (int)(L.n_embd / 32), (const Q80* const*)act, u);
        }
        for (int t = 0; t < NT; ++t) ff[t][r] = silu_mul(g[t], u[t]);
    }
}

template <int NT>
void down_rows(const Layout& L, const uint8_t* blob, const void* const* act, float* const* out, int r0, int r1) {
    float v[NT];
    for (int r = r0; r < r1; ++r) {
        const uint8_t* dr = blob + L.down_off + r * L.d_row;
        if (L.d_type == kQ6_K) row_q6_k<NT>(dr, (int)(L.n_ff / 256), (const Q8K* const*)act, v);
        else row_q8_0<NT>(dr, (int)(L.n_ff / 32), (const Q80* const*)act, v);
        for (int t = 0; t < NT; ++t) out[t][r] = v[t];
    }
}

template <template <int> class F, typename... A>
void by_nt(int nt, A... a) {
    switch (nt) {
        case 1: F<1>::run(a...); break;
        case 2: F<2>::run(a...); break;
        case 3: F<3>::run(a...); break;
        case 4: F<4>::run(a...); break;
        case 5: F<5>::run(a...); break;
        case 6: F<6>::run(a...); break;
        case 7: F<7>::run(a...); break;
        default: F<8>::run(a...); break;
    }
}
template <int NT>
struct GuRows {
    static void run(const Layout* L, const uint8_t* blob, const void* const* act, float* const* ff, int r0, int r1) {
        gu_rows<NT>(*L, blob, act, ff, r0, r1);
    }
};
template <int NT>
struct DownRows {
    static void run(const Layout* L, const uint8_t* blob, const void* const* act, float* const* out, int r0, int r1) {
        down_rows<NT>(*L, blob, act, out, r0, r1);
    }
};

// one physical core a thread, the calling thread on the first; at most max_threads
std::vector<int> physical_cpus(int max_threads) {
    cpu_set_t mask;
    CPU_ZERO(&mask);
    sched_getaffinity(0, sizeof mask, &mask);
    std::vector<int> out;
    std::set<std::pair<int, int>> seen;
    for (int c = 0; c < CPU_SETSIZE && (int)out.size() < max_threads; ++c) {
        if (!CPU_ISSET(c, &mask)) continue;
        int core = c, pkg = 0;
        char path[128];
        std::snprintf(path, sizeof path, "/sys/devices/system/cpu/cpu%d/topology/core_id", c);
        if (FILE* f = std::fopen(path, "r")) {
            if (std::fscanf(f, "%d", &core) != 1) core = c;
            std::fclose(f);
        }
        std::snprintf(path, sizeof path, "/sys/devices/system/cpu/cpu%d/topology/physical_package_id", c);
        if (FILE* f = std::fopen(path, "r")) {
            if (std::fscanf(f, "%d", &pkg) != 1) pkg = 0;
            std::fclose(f);
        }
        if (seen.insert({pkg, core}).second) out.push_back(c);
    }
    return out;
}

struct Engine {
    Layout L{};
    std::vector<int> cpus;
    int threads = 1;
    std::vector<uint8_t> act_x, act_h;   // per token activations
    std::vector<float> ff, dn;           // [n_tok * k][n_ff], [n_tok * k][n_embd]
};

Engine g_engine;

}  // namespace

extern "C" {

// Set up the pool: threads pinned one a physical core (at most max_threads); returns the thread count.
int xscpu_init(int max_threads) {
    Engine& E = g_engine;
    E.cpus = physical_cpus(max_threads > 0 ? max_threads : 1);
    E.threads = (int)E.cpus.size();
    omp_set_dynamic(0);
    omp_set_num_threads(E.threads);
#pragma omp parallel num_threads(E.threads)
    {
        cpu_set_t one;
        CPU_ZERO(&one);
        CPU_SET(E.cpus[omp_get_thread_num()], &one);
        sched_setaffinity(0, sizeof one, &one);   // tid 0: this (calling) thread
    }
    return E.threads;
}

// One decode layer on the CPU: out = residual + sum_j w_j expert_{id_j}(x) for n_tok tokens (<= 8), experts at
// arena + e * blob.  Formats: Q4_K / Q6_K and Q8_0 / Q8_0.  Returns 0, or -1 for an unsupported call.
int xscpu_layer_decode(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, int64_t gu_row, int64_t d_row,
                       int64_t up_off, int64_t down_off, const uint8_t* arena, int64_t blob, int n_expert, int k,
                       const float* x, const float* logits, const float* residual, int n_tok, float* out) {
    Engine& E = g_engine;
    if (n_tok < 1 || n_tok > kMaxTok || k < 1 || k > 16) return -1;
    const bool kq = gu_type == kQ4_K && d_type == kQ6_K, q8 = gu_type == kQ8_0 && d_type == kQ8_0;
    if (!kq && !q8) return -1;
    Layout& L = E.L;
    L = Layout{gu_type, d_type, n_embd, n_ff, gu_row, d_row, up_off, down_off, blob};
    const size_t xb = kq ? (size_t)(n_embd / 256) * sizeof(Q8K) : (size_t)(n_embd / 32) * sizeof(Q80);
    const size_t hb = kq ? (size_t)(n_ff / 256) * sizeof(Q8K) : (size_t)(n_ff / 32) * sizeof(Q80);
    const int ne = n_tok * k;
    E.act_x.resize(xb * n_tok + 64);
    E.act_h.resize(hb * ne + 64);
    E.ff.resize((size_t)ne * n_ff);
    E.dn.resize((size_t)ne * n_embd);
    int32_t ids[kMaxTok * 16];
    float wts[kMaxTok * 16];
    xso_router_top10(logits, n_tok, n_expert, k, ids, wts);
    for (int t = 0; t < n_tok; ++t) {
        if (kq) quantize_q8_k(x + t * n_embd, n_embd, (Q8K*)(E.act_x.data() + xb * t));
        else quantize_q8_0(x + t * n_embd, n_embd, (Q80*)(E.act_x.data() + xb * t));
    }
    // experts in first-routing order, each with its tokens' entries (a token's activation read once a block)
    std::vector<int> experts;
    std::vector<std::vector<int>> ent;
    for (int e = 0; e < ne; ++e) {
        auto it = std::find(experts.begin(), experts.end(), ids[e]);
        if (it == experts.end()) {
            experts.push_back(ids[e]);
            ent.emplace_back();
            it = experts.end() - 1;
        }
        ent[it - experts.begin()].push_back(e);
    }
    const int ng = (int)experts.size();
    // phase 1: gate/up rows in tasks of 32 rows; phase 2: h quantized a entry; phase 3: down rows in tasks of 64
    const int gu_chunk = 32, dn_chunk = 64;
    const int gu_tasks = (int)((n_ff + gu_chunk - 1) / gu_chunk), dn_tasks = (int)((n_embd + dn_chunk - 1) / dn_chunk);
#pragma omp parallel num_threads(E.threads)
    {
#pragma omp for schedule(dynamic, 1)
        for (int task = 0; task < ng * gu_tasks; ++task) {
            const int g = task / gu_tasks, r0 = (task % gu_tasks) * gu_chunk;
            const int r1 = (int)std::min<int64_t>(n_ff, r0 + gu_chunk);
            const void* act[kMaxTok];
            float* ffp[kMaxTok];
            const int nt = (int)ent[g].size();
            for (int j = 0; j < nt; ++j) {
                act[j] = E.act_x.data() + xb * (ent[g][j] / k);
                ffp[j] = E.ff.data() + (size_t)ent[g][j] * n_ff;
            }
            by_nt<GuRows>(nt, (const Layout*)&L, arena + (int64_t)experts[g] * blob, (const void* const*)act,
                          (float* const*)ffp, r0, r1);
        }
#pragma omp for schedule(static)
        for (int e = 0; e < ne; ++e) {
            if (kq) quantize_q8_k(E.ff.data() + (size_t)e * n_ff, n_ff, (Q8K*)(E.act_h.data() + hb * e));
            else quantize_q8_0(E.ff.data() + (size_t)e * n_ff, n_ff, (Q80*)(E.act_h.data() + hb * e));
        }
#pragma omp for schedule(dynamic, 1)
        for (int task = 0; task < ng * dn_tasks; ++task) {
            const int g = task / dn_tasks, r0 = (task % dn_tasks) * dn_chunk;
            const int r1 = (int)std::min<int64_t>(n_embd, r0 + dn_chunk);
            const void* act[kMaxTok];
            float* op[kMaxTok];
            const int nt = (int)ent[g].size();
            for (int j = 0; j < nt; ++j) {
                act[j] = E.act_h.data() + hb * ent[g][j];
                op[j] = E.dn.data() + (size_t)ent[g][j] * n_embd;
            }
            by_nt<DownRows>(nt, (const Layout*)&L, arena + (int64_t)experts[g] * blob, (const void* const*)act,
                            (float* const*)op, r0, r1);
        }
    }
    for (int t = 0; t < n_tok; ++t)
        for (int64_t c = 0; c < n_embd; ++c) {
            float s = 0.0f;
            for (int j = 0; j < k; ++j) s += E.dn[(size_t)(t * k + j) * n_embd + c] * wts[t * k + j];
            out[t * n_embd + c] = residual[t * n_embd + c] + s;
        }
    return 0;
}

// The pieces, for the checks: activations in ggml's Q8_K blocks (292 bytes a 256) and Q8_0 blocks (widened here to
// a float scale and 32 codes: 36 bytes a 32); one row dot of NT = 1 token.
void xscpu_quantize_q8_k(const float* x, int64_t n, void* y) { quantize_q8_k(x, n, (Q8K*)y); }
void xscpu_quantize_q8_0(const float* x, int64_t n, void* y) { quantize_q8_0(x, n, (Q80*)y); }
float xscpu_row_dot(int type, const uint8_t* row, int64_t n, const void* act) {
    float r = 0.0f;
    const void* a[1] = {act};
    if (type == kQ4_K) row_q4_k<1>(row, (int)(n / 256), (const Q8K* const*)a, &r);
    else if (type == kQ6_K) row_q6_k<1>(row, (int)(n / 256), (const Q8K* const*)a, &r);
    else row_q8_0<1>(row, (int)(n / 32), (const Q80* const*)a, &r);
    return r;
}

// The best of `trials` means of `reps` calls (src/kernels/iq_mmq_parity.cpp:150-163); call i takes logits set
// i % n_sets (n_sets sets of n_tok rows), so consecutive calls read other experts.  Returns microseconds a call.
double xscpu_time(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, int64_t gu_row, int64_t d_row,
                  int64_t up_off, int64_t down_off, const uint8_t* arena, int64_t blob, int n_expert, int k,
                  const float* x, const float* logit_sets, int n_sets, const float* residual, int n_tok, float* out,
                  int reps, int trials) {
    int call = 0;
    auto one = [&] {
        const float* lg = logit_sets + (size_t)(call++ % n_sets) * n_tok * n_expert;
        xscpu_layer_decode(gu_type, d_type, n_embd, n_ff, gu_row, d_row, up_off, down_off, arena, blob, n_expert, k,
                           x, lg, residual, n_tok, out);
    };
    one();
    one();
    double best = 1e30;
    for (int t = 0; t < trials; ++t) {
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < reps; ++i) one();
        best = std::min(best, std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count() /
                                  reps);
    }
    return best;
}

}  // extern "C"
