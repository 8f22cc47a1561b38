// xestrata-win_amd/csrc/experts_stream.hip - the grouped expert products of decode and verify windows (2-16 tokens)
// as a weight stream: the same canonical row arithmetic as experts_decode.hip (xs_units.h, bit for bit the oracle),
// with the memory side rebuilt for HBM bandwidth.
//
// Work: a task is (group, R = 64 / L consecutive rows of its matrix), L the canonical lanes of a row; lane (r, c) of a
// wave computes row r's canonical chain c over every entry of the group.  Tasks are dealt to the waves of a persistent
// grid in contiguous runs; a task is one or more steps, a step a slice of each of its rows (the units
// its lanes take next), at most ~10 KB.
//
// Memory: each wave owns a ring of slots in LDS.  A step's row slices reach its slot by LDS DMA
// (global_load_lds_dwordx4, 64 consecutive 16-byte chunks an instruction: one KB coalesced; issued from inline assembly
// so that the compiler adds no wait of its own before the slots' reads), issued slots - 1 steps
// ahead of the step being computed, so every wave keeps tens of KB in flight while it computes; a wave waits on its
// own vmcnt only (in-order returns), and needs no barrier (the slot is its own).  Every step issues the same number of
// DMA instructions (lanes with nothing to fetch read a harmless valid chunk into the slot's unread tail), so the wait
// count is a function of how many steps are in flight.  Rows keep their address modulo 16 in LDS, as the unit
// arithmetic expects.
//
// Activations and the group table live in LDS, so that no global load stands behind a wave's DMA queue (returns are
// in order: waiting for such a load would wait for every DMA issued before it).  Gate/up stages every token's q8_1
// row once a work-group (int8 values, scales, sums of 16); down copies its group's h rows into the wave's own copy
// when its (contiguous) run of tasks reaches a new group - the h rows quantized once by stream_h_kernel (the canonical
// SwiGLU and per-32 q8, also written as q8_1 blocks for the callers that read them).
#include "xs_device.h"
#include "xs_kernels.h"
#include "xs_units.h"

namespace xs {

constexpr int kStreamWaves = 8;   // waves a work-group: two a SIMD, one computes while the other waits
constexpr int kStreamWavesWide = 12;   // three a SIMD, for gate/up kernels whose registers allow it (<= 168 VGPRs)
constexpr int kStreamLds = 160 * 1024;
// bytes after each 256 int8 values of a staged gate/up activation row (Unit's PAD): a row's lanes read neighbouring
// 256-value blocks at once, which unpadded all fall in the same LDS banks
constexpr int kStreamPad = 16;
__host__ __device__ inline int stream_rowq(int n_in) { return n_in + ((n_in + 255) >> 8) * kStreamPad; }
constexpr int kStreamStepMax = 10 * 1024;
constexpr int kStreamNiMax = 12;   // DMA instructions a step at most (12 KB)

struct StreamGeom {
    int64_t mat_off;   // the matrix's offset in a blob
    int rows_total;    // rows of the matrix
    int rb;            // bytes a row
    int n_in;          // values a row
    int R;             // rows a task
    int rowgroups;     // tasks a group
    int steps;         // steps a task
    int su;            // units a lane a step
    int segb;          // bytes of a row a step
    int ncmax;         // 16-byte chunks of a row's slice in LDS
    int ni;            // DMA instructions a step
    int slot;          // bytes a slot
    int slots;         // slots a wave
    int ring;          // bytes a wave's ring
    int act_bytes;     // LDS bytes of the staged activations (gate/up: every token; down: the waves' copies)
    int wact;          // down: bytes of one wave's copy of its group's h rows
    int meta_bytes;    // LDS bytes of the group table
    int cap_groups, cap_entries;
    int n_tok;         // tokens staged (gate/up)
    int ne;            // the kernel's entries a pass
    int F;             // n_ff (outputs of gate/up, h width)
    int H;             // n_embd
    int waves;         // waves a work-group (kStreamWaves or kStreamWavesWide)
};

template <int T, bool DOWN, int LPR, int NE, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void stream_kernel(GroupedArgs a, StreamGeom G, const int8_t* __restrict__ hact_q,
                                                     const float* __restrict__ hact_d, const int* __restrict__ hact_s) {
    using U = Unit<T, !DOWN, DOWN ? 0 : kStreamPad>;
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n_in = G.n_in, nb32 = n_in >> 5, nb16 = n_in >> 4;
    // the group table in LDS: nothing a wave reads after its first DMA is a global load, whose wait (in-order
    // returns) would drain the wave's DMA queue
    uint64_t* m_ptr = (uint64_t*)lds;
    int* m_start = (int*)(m_ptr + G.cap_groups);
    int* m_ent = m_start + G.cap_groups + 1;
    const int ng = min(*a.n_groups, G.cap_groups);
    constexpr int NT = 64 * WAVES;
    for (int i = tid; i < ng; i += NT) m_ptr[i] = a.grp_ptr[i];
    for (int i = tid; i <= ng; i += NT) m_start[i] = a.grp_start[i];
    const int e_end = a.grp_start[ng];
    for (int i = tid; i < e_end && i < G.cap_entries; i += NT) m_ent[i] = DOWN ? a.ent_dst[i] : a.ent_tok[i];
    uint8_t* act = lds + G.meta_bytes;
    int8_t* aq = (int8_t*)act;
    const int rowq = stream_rowq(n_in);   // a staged token row's int8 bytes (gate/up)
    float* ad = (float*)(aq + G.n_tok * rowq);
    int* as16 = (int*)(ad + G.n_tok * nb32);
    if (!DOWN) {   // every token's q8_1 row: int8 values, the fp16 scale as a float, the sums of 16
        for (int i = tid; i < G.n_tok * nb32; i += NT) {
            const uint32_t* blk = (const uint32_t*)((const uint8_t*)a.x_q8_1 + (int64_t)i * 36);
            uint32_t wd[9];
#pragma unroll
            for (int j = 0; j < 9; ++j) wd[j] = blk[j];
            const int t = i / nb32, b = i - t * nb32;
            uint4* dst = (uint4*)(aq + (int64_t)t * rowq + 32 * b + kStreamPad * (b >> 3));
            dst[0] = make_uint4(wd[1], wd[2], wd[3], wd[4]);
            dst[1] = make_uint4(wd[5], wd[6], wd[7], wd[8]);
            ad[i] = h2f((uint16_t)(wd[0] & 0xFFFFu));
            int s0 = 0, s1 = 0;
#pragma unroll
            for (int j = 1; j <= 4; ++j) s0 = sdot4((int)wd[j], 0x01010101, s0);
#pragma unroll
            for (int j = 5; j <= 8; ++j) s1 = sdot4((int)wd[j], 0x01010101, s1);
            as16[2 * i] = s0;
            as16[2 * i + 1] = s1;
        }
    }
    __syncthreads();
    // down: this wave's copy of its current group's h rows (NE entries at most)
    int8_t* wq = (int8_t*)(act + wave * G.wact);
    float* wd8 = (float*)(wq + NE * n_in);
    int* ws16 = (int*)(wd8 + NE * nb32);
    uint8_t* ring = act + G.act_bytes + wave * G.ring;
    const int n_tasks = ng * G.rowgroups;
    const int W = gridDim.x * WAVES, w = blockIdx.x * WAVES + wave;
    const int per = (n_tasks + W - 1) / W;   // a contiguous range of tasks a wave: few group changes
    const int t_first = min(w * per, n_tasks), t_end = min(t_first + per, n_tasks);
    const int total = (t_end - t_first) * G.steps;
    const uint8_t* dummy = (const uint8_t*)a.gate;   // 16-byte aligned scratch: the chunks nobody reads

    // this lane's chunk of each DMA instruction, fixed for the whole kernel: row rr[j] of the task (-1: none), byte
    // cc[j] of that row's slice, rrb[j] = rr[j] * rb
    int rr[kStreamNiMax], cc[kStreamNiMax], rrb[kStreamNiMax];
#pragma unroll
    for (int j = 0; j < kStreamNiMax; ++j) {
        const int idx = 64 * j + lane;
        const int r_ = idx / G.ncmax;
        rr[j] = j < G.ni && r_ < G.R ? r_ : -1;
        cc[j] = 16 * (idx - r_ * G.ncmax);
        rrb[j] = r_ * G.rb;
    }
    const uint32_t ring_off = lds_offset(ring);
    auto issue = [&](int q) {   // the DMA of step q of this wave's sequence
        const int task = t_first + q / G.steps, i_s = q - (q / G.steps) * G.steps;
        const int i_g = task / G.rowgroups, i_rg = task - i_g * G.rowgroups;
        const uint8_t* blob = (const uint8_t*)m_ptr[i_g];
        const bool ok_b = ((uintptr_t)blob & 15u) == 0;
        const int r0_ = i_rg * G.R;
        const int so0 = (int)G.mat_off + r0_ * G.rb + i_s * G.segb;
        const uint32_t slot_off = ring_off + (uint32_t)((q % G.slots) * G.slot);
#pragma unroll
        for (int j = 0; j < kStreamNiMax; ++j) {
            if (j >= G.ni) break;
            const int so = so0 + rrb[j];
            const int a0 = so & ~15, a1 = (so + G.segb + 15) & ~15;
            const bool live = ok_b && rr[j] >= 0 && r0_ + rr[j] < G.rows_total && a0 + cc[j] < a1;
            dma16_nt(live ? blob + a0 + cc[j] : dummy, __builtin_amdgcn_readfirstlane(slot_off + 1024 * j));
        }
    };

    const int pre = min(G.slots - 1, total);   // the first slots - 1 steps in flight before any is computed
    for (int q = 0; q < pre; ++q) issue(q);
    const int r = lane / LPR, c = lane - (lane / LPR) * LPR;
    // entries a call of the unit arithmetic: two (a group has one or two entries most of the time, and the unit's
    // weights are re-read from LDS for the next two rather than held for eight in registers)
    constexpr int NP = NE < 2 ? NE : 2;
    float acc[NE];
    int src[NE];   // a rank's activation row: its token (gate/up) or its slot in this wave's copy (down)
    int n_all = 0, e0 = 0, r0 = 0, staged_g = -1, staged_p = -1;
    bool ok = false;
    for (int q = 0; q < total; ++q) {
        if (q + G.slots - 1 < total) issue(q + G.slots - 1);
        vm_wait_le(min(G.slots - 1, total - 1 - q) * G.ni);
        const int task = t_first + q / G.steps, s = q - (q / G.steps) * G.steps;
        const int g = task / G.rowgroups;
        if (s == 0) {
            r0 = (task - g * G.rowgroups) * G.R;
            e0 = m_start[g];
            n_all = m_start[g + 1] - e0;
            ok = (m_ptr[g] & 15u) == 0 && n_all > 0 && (G.steps == 1 || n_all <= NE);
            if (!ok && lane == 0 && r0 == 0) atomicOr(a.err, 1);
        }
        const uint8_t* slot = ring + (q % G.slots) * G.slot;
        const bool live = ok && r < G.R && r0 + r < G.rows_total;
        const int64_t so = G.mat_off + (int64_t)(r0 + r) * G.rb + (int64_t)s * G.segb;
        const int roff = r * G.ncmax * 16 + (int)(so & 15) - s * G.segb;
        // passes of NE entries over a one-step task's slot (down: the group's h rows staged NE at a time into this
        // wave's copy); a task of several steps has one pass (n <= NE), its chains kept across the steps
        const int npass = ok ? (n_all + NE - 1) / NE : 0;   // more than one only for one-step tasks
        for (int pass = 0; pass < npass; ++pass) {
            const int p0 = pass * NE, n = min(n_all - p0, NE);
            if (DOWN && (staged_g != g || staged_p != p0)) {   // h rows into this wave's copy (a full wait)
                staged_g = g;
                staged_p = p0;
                for (int i = lane; i < n * (n_in >> 4); i += 64) {
                    const int e = i / (n_in >> 4), k = i - e * (n_in >> 4);
                    ((uint4*)(wq + e * n_in))[k] = ((const uint4*)(hact_q + (int64_t)(e0 + p0 + e) * n_in))[k];
                }
                for (int i = lane; i < n * nb32; i += 64) {
                    const int e = i / nb32, k = i - e * nb32;
                    wd8[e * nb32 + k] = hact_d[(int64_t)(e0 + p0 + e) * nb32 + k];
                }
                for (int i = lane; i < n * nb16; i += 64) {
                    const int e = i / nb16, k = i - e * nb16;
                    ws16[e * nb16 + k] = hact_s[(int64_t)(e0 + p0 + e) * nb16 + k];
                }
            }
            if (DOWN || s == 0 || npass > 1) {
#pragma unroll
                for (int e = 0; e < NE; ++e) {
                    acc[e] = 0.0f;
                    src[e] = DOWN ? (e < n ? e : 0) : m_ent[e0 + p0 + (e < n ? e : 0)];
                }
            }
            if (live) {
                for (int i = 0; i < G.su; ++i) {
                    const int u = s * LPR * G.su + c + LPR * i;
#pragma unroll
                    for (int pp = 0; pp < NE; pp += NP) {
                        if (pp >= n) break;
                        Act av[NP];
#pragma unroll
                        for (int e = 0; e < NP; ++e) {
                            const int j = src[pp + e];
                            av[e] = DOWN ? Act{wq + j * n_in, wd8 + j * nb32, ws16 + j * nb16}
                                         : Act{aq + j * rowq, ad + j * nb32, as16 + j * nb16};
                        }
                        U::template apply<NP>(slot, roff, u, av, min(n - pp, NP), *(float(*)[NP])(acc + pp));
                    }
                }
            }
            if (s == G.steps - 1) {
#pragma unroll
                for (int e = 0; e < NE; ++e) acc[e] = group_sum<LPR>(acc[e]);
                if (live && c == 0) {
                    const int row = r0 + r;
                    for (int e = 0; e < n; ++e) {
                        if (DOWN) a.out[(int64_t)m_ent[e0 + p0 + e] * G.H + row] = acc[e];
                        else if (row < G.F) a.gate[(int64_t)(e0 + p0 + e) * G.F + row] = acc[e];
                        else a.up[(int64_t)(e0 + p0 + e) * G.F + (row - G.F)] = acc[e];
                    }
                }
            }
        }
    }
}

// h = SwiGLU(gate, up) of every entry with the canonical arithmetic, quantized per 32 (the canonical q8): int8 values,
// the fp16 scale as a float, the sums of 16 (the down stream's activations), and the same as q8_1 blocks (hq: the
// fp16 scale and the fp16 sum of the h values, q8_1_finite); 32 neighbouring lanes hold one block
__global__ __launch_bounds__(256) void stream_h_kernel(GroupedArgs a, int F, int8_t* __restrict__ hact_q,
                                                       float* __restrict__ hact_d, int* __restrict__ hact_s) {
    const int ng = min(*a.n_groups, (int)a.cap_groups);
    const int n_ent = a.grp_start[ng] - a.grp_start[0];
    const int e_first = a.grp_start[0];
    const int64_t total = (int64_t)n_ent * F;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i - threadIdx.x < total; i += (int64_t)gridDim.x * 256) {
        const bool live = i < total;
        const int64_t gi = (int64_t)e_first * F + (live ? i : 0);
        const float h = canon_silu_mul(a.gate[gi], a.up[gi]);
        const float amax = group_max<32>(fabsf(h));
        const float sum = group_sum<32>(h);
        const float d = q8_scale(amax);
        const int q = q8_value(h, q8_inv(d));
        const int qs16 = (int)group_sum<16>((float)q);   // exact: at most 16 x 127
        if (!live) continue;
        const int64_t e = gi / F, col = gi - e * F;
        hact_q[gi] = (int8_t)q;
        const uint16_t hd = f2h(d);
        if ((col & 31) == 0) hact_d[e * (F >> 5) + (col >> 5)] = h2f(hd);
        if ((col & 15) == 0) hact_s[e * (F >> 4) + (col >> 4)] = qs16;
        uint8_t* blk = (uint8_t*)a.hq + (e * (F >> 5) + (col >> 5)) * 36;
        blk[4 + (col & 31)] = (uint8_t)q;
        if ((col & 31) == 0) *(uint32_t*)blk = (uint32_t)hd | ((uint32_t)f2h(q8_1_finite(sum)) << 16);
    }
}

namespace {

template <bool DOWN>
bool stream_geom(const ExpertLayout& L, int unit, int block_values, int block_bytes, int n_tok, int64_t cap_groups,
                 int64_t cap_entries, StreamGeom& G, bool wide = false) {
    G.n_in = DOWN ? (int)L.n_ff : (int)L.n_embd;
    G.rows_total = DOWN ? (int)L.n_embd : (int)(2 * L.n_ff);
    G.rb = (int)(DOWN ? L.d_row : L.gu_row);
    G.mat_off = DOWN ? L.down_off : 0;
    G.F = (int)L.n_ff;
    G.H = (int)L.n_embd;
    if (cap_groups <= 0 || cap_entries <= 0 || cap_groups > 4096 || cap_entries > 4096) return false;
    G.cap_groups = (int)cap_groups;
    G.cap_entries = (int)cap_entries;
    G.meta_bytes = (int)((8 * cap_groups + 4 * (cap_groups + 1) + 4 * cap_entries + 15) & ~15);
    const int units = G.n_in / unit;
    const int lpr = canon_lanes(units);
    if (lpr < 4) return false;
    const int upl = units / lpr;
    const int upb = block_values / unit;   // units a block
    G.R = 64 / lpr;
    G.rowgroups = (G.rows_total + G.R - 1) / G.R;
    const int unit_bytes = block_bytes / upb;   // exact when the step is whole blocks
    G.su = 0;
    for (int su = upl; su >= 1; --su) {
        if (upl % su || (lpr * su) % upb) continue;
        if (G.R * lpr * su * unit_bytes <= kStreamStepMax || su == 1) {
            G.su = su;
            break;
        }
    }
    if (G.su == 0) return false;
    G.steps = upl / G.su;
    G.segb = lpr * G.su / upb * block_bytes;
    // a row's slice in 16-byte chunks: exact when every slice starts on a 16-byte boundary, else one more
    const bool al16 = G.rb % 16 == 0 && G.mat_off % 16 == 0 && G.segb % 16 == 0;
    G.ncmax = al16 ? G.segb / 16 : (G.segb + 15) / 16 + 1;
    G.ni = (G.R * G.ncmax + 63) / 64;
    if (G.ni > kStreamNiMax) return false;
    G.slot = G.ni * 1024;
    const int row_act = G.n_in + G.n_in / 32 * 4 + G.n_in / 16 * 4;
    G.n_tok = DOWN ? 0 : n_tok;
    G.ne = DOWN ? 4 : n_tok <= 4 ? 4 : 8;   // the kernel's NE: entries a pass
    if (G.steps != 1 && n_tok > G.ne) return false;   // passes re-read their one step's slot
    G.wact = DOWN ? ((G.ne * row_act + 15) & ~15) : 0;
    auto fit = [&](int waves) {
        G.waves = waves;
        G.act_bytes = DOWN ? waves * G.wact : ((n_tok * (row_act + stream_rowq(G.n_in) - G.n_in) + 15) & ~15);
        const int ring = (kStreamLds - G.meta_bytes - G.act_bytes) / waves;
        G.slots = ring / G.slot;
        while (G.slots > 1 && (G.slots - 1) * G.ni > 63) --G.slots;
    };
    fit(kStreamWaves);
    if (G.slots < 1) return false;
    // one slot a ring: every wave waits for each step it fetches, so more waves a SIMD hide more; three a SIMD where
    // the rings still hold a slot and the kernel's registers allow it (gate/up of the formats but Q4_K)
    if (G.slots == 1 && wide) {
        fit(kStreamWavesWide);
        if (G.slots < 1) fit(kStreamWaves);
    }
    G.ring = G.slots * G.slot;
    return true;
}

template <int T, bool DOWN, int LPR>
hipError_t launch_lpr(const GroupedArgs& a, const StreamGeom& G, hipStream_t s, const int8_t* hq, const float* hd,
                      const int* hs) {
    constexpr bool kWide = !DOWN && T != kQ4_K;   // the instances that fit three waves a SIMD
    void (*kern)(GroupedArgs, StreamGeom, const int8_t*, const float*, const int*) =
        kWide && G.waves == kStreamWavesWide
            ? (G.ne <= 4 ? stream_kernel<T, DOWN, LPR, 4, kWide ? kStreamWavesWide : kStreamWaves>
                         : stream_kernel<T, DOWN, LPR, 8, kWide ? kStreamWavesWide : kStreamWaves>)
            : (G.ne <= 4 ? stream_kernel<T, DOWN, LPR, 4, kStreamWaves> : stream_kernel<T, DOWN, LPR, 8, kStreamWaves>);
    const size_t lds = (size_t)G.meta_bytes + (size_t)G.act_bytes + (size_t)G.waves * G.ring;
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    hipLaunchKernelGGL(kern, dim3((unsigned)cus), dim3(64 * G.waves), lds, s, a, G, hq, hd, hs);
    return hipGetLastError();
}

template <int T, bool DOWN>
hipError_t launch_stream_t(const ExpertLayout& L, const GroupedArgs& a, hipStream_t s) {
    constexpr int bv = T == kQ8_0 ? 32 : 256;
    constexpr int bb = T == kQ8_0 ? 34 : T == kQ4_K ? 144 : T == kQ6_K ? 210 : 136;
    const int unit = DOWN || T == kQ8_0 ? 32 : 256;
    StreamGeom G;
    if (!stream_geom<DOWN>(L, unit, bv, bb, a.max_entries, a.cap_groups, a.cap_entries_hint, G, !DOWN && T != kQ4_K))
        return hipErrorNotSupported;
    const size_t f = (size_t)a.cap_entries_hint * (size_t)L.n_ff;   // the h region's int8 values
    int8_t* hq = (int8_t*)a.hact;
    float* hd = (float*)(hq + ((f + 255) & ~(size_t)255));
    int* hs = (int*)((uint8_t*)hd + (((f / 32) * 4 + 255) & ~(size_t)255));
    if (DOWN) {
        hipLaunchKernelGGL(stream_h_kernel, dim3(1024), dim3(256), 0, s, a, (int)L.n_ff, hq, hd, hs);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    switch (canon_lanes(G.n_in / unit)) {
        case 8: return launch_lpr<T, DOWN, 8>(a, G, s, hq, hd, hs);
        case 4: return launch_lpr<T, DOWN, 4>(a, G, s, hq, hd, hs);
        default: return hipErrorNotSupported;
    }
}

}  // namespace

bool stream_usable(const ExpertLayout& L, int n_tok, int64_t cap_groups, int64_t cap_entries) {
    if (n_tok < 2 || n_tok > 16 || mixed_gu(L)) return false;   // (one gate/up type: the gate and up rows as one matrix)
    // the DMA reads whole 16-byte chunks: a matrix's last chunk must stay inside the blob
    if (L.bytes % 16 || L.up_off % 16 || L.down_off % 16) return false;
    const int types[2] = {L.gu_type, L.d_type};
    for (int t : types)
        if (t != kQ4_K && t != kQ6_K && t != kQ8_0 && t != kIQ4_XS) return false;
    StreamGeom G;
    const int gbv = L.gu_type == kQ8_0 ? 32 : 256, dbv = L.d_type == kQ8_0 ? 32 : 256;
    auto bytes = [](int t) { return t == kQ8_0 ? 34 : t == kQ4_K ? 144 : t == kQ6_K ? 210 : 136; };
    return stream_geom<false>(L, L.gu_type == kQ8_0 ? 32 : 256, gbv, bytes(L.gu_type), n_tok, cap_groups, cap_entries,
                              G) &&
           stream_geom<true>(L, 32, dbv, bytes(L.d_type), n_tok, cap_groups, cap_entries, G);
}

hipError_t launch_stream_gu(const ExpertLayout& L, const GroupedArgs& a, hipStream_t s) {
    switch (L.gu_type) {
        case kQ4_K: return launch_stream_t<kQ4_K, false>(L, a, s);
        case kQ6_K: return launch_stream_t<kQ6_K, false>(L, a, s);
        case kQ8_0: return launch_stream_t<kQ8_0, false>(L, a, s);
        case kIQ4_XS: return launch_stream_t<kIQ4_XS, false>(L, a, s);
        default: return hipErrorNotSupported;
    }
}

hipError_t launch_stream_down(const ExpertLayout& L, const GroupedArgs& a, hipStream_t s) {
    switch (L.d_type) {
        case kQ4_K: return launch_stream_t<kQ4_K, true>(L, a, s);
        case kQ6_K: return launch_stream_t<kQ6_K, true>(L, a, s);
        case kQ8_0: return launch_stream_t<kQ8_0, true>(L, a, s);
        case kIQ4_XS: return launch_stream_t<kIQ4_XS, true>(L, a, s);
        default: return hipErrorNotSupported;
    }
}

}  // namespace xs
