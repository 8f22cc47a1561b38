"""The CPU oracle (oracle/xs_oracle.c) pinned before it is trusted as the checker of the HIP kernels.

Pins, per function:
  dequantizers, fp16 -> fp32, canonical exp / rcp / SwiGLU: bit for bit against outputs of the reference's own
      host code (include/strata/artifact/dequant.hpp, include/strata/kernels/canon_math.hpp), committed in
      tests/golden/reference_vectors.npz, and against oracle/_ref live where the reference tree is present;
      dequantizers also against their closed forms (structural invariants).
  router: the reference test's seeded cases (src/kernels/router_top10_parity.cpp:138-184) against a stable-sort
      restatement in double (its host reference's specification), ids exact, weights 1e-5; the non-512 case of
      src/kernels/native_multi_parity.cpp:88-118 against its closed form.
  q8_1 activations: the scale / value / sum contract, brute-forced per block.
  row dots: exact double sums of the dequantized operands.
  grouped experts: the reference test's float criterion (src/kernels/native_expert_parity.cpp:46-50, sum-rel < 3e-2)
      and the exact-operand sum (1e-5).
  plan and permutation: brute-force group-bys (first occurrence; numpy's stable argsort).
  combine: a numpy float32 replay of the contract (src/kernels/native_multi_parity.cpp:136-150).
A planted mistake in the oracle (a dropped min term, a wrong nibble, a transposed operand) fails one of these.
"""
import numpy as np
import pytest


def test_fp16_exhaustive(xo, golden):
    ref, _ = golden
    got = np.array([xo.lib().xso_fp16_to_fp32(h) for h in range(65536)], np.float32)
    want = ref["fp16_to_fp32"]
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_fp32_to_fp16_matches_numpy(xo):
    rng = np.random.default_rng(1)
    f = (rng.standard_normal(50000) * np.exp(rng.uniform(-25, 12, 50000))).astype(np.float32)
    f = np.concatenate([f, np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, 5.96e-8, 2.98e-8, 2.99e-8], np.float32)])
    mine = np.array([xo.lib().xso_fp32_to_fp16(float(v)) for v in f], np.uint16)
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(mine, want)


@pytest.mark.parametrize("t", [8, 12, 14, 23])
def test_dequant_matches_reference_vectors(xo, golden, t):
    ref, _ = golden
    b = ref[f"blocks_{t}"]
    want = ref[f"dequant_{t}"]
    got = xo.dequant(t, b, want.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", [8, 12, 14, 23])
def test_dequant_matches_reference_live(xo, t):
    R = xo.ref()
    if R is None:
        pytest.skip("oracle/_ref not built here (the reference tree is only in the build container)")
    rng = np.random.default_rng(t)
    nb = 2048
    b = rng.integers(0, 256, size=nb * xo.BLOCK_BYTES[t], dtype=np.uint8)
    want = np.zeros(nb * xo.BLOCK_VALUES[t], np.float32)
    R.xsref_dequant(t, xo._a(b), nb, xo._a(want))
    got = xo.dequant(t, b, want.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _h(b, off):
    return b[off:off + 2].copy().view(np.float16).astype(np.float32)[0]


def test_dequant_structure(xo):
    """Closed forms of each format, written from the GGUF layouts independently of the oracle's loops."""
    rng = np.random.default_rng(7)
    kv = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)
    for _ in range(20):
        b = rng.integers(0, 256, 34, dtype=np.uint8)
        b[0:2] = np.float16(rng.standard_normal() * 0.01).reshape(1).view(np.uint8)
        y = xo.dequant(8, b, 32)
        assert np.array_equal(y, b[2:].view(np.int8).astype(np.float32) * _h(b, 0))
        # Q4_K: a sub-block s < 4 takes scales[s] & 63 and scales[s + 4] & 63; its codes are nibbles of qs
        b = rng.integers(0, 256, 144, dtype=np.uint8)
        b[0:2] = np.float16(abs(rng.standard_normal()) * 0.01).reshape(1).view(np.uint8)
        b[2:4] = np.float16(abs(rng.standard_normal()) * 0.01).reshape(1).view(np.uint8)
        y = xo.dequant(12, b, 256)
        d, dmin = _h(b, 0), _h(b, 2)
        for s in range(4):
            sc, m = b[4 + s] & 63, b[8 + s] & 63
            qs = b[16 + 32 * (s // 2):16 + 32 * (s // 2) + 32]
            q = (qs >> (4 * (s % 2))) & 15
            want = np.float32(d * np.float32(sc)) * q.astype(np.float32) - np.float32(dmin * np.float32(m))
            assert np.array_equal(y[32 * s:32 * s + 32], want.astype(np.float32))
        # Q6_K: value 0 = (ql[0] & 15 | (qh[0] & 3) << 4) - 32 times sc[0] times d
        b = rng.integers(0, 256, 210, dtype=np.uint8)
        b[208:210] = np.float16(rng.standard_normal() * 0.01).reshape(1).view(np.uint8)
        y = xo.dequant(14, b, 256)
        d = _h(b, 208)
        sc = b[192:208].view(np.int8)
        for v in (0, 17, 40, 70, 100, 130, 200, 255):
            n, r = divmod(v, 128)
            s, l = divmod(r, 32)
            qlb = b[64 * n + 32 * (s & 1) + l]
            q = int(((qlb >> (4 * (s >> 1))) & 15) | (((b[128 + 32 * n + l] >> (2 * s)) & 3) << 4)) - 32
            want = np.float32(np.float32(d * np.float32(sc[8 * n + 2 * s + l // 16])) * np.float32(q))
            assert y[v] == want
        # IQ4_XS: codebook values times d (ls - 32)
        b = rng.integers(0, 256, 136, dtype=np.uint8)
        b[0:2] = np.float16(rng.standard_normal() * 0.01).reshape(1).view(np.uint8)
        y = xo.dequant(23, b, 256)
        sh = int(b[2]) | (int(b[3]) << 8)
        for sb in range(8):
            ls = int(((b[4 + sb // 2] >> (4 * (sb % 2))) & 15) | (((sh >> (2 * sb)) & 3) << 4))
            dl = np.float32(_h(b, 0) * np.float32(ls - 32))
            qs = b[8 + 16 * sb:8 + 16 * sb + 16]
            assert np.array_equal(y[32 * sb:32 * sb + 16], dl * kv[qs & 15])
            assert np.array_equal(y[32 * sb + 16:32 * sb + 32], dl * kv[qs >> 4])


def test_canon_matches_reference_vectors(xo, golden):
    ref, _ = golden
    got = xo.canon_exp(ref["canon_exp_x"])
    assert np.array_equal(got.view(np.uint32), ref["canon_exp_y"].view(np.uint32))
    got = xo.canon_rcp(ref["canon_rcp_x"])
    assert np.array_equal(got.view(np.uint32), ref["canon_rcp_y"].view(np.uint32))
    got = xo.canon_silu_mul(ref["silu_g"], ref["silu_u"])
    assert np.array_equal(got.view(np.uint32), ref["silu_h"].view(np.uint32))


def test_canon_close_to_libm(xo):
    x = np.linspace(-30, 30, 10001).astype(np.float32)
    e = xo.canon_exp(x).astype(np.float64)
    assert np.max(np.abs(e / np.exp(x.astype(np.float64)) - 1)) < 4e-7
    r = np.abs(x) + 0.5
    assert np.max(np.abs(xo.canon_rcp(r) * r.astype(np.float64) - 1)) < 2e-7


# ------------------------------------------------------------------------------------------------ router

def sort_router(logits, k):
    """router_top10_parity.cpp's specification: softmax in double over all experts, stable descending sort (ties by
    index), gather, renormalise with the 2^-14 clamp."""
    T, E = logits.shape
    ids = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    for t in range(T):
        l = logits[t].astype(np.float64)
        p = np.exp(l - l.max())
        p /= p.sum()
        order = np.argsort(-p, kind="stable")[:k]
        ids[t] = order
        s = max(p[order].sum(), 6.103515625e-05)
        w[t] = (p[order].astype(np.float32).astype(np.float64) / s).astype(np.float32)
    return ids, w


def test_router_reference_cases(xo, golden):
    _, seeded = golden
    cases = seeded["router_cases"]
    base = cases[:256]                              # normal, all equal, 12-way tie, dominant: 64 rows each
    ids, w = xo.router_top10(base, 10)
    rids, rw = sort_router(base, 10)
    assert np.array_equal(ids, rids)
    assert np.max(np.abs(w - rw) / np.abs(rw)) <= 1e-5
    assert np.array_equal(ids[64:128], np.tile(np.arange(10), (64, 1)))          # all equal: the lowest indices
    for t in range(128, 192):                                                    # 12-way tie: ascending among ties
        tied = [e for e in ids[t] if e < 12]
        assert tied == sorted(tied) and tied == list(range(len(tied)))
    assert np.all(ids[192:256, 0] == np.arange(64) % 512)                        # dominant expert first
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)


def test_router_variant_rows(xo, golden):
    """The reference's variant rows (near-ties, x8 logits, NaN rows): the clean rows match the sort restatement;
    a NaN row ranks nothing and leaves the buffer's contents renormalised (router.cpp:113-115, 127-133)."""
    _, seeded = golden
    v = seeded["router_cases"][256:]
    nan_rows = np.isnan(v).any(axis=1)
    ids, w = xo.router_top10(v[~nan_rows], 10)
    rids, rw = sort_router(v[~nan_rows], 10)
    assert np.array_equal(ids, rids)
    assert np.max(np.abs(w - rw) / np.abs(rw)) <= 1e-5
    prev_ids = np.full((int(nan_rows.sum()), 10), -7, np.int32)
    prev_w = np.full((int(nan_rows.sum()), 10), 0.25, np.float32)
    ids, w = xo.router_top10(v[nan_rows], 10, prev_ids, prev_w)
    assert np.all(ids == -7)
    assert np.allclose(w, 0.1)   # ten 0.25s renormalised by their sum


def test_router_256_case(xo, golden):
    """native_multi_parity.cpp:88-118: ids in logit order (ties by index), weights exp(l - l_top) / sum over the k."""
    _, seeded = golden
    lg = seeded["router256"]
    ids, w = xo.router_top10(lg, 10)
    for t in range(3):
        order = sorted(range(256), key=lambda e: (-lg[t, e], e))[:10]
        assert list(ids[t]) == order
        ex = np.exp(lg[t, order].astype(np.float64) - lg[t, order[0]])
        assert np.max(np.abs(w[t] - ex / ex.sum())) <= 1e-5


@pytest.mark.parametrize("E,k", [(8, 2), (128, 8), (256, 8), (16, 16)])
def test_router_brute_force(xo, E, k):
    rng = np.random.default_rng(E * 31 + k)
    lg = (rng.standard_normal((64, E)) * 2).astype(np.float32)
    lg[::7] = np.round(lg[::7])                       # ties
    ids, w = xo.router_top10(lg, k)
    rids, rw = sort_router(lg, k)
    assert np.array_equal(ids, rids)
    assert np.max(np.abs(w - rw) / np.abs(rw)) <= 1e-5


def hf_group_limited(logits, bias, n_group, topk_group, k, scale, xo):
    """DeepSeek-V3's group-limited routing as its reference model code formulates it with tensors (scores, biased
    choice scores, per-group top-2 sums, group mask, masked top-k, gather, normalise): an independent formulation of
    the oracle's loops.  Uses the canonical sigmoid so scores are the same bits."""
    T, E = logits.shape
    s = xo.canon_rcp(np.float32(1.0) + xo.canon_exp(-logits)).reshape(T, E)
    c = s + bias[None, :]
    grp = np.sort(c.reshape(T, n_group, -1), axis=-1)[:, :, -2:].sum(-1)
    ids = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    for t in range(T):
        gsel = np.argsort(-grp[t], kind="stable")[:topk_group]
        mask = np.zeros(E, bool)
        for g in gsel:
            mask[g * (E // n_group):(g + 1) * (E // n_group)] = True
        cm = np.where(mask, c[t], -np.inf)
        order = np.argsort(-cm, kind="stable")[:k]
        ids[t] = order
        tot = np.float32(0)
        for e in order:
            tot = np.float32(tot + s[t, e])
        w[t] = (s[t, order] / tot * np.float32(scale)).astype(np.float32)
    return ids, w


def test_grouped_sigmoid_router(xo):
    rng = np.random.default_rng(5)
    lg = (rng.standard_normal((32, 256)) * 2).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.1).astype(np.float32)
    ids, w = xo.router_grouped_sigmoid(lg, bias, 8, 4, 8, 2.5)
    rids, rw = hf_group_limited(lg, bias, 8, 4, 8, 2.5, xo)
    assert np.array_equal(ids, rids)
    assert np.array_equal(w.view(np.uint32), rw.view(np.uint32))
    assert np.allclose(w.sum(1), 2.5, rtol=1e-6)


# ------------------------------------------------------------------------------------------------ q8_1

@pytest.mark.parametrize("cols", [256, 2048, 96])
def test_q8_1_contract(xo, cols):
    rng = np.random.default_rng(cols)
    x = rng.standard_normal((3, cols)).astype(np.float32)
    x[0, :32] = 0.0                                        # an all-zero block
    y = xo.quantize_q8_1_rows(x)
    q, d, s = xo.q8_1_values(y)
    group = 256 if cols % 256 == 0 else 32
    xb = x.reshape(-1, group)
    amax = np.abs(xb).max(1)
    dgrp = (amax * np.float32(1.0 / 127.0)).astype(np.float32)
    want_d = np.repeat(dgrp, group // 32).astype(np.float16).astype(np.float32)
    assert np.array_equal(d, want_d)
    # each value: rounded half away from zero of x * rcp(d), held to +-127
    idv = np.repeat(np.where(dgrp >= 1e-30, xo.canon_rcp(np.where(dgrp > 0, dgrp, 1)), 0), group).astype(np.float32)
    t = (x.ravel() * idv).astype(np.float32)
    want_q = np.clip(np.trunc((t + np.where(t < 0, -0.5, 0.5)).astype(np.float32)), -127, 127).astype(np.int8)
    assert np.array_equal(q.ravel(), want_q)
    assert np.allclose(s, x.reshape(-1, 32).sum(1).astype(np.float16).astype(np.float32), rtol=2e-3, atol=1e-3)


def _q8_blocks(golden):
    """The reference's canon q8 vectors (oracle/_ref's xsref_canon_q8 over canon_math.hpp:94-108): per block its
    values, scale d, inverse id and int8 codes."""
    ref, _ = golden
    n = ref["q8_n"]
    at = np.concatenate([[0], np.cumsum(n)])
    for b in range(n.size):
        yield ref["q8_x"][at[b]:at[b + 1]], ref["q8_d"][b], ref["q8_id"][b], ref["q8_q"][at[b]:at[b + 1]]


def test_q8_1_matches_reference_canon_vectors(xo, golden):
    """The oracle's q8_1 blocks against the reference's own q8_scale / q8_inv / q8_value (compiled from
    canon_math.hpp): a 256-value block is one row of 256 (one scale a 256, iq_kernels.cpp:1850-1879), a 32-value block
    one row of 32 (per-32, :1209-1223).  Codes bit for bit; the stored scale is the reference's d rounded to fp16
    (make_half2, RNE), including d held at 65504 past amax = 8.3e6 and the blocks below the 1e-30 inverse cut."""
    seen = {"zero": 0, "clamped": 0, "tiny": 0}
    for x, d, _id, q in _q8_blocks(golden):
        y = xo.quantize_q8_1_rows(x.reshape(1, -1))
        qq, dd, _ = xo.q8_1_values(y)
        assert np.array_equal(qq.ravel(), q), (x.size, d)
        assert np.array_equal(dd.astype(np.float16).view(np.uint16),
                              np.full(x.size // 32, d, np.float32).astype(np.float16).view(np.uint16))
        seen["zero"] += d == 0
        seen["clamped"] += d == 65504.0
        seen["tiny"] += 0 < d < 1e-29
    assert seen["zero"] >= 4 and seen["clamped"] >= 4 and seen["tiny"] >= 2, seen


def test_q8_1_matches_reference_live(xo):
    """The same against oracle/_ref directly, on fresh blocks (this container only: skipped where the reference tree
    was not compiled)."""
    R = xo.ref()
    if R is None:
        pytest.skip("oracle/_ref is not built here")
    rng = np.random.default_rng(77)
    for n in (256, 32):
        for _ in range(200):
            x = (rng.standard_normal(n) * np.exp(rng.uniform(-8, 16))).astype(np.float32)
            d, i, q = np.zeros(1, np.float32), np.zeros(1, np.float32), np.zeros(n, np.int8)
            R.xsref_canon_q8(xo._a(x), n, xo._a(d), xo._a(i), xo._a(q))
            qq, dd, _ = xo.q8_1_values(xo.quantize_q8_1_rows(x.reshape(1, -1)))
            assert np.array_equal(qq.ravel(), q)
            assert np.array_equal(dd, np.full(n // 32, d[0], np.float32).astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("cols", [256, 32])
def test_q8_1_block_sum_closed_form(xo, cols):
    """The fp16 sum of each block's 32 raw values (block_q8_1's s, the K-quants' min term), on values whose partial
    sums are all exact in fp32 (multiples of 1/64 below 2^17), so that every summation order gives the exact sum: the
    stored s must be that sum rounded to fp16 - and, past the largest finite half, held at +-65504 rather than inf
    (q8_1_finite, src/kernels/xe/q8_1_finite.hpp:24).  A NaN-free block stays finite."""
    rng = np.random.default_rng(cols + 5)
    rows = []
    for scale in (1.0, 40.0, 2000.0, 4000.0):                      # sums from ~10 to ~1e5
        rows.append(np.round(rng.standard_normal(cols) * scale * 64) / 64)
    rows.append(np.full(cols, 3000.0))                              # 96000 a block: held at 65504
    rows.append(np.full(cols, -3000.0))
    r = np.full(cols, 2047.0)
    r[::32] = 2047.0 + 65504.0 - 32 * 2047.0 + 8.0                  # 65512: rounds to 65504 as a half anyway
    rows.append(r)
    r = np.zeros(cols)
    r[::32] = 65519.0                                               # 65519: below the half rounding edge 65520
    rows.append(r)
    x = np.stack(rows).astype(np.float32)
    exact = x.astype(np.float64).reshape(-1, 32).sum(1)
    assert np.all(np.abs(x) < 2 ** 17) and np.all(np.abs(exact) < 2 ** 17)   # every partial sum exact
    _, _, s = xo.q8_1_values(xo.quantize_q8_1_rows(x))
    want = np.where(np.abs(exact) > 65504.0, np.sign(exact) * 65504.0, exact).astype(np.float16).astype(np.float32)
    assert np.isfinite(s).all()
    assert np.array_equal(s, want), np.flatnonzero(s != want)[:8]
    assert (np.abs(s) == 65504.0).sum() >= 3 * (cols // 32)


# ------------------------------------------------------------------------------------------------ row dots

def random_rows(xo, t, rows, n, rng):
    """Valid random rows of type t: random codes with small random fp16 scales."""
    bs = xo.BLOCK_BYTES[t]
    nb = rows * n // xo.BLOCK_VALUES[t]
    b = rng.integers(0, 256, size=(nb, bs), dtype=np.uint8)
    d = (rng.standard_normal(nb) * 0.003).astype(np.float16).view(np.uint8).reshape(nb, 2)
    if t == 14:
        b[:, 208:210] = d
    else:
        b[:, 0:2] = d
    if t == 12:
        b[:, 2:4] = np.abs(rng.standard_normal(nb) * 0.003).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


@pytest.mark.parametrize("t,n", [(8, 1024), (12, 2048), (14, 768), (23, 4096), (14, 2048), (12, 768 * 0 + 512)])
@pytest.mark.parametrize("s256", [True, False])
def test_vec_dot_exact_operands(xo, t, n, s256):
    rng = np.random.default_rng(t * 1000 + n)
    row = random_rows(xo, t, 1, n, rng)
    x = rng.standard_normal((1, n)).astype(np.float32)
    xq = xo.quantize_q8_1_rows(x) if s256 else xo.quantize_q8_1_per32(x)
    q, d, _ = xo.q8_1_values(xq)
    a = q.astype(np.float64) * d[:, None].astype(np.float64)
    wv = xo.dequant(t, row, n).astype(np.float64)
    exact = float(np.dot(wv, a.ravel()))
    scale = float(np.sum(np.abs(wv * a.ravel())))
    for calls in (False, True):    # the canonical order and the reference's per-call expressions
        got = xo.vec_dot(t, row, xq, n, s256, calls=calls)
        assert abs(got - exact) <= 1e-5 * scale


# ------------------------------------------------------------------------------------------------ experts

@pytest.mark.parametrize("gu,dt,H,F", [(8, 8, 1024, 512), (12, 14, 2048, 768), (23, 23, 1024, 512), (12, 12, 512, 256)])
def test_expert_grouped_against_float(xo, gu, dt, H, F):
    rng = np.random.default_rng(H + F + gu)
    L = xo.layout(gu, dt, H, F)
    blobs = []
    for _ in range(3):
        g = random_rows(xo, gu, F, H, rng)
        u = random_rows(xo, gu, F, H, rng)
        dn = random_rows(xo, dt, H, F, rng)
        blobs.append(np.concatenate([g, u, dn]))
        assert blobs[-1].size == L.bytes
    T = 3
    x = rng.standard_normal((T, H)).astype(np.float32)
    xq = xo.quantize_q8_1_rows(x)
    start = np.array([0, 2, 3, 5], np.int32)       # 3 groups: 2, 1 and 2 entries
    tok = np.array([0, 2, 1, 1, 2], np.int32)
    dst = np.array([4, 0, 2, 1, 3], np.int32)
    out, gate, up, hq = xo.native_expert_grouped(L, blobs, start, dst, tok, xq, 5, want_inner=True)
    gb = [blobs[0], blobs[0], blobs[1], blobs[2], blobs[2]]
    ref = xo.expert_float(L, gb, x, tok)
    for e in range(5):
        assert xo.rel_sum(out[dst[e]], ref[e]) < 3e-2               # native_expert_parity.cpp:420
    # gate rows exactly: the integer contract is the exact dot of the dequantized operands
    q, d, _ = xo.q8_1_values(xq)
    a = (q.astype(np.float64) * d[:, None]).reshape(T, H)
    for e in range(5):
        wg = xo.dequant(gu, gb[e][:F * L.gu_row], F * H).reshape(F, H).astype(np.float64)
        exact = wg @ a[tok[e]]
        scale = np.abs(wg) @ np.abs(a[tok[e]])
        assert np.all(np.abs(gate[e] - exact) <= 1e-5 * scale + 1e-30)
        # the SwiGLU and its q8_1 are the canonical ones, bit for bit
        h = xo.canon_silu_mul(gate[e], up[e])
        assert np.array_equal(hq[e * (F // 32) * 36:(e + 1) * (F // 32) * 36], xo.quantize_q8_1_per32(h))


# ------------------------------------------------------------------------------------------------ plans

def test_decode_plan_reference_cases(xo, golden):
    _, seeded = golden
    ids_all = seeded["plan_ids"]
    off = 0
    for n in range(1, 81):
        for pool in (3, 12, 40, 512):
            ids = ids_all[off:off + n]
            off += n
            p = xo.decode_plan(ids, 10)
            firsts = list(dict.fromkeys(ids.tolist()))          # distinct experts in order of first occurrence
            assert p["groups"] == len(firsts) and list(p["experts"]) == firsts
            dst = [i for e in firsts for i in range(n) if ids[i] == e]
            assert list(p["dst"]) == dst and list(p["tok"]) == [i // 10 for i in dst]
            sizes = [int((ids == e).sum()) for e in firsts]
            assert list(p["start"]) == list(np.concatenate([[0], np.cumsum(sizes)]))
            assert list(p["counts"][:3]) == [len(firsts), n, 0]
    assert off == ids_all.size


@pytest.mark.parametrize("n,E,zipf", [(16384, 128, True), (32, 8, False), (1000, 256, False), (4096, 1024, True)])
def test_prefill_route(xo, n, E, zipf):
    rng = np.random.default_rng(n + E)
    if zipf:
        p = 1.0 / np.arange(1, E + 1) ** 1.2
        ids = rng.choice(E, size=n, p=p / p.sum()).astype(np.int32)
    else:
        ids = rng.integers(0, E, n).astype(np.int32)
    k = 8
    r = xo.prefill_route(ids, k, E)
    order = np.argsort(ids, kind="stable")                 # rows: entries by expert, stable
    assert np.array_equal(r["entry"], order)
    assert np.array_equal(r["src"], order // k)
    inv = np.empty(n, np.int32)
    inv[order] = np.arange(n)
    assert np.array_equal(r["slot"], inv)
    ex = np.unique(ids)
    assert np.array_equal(r["experts"], ex)
    cnt = np.bincount(ids, minlength=E)
    assert np.array_equal(r["bounds"], np.concatenate([[0], np.cumsum(cnt[ex])]).astype(np.int32))


def test_combine_replay(xo):
    rng = np.random.default_rng(3)
    for k, shared in ((10, True), (9, True), (10, False), (2, False), (8, True)):
        n, N = 5, 2048
        parts = rng.standard_normal((n * k, N)).astype(np.float32)
        w = (rng.integers(0, 1000, n * k) / 1000.0).astype(np.float32)
        sh = rng.standard_normal((n, N)).astype(np.float32)
        got = xo.combine(parts, w, sh if shared else None, None, N, k, n)
        want = np.zeros((n, N), np.float32)
        for t in range(n):
            s = parts[t * k] * w[t * k]
            for e in range(1, k):
                s = (s + (parts[t * k + e] * w[t * k + e]).astype(np.float32)).astype(np.float32)
            if shared:
                s = (s + sh[t]).astype(np.float32)
            want[t] = s
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------------------------------------ int8 MMQ activations

def _mmq_blocks(rows=64, cols=256, seed=7):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols)).astype(np.float32) * np.float32(0.05)
    x[0, :32] = 0.0                                   # an all-zero block: d = 0, id = 0, q = 0
    x[1, 40] = 3.0e4                                  # one outlier owns its block
    x[2, :32] = np.linspace(-1, 1, 32, dtype=np.float32)
    x[3, :32] = -7.5e-20                              # a tiny block (below ~3.7e-37 the inverse overflows to inf and
                                                      # the reference's float -> int conversion is undefined)
    return x


def test_mmq_quantize_round_to_nearest_bound(xo):
    """Every code is a nearest integer to v / d, computed in float64 (|v - q d| <= d/2, up to the one float32
    rounding of v * id); |q| <= 127 and the block's largest |v| takes |q| = 127; a zero block is all zeros.  A
    wrong scale (128, 255), a truncation for the rounding or a wrong block index fails this."""
    x = _mmq_blocks()
    rows, cols = x.shape
    q, d, s = xo.mmq_quantize_parts(xo.mmq_quantize(x, None, cols, rows, True), rows, cols)
    v = x.reshape(rows, cols // 32, 32).astype(np.float64)
    qq = q.reshape(rows, cols // 32, 32).astype(np.float64)
    dd = d.astype(np.float64)[:, :, None]
    assert np.all(np.abs(qq) <= 127)
    err = np.abs(v - qq * dd)
    assert np.all(err <= dd * (0.5 + 1e-5) + 1e-45)
    amax = np.abs(v).max(axis=2)
    live = amax > 0
    assert np.all(np.abs(qq).max(axis=2)[live] == 127)
    assert np.all(qq[~live] == 0) and np.all(d[~live] == 0)
    np.testing.assert_array_equal(d, amax.astype(np.float32) / np.float32(127))


def test_mmq_quantize_halves_round_away(xo):
    """sycl::round takes halves away from zero: with amax = 127 the scale is 1 and the inverse 1, so 2.5 -> 3,
    -2.5 -> -3, 0.5 -> 1, -126.5 -> -127 (a half-to-even rounding would give 2, -2, 0, -126)."""
    x = np.zeros((1, 32), np.float32)
    x[0, :5] = [127.0, 2.5, -2.5, 0.5, -126.5]
    q, d, s = xo.mmq_quantize_parts(xo.mmq_quantize(x, None, 32, 1, True), 1, 32)
    assert d[0, 0] == 1.0
    assert list(q[0, :5]) == [127, 3, -3, 1, -127]
    assert s[0, 0] == np.float32(127 + 3 - 3 + 1 - 127)


def test_mmq_quantize_sums_ids_dup_layout(xo):
    """The block sum is d times the codes' sum in float32; rows come from ids; with dup each block (codes, scale,
    sum) appears twice in a row of 2 cols; without sums that part stays zero; the byte count is
    iq_mmq_act_bytes = rows * oc + 8 * rows * oc / 32."""
    x = _mmq_blocks(16, 128, 9)
    ids = np.array([5, 0, 15, 5, 3], np.int64)
    buf = xo.mmq_quantize(x, ids, 128, 5, True)
    assert buf.size == 5 * 128 + 8 * 5 * 4
    q, d, s = xo.mmq_quantize_parts(buf, 5, 128)
    whole_q, whole_d, whole_s = xo.mmq_quantize_parts(xo.mmq_quantize(x, None, 128, 16, True), 16, 128)
    np.testing.assert_array_equal(q, whole_q[ids])
    np.testing.assert_array_equal(d, whole_d[ids])
    np.testing.assert_array_equal(s, (d * q.reshape(5, 4, 32).astype(np.int64).sum(axis=2).astype(np.float32)))
    qd, dd, sd = xo.mmq_quantize_parts(xo.mmq_quantize(x, ids, 128, 5, True, dup=True), 5, 256)
    np.testing.assert_array_equal(qd.reshape(5, 4, 2, 32)[:, :, 1], q.reshape(5, 4, 32))
    np.testing.assert_array_equal(qd.reshape(5, 4, 2, 32)[:, :, 0], q.reshape(5, 4, 32))
    np.testing.assert_array_equal(dd.reshape(5, 4, 2)[:, :, 1], d)
    np.testing.assert_array_equal(sd.reshape(5, 4, 2)[:, :, 0], s)
    _, _, s0 = xo.mmq_quantize_parts(xo.mmq_quantize(x, ids, 128, 5, False), 5, 128)
    assert not s0.any()


# ------------------------------------------------------------------------------------------------ router projections

def test_bf16_from_f32_reference_vectors(xo, golden):
    """The oracle's f32 -> bf16 against the reference's own bf16_from_f32 (bf16_bits.hpp, compiled into the committed
    vectors): ties to even on both parities, the carry into the exponent, rounding to inf, NaNs kept quiet."""
    ref, _ = golden
    assert np.array_equal(xo.bf16_from_f32(ref["bf16_x"]), ref["bf16_y"])


def test_bf16_from_f32_reference_live(xo):
    R = xo.ref()
    if R is None:
        pytest.skip("oracle/_ref is not built (no reference tree)")
    x = np.random.default_rng(3).integers(0, 2**32, 1 << 16, dtype=np.uint64).astype(np.uint32).view(np.float32)
    y = np.zeros(x.size, np.uint16)
    R.xsref_bf16_from_f32(xo._a(x), x.size, xo._a(y))
    assert np.array_equal(xo.bf16_from_f32(x), y)


def _int_operands(rng, n_tok, n_out, n_in):
    """Small integers: every partial sum is exact in f32, so any summation order gives the integer dot product."""
    x = rng.integers(-8, 9, (n_tok, n_in)).astype(np.float32)
    w = rng.integers(-8, 9, (n_out, n_in)).astype(np.float32)
    return x, w, (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32)


@pytest.mark.parametrize("n_tok,n_out,n_in", [(1, 7, 64), (3, 5, 192), (8, 4, 2048), (2, 3, 7168), (1, 2, 1000)])
def test_projection_orders_exact_on_integers(xo, n_tok, n_out, n_in):
    """Where every sum is exact, each order returns the integer dot product: a wrong index, a transposed operand, a
    dropped pair or tail, a wrong stride fails this."""
    x, w, want = _int_operands(np.random.default_rng(n_in), n_tok, n_out, n_in)
    if n_in % 2 == 0:
        np.testing.assert_array_equal(xo.mmvf(x, w), want)
        wb = xo.bf16_from_f32(w)                       # small integers are exact in bf16
        np.testing.assert_array_equal(xo.mmvf(x, wb), want)
    np.testing.assert_array_equal(xo.gemm_rows(x, w), want)
    xb = xo.bf16_from_f32(x[0])
    wb = xo.bf16_from_f32(w)
    for form, tpr in ((0, 32), (1, 1), (2, 64), (2, 256)):
        np.testing.assert_array_equal(xo.bf16_gemv(xb, wb, form, tpr), want[0])


def test_projection_orders_close_to_fp64(xo):
    """Random operands: within the summation error bound n * eps * sum |x w| of the float64 dot products."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((4, 2048)).astype(np.float32)
    w = rng.standard_normal((16, 2048)).astype(np.float32)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    bound = 2048 * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    for got in (xo.mmvf(x, w), xo.gemm_rows(x, w)):
        assert np.all(np.abs(got - exact) <= bound)


def _spike(n_in, lanes_at):
    """x = 1, w zero but for 2^24 at element 0 and 1 at the given elements."""
    x = np.ones((1, n_in), np.float32)
    w = np.zeros((1, n_in), np.float32)
    w[0, 0] = 2.0 ** 24
    for i in lanes_at:
        w[0, i] = 1.0
    return x, w


def test_projection_order_known_answers(xo):
    """The reductions' shapes, from values where the order decides the bits (2^24 + 1 rounds back to 2^24, 2^24 + 2
    is exact):
    - mmvf at n_in 64 (B = 32, one pair a thread): ones at the pairs of threads 8 and 24 meet first in the xor
      butterfly (offset 16) and reach thread 0 as 2 -> 2^24 + 2; a sequential or an upward (1, 2, ..., 16) butterfly
      gives 2^24;
    - mmvf at n_in 2048 (B = 256, 8 groups of 32): ones in groups 2 and 6 meet in the partials' butterfly at offset
      4 -> 2^24 + 2;
    - gemm_rows: one chain in k order -> 2^24;
    - bf16 warp (lanes l, l + 32, ...): the same butterfly as mmvf -> 2^24 + 2; naive: one chain -> 2^24; the tree at
      64 threads pairs t with t + 32, then 16, ...: ones at threads 8 and 40 meet first -> 2^24 + 2."""
    x, w = _spike(64, [16, 48])                       # pairs 8 and 24 (elements 16 and 48)
    assert xo.lib().xso_mmvf_block(64) == 32
    assert xo.mmvf(x, w)[0, 0] == 2.0 ** 24 + 2
    x, w = _spike(2048, [2 * 64, 2 * 192])            # threads 64 and 192: groups 2 and 6
    assert xo.lib().xso_mmvf_block(2048) == 256
    assert xo.mmvf(x, w)[0, 0] == 2.0 ** 24 + 2
    x, w = _spike(64, [1, 2])
    assert xo.gemm_rows(x, w)[0, 0] == 2.0 ** 24
    x, w = _spike(128, [8, 24])                       # warp lanes 8 and 24
    xb, wb = xo.bf16_from_f32(x[0]), xo.bf16_from_f32(w)
    assert xo.bf16_gemv(xb, wb, 0)[0] == 2.0 ** 24 + 2
    assert xo.bf16_gemv(xb, wb, 1)[0] == 2.0 ** 24
    x, w = _spike(128, [8, 40])
    xb, wb = xo.bf16_from_f32(x[0]), xo.bf16_from_f32(w)
    assert xo.bf16_gemv(xb, wb, 2, 64)[0] == 2.0 ** 24 + 2


def test_mmvf_block_size_known_answers(xo):
    """mmvf_block_size: the fewest pair iterations, the smaller size on a tie: 64 -> 32, 192 -> 96, 448 -> 224,
    2048 -> 256, 7168 -> 256, 2 -> 32."""
    for n_in, b in ((64, 32), (192, 96), (448, 224), (2048, 256), (7168, 256), (2, 32)):
        assert xo.lib().xso_mmvf_block(n_in) == b, n_in


@pytest.mark.parametrize("gu,up", [(12, 14), (14, 8), (8, 23)])
def test_mixed_layer_pinned_to_single_type(xo, gu, up):
    """A mixed layer's rows (iq_kernels.cpp:2003-2005, 2021-2036: gate and up each a gate/up type of its own): its gate
    rows are read as a same-type layer of the gate's type reads its gate rows, its up rows as a same-type layer of the
    up type reads its gate rows - the oracle's mixed restatement equals its single-type one (pinned to the reference's
    vectors above) row for row; and the down product sees that h."""
    rng = np.random.default_rng(gu * 100 + up)
    H, F, d = 512, 256, 14
    M = xo.layout(gu, d, H, F, up)
    A = xo.layout(gu, d, H, F)       # gate rows of the gate's type
    B = xo.layout(up, d, H, F)       # the mixed layer's up rows as this layer's gate rows
    g_rows = random_rows(xo, gu, F, H, rng)
    u_rows = random_rows(xo, up, F, H, rng)
    dn = random_rows(xo, d, H, F, rng)
    mixed = np.concatenate([g_rows, u_rows, dn])
    assert mixed.size == M.bytes
    la = np.concatenate([g_rows, g_rows, dn])
    lb = np.concatenate([u_rows, u_rows, dn])
    assert la.size == A.bytes and lb.size == B.bytes
    T = 3
    x = rng.standard_normal((T, H)).astype(np.float32)
    xq = xo.quantize_q8_1_rows(x)
    start, tok, dst = np.array([0, T], np.int32), np.arange(T, dtype=np.int32), np.arange(T, dtype=np.int32)
    _, gm, um, hm = xo.native_expert_grouped(M, [mixed], start, dst, tok, xq, T, want_inner=True)
    _, ga, _, _ = xo.native_expert_grouped(A, [la], start, dst, tok, xq, T, want_inner=True)
    _, gb, _, _ = xo.native_expert_grouped(B, [lb], start, dst, tok, xq, T, want_inner=True)
    assert np.array_equal(gm.view(np.uint32), ga.view(np.uint32))
    assert np.array_equal(um.view(np.uint32), gb.view(np.uint32))
    # h = SwiGLU(gate, up) to q8_1, then the down rows: as the oracle's own steps compute them
    h = xo.canon_silu_mul(gm, um)
    assert np.array_equal(hm, xo.quantize_q8_1_per32(h.reshape(-1)))
