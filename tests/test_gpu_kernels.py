"""GPU parity of the single kernels against the CPU oracle, through the C ABI (libxsmoe.so).

Bars: integer / byte / index results bit for bit (dequantized weights, q8_1 blocks, ids, plans, permutations, the
combine's bits); floating-point results within the tolerance written in each test."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def t2n(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("t", [8, 12, 14, 23])
def test_dequant_reference_vectors(xm, golden, t):
    """The GPU dequantizer against outputs of the reference's own host dequantizer (dequant.hpp), bit for bit."""
    ref, _ = golden
    b = torch.from_numpy(ref[f"blocks_{t}"].ravel()).to(DEV)
    want = ref[f"dequant_{t}"]
    got = t2n(xm.iq_dequant_f32(t, b, want.size))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t,tol", [(8, 0.01), (12, 0.12), (14, 0.04), (23, 0.12)])
def test_quantize_dequantize(xm, xo, t, tol):
    """This library's quantizer gives valid blocks close to the input; the GPU dequantizer equals the oracle's on
    them bit for bit; the bf16 dequantizer is the fp32 one rounded to nearest even."""
    g = torch.Generator().manual_seed(t)
    x = (torch.randn(64, 2048, generator=g) * 0.02).to(DEV)
    blocks = xm.quantize_rows(t, x.reshape(-1))
    n = x.numel()
    got = xm.iq_dequant_f32(t, blocks, n)
    want = xo.dequant(t, t2n(blocks), n)
    assert np.array_equal(t2n(got).view(np.uint32), want.view(np.uint32))
    err = float(torch.sqrt(torch.mean((got - x.reshape(-1)) ** 2)) / torch.sqrt(torch.mean(x ** 2)))
    assert err < tol, err
    bf = xm.iq_dequant_bf16(t, blocks, n)
    assert torch.equal(bf.view(torch.bfloat16), got.to(torch.bfloat16))


@pytest.mark.parametrize("rows,cols", [(1, 2048), (16, 2048), (4, 1024), (3, 7168), (5, 96), (7, 768)])
def test_quantize_q8_1_rows(xm, xo, rows, cols):
    g = torch.Generator().manual_seed(rows * cols)
    x = torch.randn(rows, cols, generator=g)
    x[0, :32] = 0.0
    x[-1, 5] = 1e6                                    # a massive activation: the fp16 sum clamps (q8_1_finite)
    got = t2n(xm.quantize_q8_1_rows(x.to(DEV)))
    want = xo.quantize_q8_1_rows(x.numpy())
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n", [256, 32])
def test_quantize_q8_1_reference_canon_vectors(xm, xo, golden, n):
    """q8_1 on the GPU against the reference's own canon q8_scale / q8_inv / q8_value (compiled from canon_math.hpp
    into tests/golden/reference_vectors.npz): each n-value block as one row; codes bit for bit, the stored scale the
    reference's d rounded to fp16 - including amax = 0, amax under the 1e-30 inverse cut, d held at 65504.  The block
    sums equal the oracle's (whose sums are pinned in closed form, tests/test_oracle.py)."""
    ref, _ = golden
    sizes = ref["q8_n"]
    at = np.concatenate([[0], np.cumsum(sizes)])
    sel = np.flatnonzero(sizes == n)
    x = np.stack([ref["q8_x"][at[b]:at[b + 1]] for b in sel])
    got = t2n(xm.quantize_q8_1_rows(torch.from_numpy(x).to(DEV)))
    q, d, _ = xo.q8_1_values(got)
    assert np.array_equal(q.reshape(len(sel), n), np.stack([ref["q8_q"][at[b]:at[b + 1]] for b in sel]))
    want_d = np.repeat(ref["q8_d"][sel], n // 32).astype(np.float16)
    assert np.array_equal(d.astype(np.float16).view(np.uint16), want_d.view(np.uint16))
    assert np.array_equal(got, xo.quantize_q8_1_rows(x))


def router_cases(golden):
    _, seeded = golden
    return seeded["router_cases"]


def test_router_reference_cases(xm, xo, golden):
    """The reference test's seeded logits (router_top10_parity.cpp:138-184, E=512, k=10): ids exact, weights bit for
    bit against the oracle; NaN rows leave their ranks' previous contents, renormalised."""
    lg = router_cases(golden)
    prev_ids = np.full((lg.shape[0], 10), -7, np.int32)
    prev_w = np.full((lg.shape[0], 10), 0.25, np.float32)
    ids = torch.from_numpy(prev_ids).to(DEV)
    w = torch.from_numpy(prev_w).to(DEV)
    xm.router_top10(torch.from_numpy(lg).to(DEV), 10, ids, w)
    rids, rw = xo.router_top10(lg, 10, prev_ids, prev_w)
    assert np.array_equal(t2n(ids), rids)
    assert np.array_equal(t2n(w).view(np.uint32), rw.view(np.uint32))


@pytest.mark.parametrize("T,E,k", [(4, 8, 2), (16, 128, 8), (2048, 128, 8), (8, 256, 8), (3, 256, 10), (64, 1024, 64),
                                   (33, 100, 7)])
def test_router_shapes(xm, xo, T, E, k):
    g = torch.Generator().manual_seed(T * E + k)
    lg = torch.randn(T, E, generator=g) * 2
    lg[::5] = torch.round(lg[::5])                          # exact ties
    ids, w = xm.router_top10(lg.to(DEV), k)
    rids, rw = xo.router_top10(lg.numpy(), k)
    assert np.array_equal(t2n(ids), rids)
    assert np.array_equal(t2n(w).view(np.uint32), rw.view(np.uint32))


def _edge_logits(kind, T, E, rng):
    if kind == "equal":           # every p equal: the tie order alone decides (too many candidates for the fast path)
        return np.zeros((T, E), np.float32)
    if kind == "near_equal":      # p within a few ulps: one crowded bucket
        return (rng.standard_normal((T, E)) * 1e-6).astype(np.float32)
    if kind == "few_large":       # k clear winners, the rest far below (a candidate set of exactly k)
        lg = rng.standard_normal((T, E)).astype(np.float32) - 40.0
        for t in range(T):
            lg[t, rng.choice(E, 8, replace=False)] += 60.0
        return lg
    if kind == "underflow":       # exp underflows to 0 for most experts: zero p ranked by index
        return np.tile(np.linspace(0.0, -3000.0, E, dtype=np.float32)[rng.permutation(E)], (T, 1))
    if kind == "neg_inf":         # -inf logits: p = 0 exactly
        lg = rng.standard_normal((T, E)).astype(np.float32)
        lg[:, ::3] = -np.inf
        return lg
    if kind == "two_levels":      # two tied levels straddling rank k
        lg = np.full((T, E), -1.0, np.float32)
        lg[:, : E // 16 + 3] = 1.0
        return lg
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["equal", "near_equal", "few_large", "underflow", "neg_inf", "two_levels"])
@pytest.mark.parametrize("E,k", [(128, 8), (256, 8), (512, 10), (64, 6), (1024, 40)])
def test_router_selection_edges(xm, xo, kind, E, k):
    """Distributions that take each branch of the device selection (the bucket fast path, its fallback to k argmax
    passes, ties at the k-th key, zero p, k above 32): ids and weights bit for bit against the oracle."""
    rng = np.random.default_rng(E * 31 + k)
    lg = _edge_logits(kind, 12, E, rng)
    ids, w = xm.router_top10(torch.from_numpy(lg).to(DEV), k)
    rids, rw = xo.router_top10(lg, k)
    assert np.array_equal(t2n(ids), rids)
    assert np.array_equal(t2n(w).view(np.uint32), rw.view(np.uint32))


def test_router_zipf_prefill(xm, xo):
    """Config 3's skewed logits: log-Zipf(1.2) popularity plus per-token Gumbel noise."""
    rng = np.random.default_rng(3)
    E, T = 128, 2048
    pop = -1.2 * np.log(np.arange(1, E + 1))[rng.permutation(E)]
    lg = (pop[None, :] + rng.gumbel(size=(T, E))).astype(np.float32)
    ids, w = xm.router_top10(torch.from_numpy(lg).to(DEV), 8)
    rids, rw = xo.router_top10(lg, 8)
    assert np.array_equal(t2n(ids), rids)
    assert np.array_equal(t2n(w).view(np.uint32), rw.view(np.uint32))


@pytest.mark.parametrize("E,G,TG,k,ties", [(256, 8, 4, 8, False), (256, 8, 4, 8, True), (64, 4, 2, 6, True),
                                          (128, 8, 3, 8, False), (160, 5, 2, 8, True), (512, 8, 4, 8, False),
                                          (72, 3, 2, 6, True), (1024, 64, 8, 16, False)])
def test_grouped_sigmoid_router(xm, xo, E, G, TG, k, ties):
    # the register form (groups on whole lanes: 256/8, 64/4, 128/8, 160/5 with idle lanes, 512/8, 1024/64) and the
    # LDS form (72/3: 12 lanes a group); ties: logits on a 0.25 grid and no bias, so group scores and experts tie
    rng = np.random.default_rng(E + G + k)
    T = 37                                              # not a multiple of the 4 tokens a work-group
    lg = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    if ties:
        lg = (np.round(lg * 4) / 4).astype(np.float32)
        bias = None
    ids, w = xm.router_grouped_sigmoid(torch.from_numpy(lg).to(DEV), None if bias is None else
                                       torch.from_numpy(bias).to(DEV), G, TG, k, 2.5)
    rids, rw = xo.router_grouped_sigmoid(lg, bias, G, TG, k, 2.5)
    assert np.array_equal(t2n(ids), rids)
    assert np.array_equal(t2n(w).view(np.uint32), rw.view(np.uint32))


def test_router_logits(xm):
    g = torch.Generator().manual_seed(9)
    x = torch.randn(4, 1024, generator=g)
    wr = torch.randn(8, 1024, generator=g) * 0.02
    got = t2n(xm.router_logits_f32(x.to(DEV), wr.to(DEV))).astype(np.float64)
    want = x.double().numpy() @ wr.double().numpy().T
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(x.numpy()) @ np.abs(wr.numpy()).T)


def test_resident_plan_reference_cases(xm, xo, golden):
    """resident_plan_parity.cpp's cases: n = 1..80 entries from pools of 3..512 experts (seeded ids), a slot table
    that is not the identity, with and without slot offsets; every word the host pool reads, and the skip word."""
    _, seeded = golden
    ids_all = seeded["plan_ids"]
    K, NE, capx, blob, ring = 10, 512, 80, 1337, 7
    cache_base = 0x40000000                                    # never dereferenced
    res = np.array([(e * 37 + 11) % 1000 for e in range(NE)], np.int32)
    off = np.array([s * 4096 + (s % 7) * 64 for s in range(1024)], np.uint64)
    d_res = torch.from_numpy(res).to(DEV)
    d_off = torch.from_numpy(off.view(np.int64)).to(DEV)
    words = xm.plan_words(capx)
    o = xm.plan_offsets(capx)
    at = 0
    for n in range(1, 81):
        for variant, pool in enumerate((3, 12, 40, 512)):
            ids = ids_all[at:at + n]
            at += n
            use_off = (n + variant) % 2 == 1
            plan = torch.full((words + 2,), -1414812757, dtype=torch.int32, device=DEV)   # 0xABABABAB
            skip = torch.zeros(1, dtype=torch.int32, device=DEV)
            xm.resident_plan(torch.from_numpy(ids).to(DEV), K, d_res, NE, cache_base, d_off if use_off else None,
                             blob, plan, capx, skip, ring)
            p = t2n(plan)
            r = xo.decode_plan(ids, K)
            g = r["groups"]
            assert int(t2n(skip)[0]) == ring
            assert list(p[:3]) == [g, n, 0]
            assert np.array_equal(p[4:4 + g + 1], r["start"])
            assert np.array_equal(p[o["dst"]:o["dst"] + n], r["dst"])
            assert np.array_equal(p[o["tok"]:o["tok"] + n], r["tok"])
            ptr = p[o["ptr"]:o["ptr"] + 2 * g].view(np.uint64)
            slots = res[r["experts"]]
            want = cache_base + (off[slots] if use_off else slots.astype(np.uint64) * blob)
            assert np.array_equal(ptr, want.astype(np.uint64))
            assert p[o["start2"]] == n


def test_resident_plan_not_resident(xm):
    res = torch.arange(512, dtype=torch.int32, device=DEV)
    res[5] = -1
    plan = torch.full((xm.plan_words(80),), 7, dtype=torch.int32, device=DEV)
    skip = torch.full((1,), 7, dtype=torch.int32, device=DEV)
    ids = torch.arange(1, 11, dtype=torch.int32, device=DEV)
    xm.resident_plan(ids, 10, res, 512, 0x40000000, None, 1337, plan, 80, skip, 7)
    assert int(skip[0]) == 0
    assert bool((plan == 7).all())


@pytest.mark.parametrize("n,E,zipf", [(16384, 128, True), (32, 8, False), (4096, 1024, True), (1000, 256, False),
                                      (4, 128, False), (65536, 256, True)])
def test_prefill_route(xm, xo, n, E, zipf):
    rng = np.random.default_rng(n + E)
    if zipf:
        p = 1.0 / np.arange(1, E + 1) ** 1.2
        ids = rng.choice(E, size=n, p=p / p.sum()).astype(np.int32)
    else:
        ids = rng.integers(0, E, n).astype(np.int32)
    k = 8
    r = xm.prefill_route(torch.from_numpy(ids).to(DEV), k, E, cache_base=0x1000, blob=4096, with_ptr=True)
    want = xo.prefill_route(ids, k, E)
    g = int(r["n_groups"][0])
    assert g == want["groups"]
    for key in ("src", "slot", "entry"):
        assert np.array_equal(t2n(r[key]), want[key]), key
    assert np.array_equal(t2n(r["bounds"])[:g + 1], want["bounds"])
    assert np.array_equal(t2n(r["experts"])[:g], want["experts"])
    assert np.array_equal(t2n(r["grp_ptr"])[:g], 0x1000 + want["experts"].astype(np.int64) * 4096)


def test_prefill_route_bad_id(xm):
    ids = torch.tensor([1, 2, 300, 4], dtype=torch.int32, device=DEV)
    r = xm.prefill_route(ids, 2, 128)
    assert int(r["n_groups"][0]) == -1


@pytest.mark.parametrize("k,shared,gated,n", [(8, False, False, 16), (10, True, False, 5), (9, True, False, 3),
                                              (2, False, False, 4), (8, True, True, 6), (1, False, False, 2)])
def test_combine(xm, xo, k, shared, gated, n):
    N = 2048
    g = torch.Generator().manual_seed(k * 100 + n)
    parts = torch.randn(n * k, N, generator=g)
    w = torch.randint(0, 1000, (n * k,), generator=g).float() / 1000
    sh = torch.randn(n, N, generator=g)
    gate = torch.randn(n, generator=g)
    out = torch.empty(n, N, device=DEV)
    xm.native_moe_combine_multi(parts.to(DEV), w.to(DEV), sh.to(DEV) if shared else None, out, N, k, n,
                                shared_gate=gate.to(DEV) if gated else None)
    want = xo.combine(parts.numpy(), w.numpy(), sh.numpy() if shared else None, gate.numpy() if gated else None, N,
                      k, n)
    got = t2n(out)
    if gated:   # the gate's sigmoid uses each side's own expf: within an ulp or two of each other
        assert np.max(np.abs(got - want)) <= 1e-6 * np.max(np.abs(want))
    else:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # fused residual: x + combine, bit for bit the combine then add_inplace
    res = torch.randn(n, N, generator=g)
    out2 = res.clone().to(DEV)
    xm.moe_combine_residual(parts.to(DEV), w.to(DEV), out2, out2, N, k, n, shared=sh.to(DEV) if shared else None,
                            shared_gate=gate.to(DEV) if gated else None)
    want2 = (res.numpy() + got).astype(np.float32)
    assert np.array_equal(t2n(out2).view(np.uint32), want2.view(np.uint32))
