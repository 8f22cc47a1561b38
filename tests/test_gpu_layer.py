"""Whole MoE layers on the GPU (xs_moe_layer_decode / xs_moe_layer_prefill and the shared-expert composition) at the
BASELINE configs' shapes, against the CPU oracle on the same seeded inputs.

Bars: expert ids and the plan bit for bit (the router's and plan's own tests); layer output (residual + MoE) within
max|a - b| / max|ref| <= 1e-3 for the fp32-accumulate decode path, <= 2e-2 for the f16 MFMA prefill path."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def t2n(t):
    return t.detach().cpu().numpy()


def decode_case(xm, xo, arena, L, E, k, T, logits, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(T, L.n_embd, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, L.n_embd, device=DEV, generator=g)
    layer = xm.MoeLayer(L, arena, E, k, T)
    out = torch.empty_like(res)
    layer(x, logits, res, out)
    torch.cuda.synchronize()
    ids, _ = xo.router_top10(t2n(logits), k)
    used = sorted(set(ids.ravel().tolist()))
    blobs = t2n(arena[:E]) if E <= 32 else None
    by_expert = [blobs[e] if blobs is not None else (t2n(arena[e]) if e in used else np.zeros(16, np.uint8))
                 for e in range(E)]
    ol = xo.layout(L.gu_type, L.d_type, L.n_embd, L.n_ff)
    want = xo.moe_layer_decode(ol, by_expert, k, t2n(x), t2n(logits), t2n(res), n_threads=8)
    # the decode path is the oracle's canonical arithmetic end to end: the layer output bit for bit
    assert np.array_equal(t2n(out).view(np.uint32), want.view(np.uint32)), xo.rel_max(t2n(out), want)
    moe_rel = xo.rel_max(t2n(out) - t2n(res), want - t2n(res))
    return xo.rel_max(t2n(out), want), moe_rel


def test_config1_host_path_layer(xm, xo):
    """Config 1: hidden 1024, 8 experts, top-2, F 512, Q8_0, router weights N(0, 0.02), 4 tokens, seed 0."""
    H, E, k, F, T = 1024, 8, 2, 512, 4
    arena, L = xm.build_arena(E, H, F, 8, 8, seed=0, gen_device="cpu")
    g = torch.Generator().manual_seed(0)
    x = torch.randn(T, H, generator=g).to(DEV)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(DEV)
    logits = xm.router_logits_f32(x, wr)
    rel, moe_rel = decode_case(xm, xo, arena, L, E, k, T, logits, 0)
    assert rel <= 1e-3 and moe_rel <= 1e-3, (rel, moe_rel)


@pytest.fixture(scope="module")
def c2_arena(xm):
    return xm.build_arena(128, 2048, 768, 12, 14, seed=2)


@pytest.mark.parametrize("T", [1, 4, 16])
def test_config2_decode(xm, xo, c2_arena, T):
    """Config 2: Qwen3-30B-A3B-shaped, Q4_K gate/up, Q6_K down, uniform routing, batch 1 / 4 / 16."""
    arena, L = c2_arena
    g = torch.Generator(device=DEV).manual_seed(100 + T)
    logits = torch.randn(T, 128, device=DEV, generator=g)
    rel, moe_rel = decode_case(xm, xo, arena, L, 128, 8, T, logits, T)
    assert rel <= 1e-3 and moe_rel <= 1e-3, (rel, moe_rel)


def zipf_logits(T, E, seed):
    rng = np.random.default_rng(seed)
    pop = -1.2 * np.log(np.arange(1, E + 1))[rng.permutation(E)]
    return torch.from_numpy((pop[None, :] + rng.gumbel(size=(T, E))).astype(np.float32)).to(DEV)


def test_config3_verify_decode_path(xm, xo, c2_arena):
    """Config 3's 4-token spec-verify batch with Zipf-skewed logits, on the decode path."""
    arena, L = c2_arena
    rel, moe_rel = decode_case(xm, xo, arena, L, 128, 8, 4, zipf_logits(4, 128, 7), 4)
    assert rel <= 1e-3 and moe_rel <= 1e-3, (rel, moe_rel)


@pytest.mark.parametrize("T", [4, 2048])
def test_config3_prefill(xm, c2_arena, T):
    """Config 3: prefill 2048 tokens and the 4-token verify batch through the f16 MFMA path, against a plain PyTorch
    fp32 reference over the exactly dequantized weights (router ids shared: they are pinned bit for bit elsewhere)."""
    from test_gpu_experts import torch_reference_prefill
    arena, L = c2_arena
    E, k = 128, 8
    g = torch.Generator(device=DEV).manual_seed(T)
    x = torch.randn(T, L.n_embd, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, L.n_embd, device=DEV, generator=g)
    logits = zipf_logits(T, E, 3 + T)
    layer = xm.MoeLayer(L, arena, E, k, T, prefill=True)
    out = torch.empty_like(res)
    layer(x, logits, res, out)
    ids, w = xm.router_top10(logits, k)
    parts = torch_reference_prefill(xm, arena, L, x, ids, E)
    moe = (parts.reshape(T, k, -1) * w[:, :, None]).sum(1)
    rel = float(((out - res) - moe).abs().max() / moe.abs().max())
    assert rel <= 2e-2, rel


def test_prefill_outlier_activation(xm, c2_arena):
    """The f16 prompt path saturates activations and h at +-65504 (the f16 range), never to inf or NaN, and says so: a
    token with a 1e6 activation gets a finite output row (computed from the saturated values), the layer's status word
    carries bit 8 (MoeLayer.check -> xs_moe_status_check raises and clears it), every other token's row stays within
    2e-2 of the fp32 reference (the outlier touches only its own rows), and a call without the outlier leaves the word
    clear."""
    from test_gpu_experts import torch_reference_prefill
    arena, L = c2_arena
    E, k, T, bad = 128, 8, 64, 17
    g = torch.Generator(device=DEV).manual_seed(91)
    x = torch.randn(T, L.n_embd, device=DEV, generator=g).to(torch.bfloat16).float()
    clean = x.clone()
    x[bad, 5] = 1e6
    res = torch.randn(T, L.n_embd, device=DEV, generator=g)
    logits = zipf_logits(T, E, 91)
    out = torch.empty_like(res)
    layer = xm.MoeLayer(L, arena, E, k, T, prefill=True)
    layer(x, logits, res, out)
    assert layer.status() & 8
    with pytest.raises(xm.XsError, match="f16 range"):
        layer.check()
    assert layer.status() == 0
    layer(clean, logits, res, torch.empty_like(res))
    layer.check()
    assert bool(torch.isfinite(out).all())
    ids, w = xm.router_top10(logits, k)
    keep = torch.arange(T, device=DEV) != bad
    parts = torch_reference_prefill(xm, arena, L, x, ids, E)
    moe = (parts.reshape(T, k, -1) * w[:, :, None]).sum(1)
    rel = float(((out - res) - moe)[keep].abs().max() / moe[keep].abs().max())
    assert rel <= 2e-2, rel


def test_prefill_matches_decode_path(xm, xo, c2_arena):
    """The same 16 tokens through both paths: the f16 MFMA layer within 2e-2 of the fp32-accumulate one."""
    arena, L = c2_arena
    T = 16
    g = torch.Generator(device=DEV).manual_seed(77)
    x = torch.randn(T, L.n_embd, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.zeros(T, L.n_embd, device=DEV)
    logits = torch.randn(T, 128, device=DEV, generator=g)
    a = torch.empty_like(res)
    b = torch.empty_like(res)
    xm.MoeLayer(L, arena, 128, 8, T)(x, logits, res, a)
    xm.MoeLayer(L, arena, 128, 8, T, prefill=True)(x, logits, res, b)
    assert xo.rel_max(t2n(b), t2n(a)) <= 2e-2


@pytest.mark.parametrize("T", [1, 8])
def test_config4_iq4_xs(xm, xo, T):
    """Config 4's layer shape (hidden 4096, 128 experts, top-8, F 1536, IQ4_XS both sides), decode batch 1 and 8;
    16 distinct experts resident here (the oracle reads only the routed ones)."""
    E = 16
    arena, L = xm.build_arena(E, 4096, 1536, 23, 23, seed=4)
    g = torch.Generator(device=DEV).manual_seed(40 + T)
    logits = torch.randn(T, E, device=DEV, generator=g)
    rel, moe_rel = decode_case(xm, xo, arena, L, E, 8, T, logits, T)
    assert rel <= 1e-3 and moe_rel <= 1e-3, (rel, moe_rel)


@pytest.mark.parametrize("k", [8, 6])
def test_config5_shape_fused_decode(xm, xo, k):
    """The fused layer at config 5's expert shape (hidden 7168, F 2048, Q4_K both sides), one token: far more units
    than work-groups, so each work-group runs several gate/up units and a run of consecutive down units (its entry's
    h gathered once a run); bit for bit with the oracle (softmax routing over 16 resident experts)."""
    E = 16
    arena, L = xm.build_arena(E, 7168, 2048, 12, 12, seed=57)
    g = torch.Generator(device=DEV).manual_seed(58 + k)
    logits = torch.randn(1, E, device=DEV, generator=g)
    rel, moe_rel = decode_case(xm, xo, arena, L, E, k, 1, logits, 59)
    assert rel <= 1e-3 and moe_rel <= 1e-3, (rel, moe_rel)


def test_config5_deepseek_decode(xm, xo):
    """Config 5: hidden 7168, 256 routed Q4_K experts + 1 shared Q8_0, sigmoid + bias, 8 groups / top-4 / top-8, F
    2048, decode batch 1: the routed experts through the plan and the grouped kernels, the shared expert as one
    more group, the combine adding it once."""
    H, F, E, k, T = 7168, 2048, 256, 8, 1
    arena, L = xm.build_arena(E, H, F, 12, 12, seed=5)
    sh_arena, SL = xm.build_arena(1, H, F, 8, 8, seed=55)
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, H, device=DEV, generator=g)
    logits = torch.randn(T, E, device=DEV, generator=g)
    bias = torch.randn(E, device=DEV, generator=g) * 0.1
    ids, w = xm.router_grouped_sigmoid(logits, bias, 8, 4, k, 2.5)
    n = T * k
    plan = torch.zeros(xm.plan_words(n) + 2, dtype=torch.int32, device=DEV)
    skip = torch.zeros(1, dtype=torch.int32, device=DEV)
    xm.resident_plan(ids.reshape(-1), k, None, E, arena.data_ptr(), None, L.bytes, plan, n, skip, 1)
    o = xm.plan_offsets(n)
    xq = xm.quantize_q8_1_rows(x)
    scratch = torch.zeros(xm.native_expert_scratch_bytes(n, F), dtype=torch.uint8, device=DEV)
    parts = torch.zeros(n, H, device=DEV)
    ptr = plan[o["ptr"]:o["ptr"] + 2 * n].view(torch.int64)
    xm.native_expert_grouped(L, ptr, plan[4:], plan[0:1], plan[o["dst"]:], plan[o["tok"]:], min(n, E), n, xq, scratch,
                             parts)
    sh_ptr = torch.tensor([sh_arena.data_ptr()], dtype=torch.int64, device=DEV)
    one = torch.tensor([0, 1], dtype=torch.int32, device=DEV)
    zero = torch.zeros(1, dtype=torch.int32, device=DEV)
    sh_scratch = torch.zeros(xm.native_expert_scratch_bytes(1, F), dtype=torch.uint8, device=DEV)
    shared = torch.zeros(T, H, device=DEV)
    xm.native_expert_grouped(SL, sh_ptr, one, one[1:], zero, zero, 1, 1, xq, sh_scratch, shared)
    out = res.clone()
    xm.moe_combine_residual(parts, w, out, out, H, k, T, shared=shared)
    torch.cuda.synchronize()
    # the oracle: the same composition
    rids, rw = xo.router_grouped_sigmoid(t2n(logits), t2n(bias), 8, 4, k, 2.5)
    assert np.array_equal(t2n(ids), rids) and np.array_equal(t2n(w).view(np.uint32), rw.view(np.uint32))
    p = xo.decode_plan(rids, k)
    oxq = xo.quantize_q8_1_rows(t2n(x))
    ol = xo.layout(12, 12, H, F)
    blobs = [t2n(arena[e]) for e in p["experts"]]
    oparts = xo.native_expert_grouped(ol, blobs, p["start"], p["dst"], p["tok"], oxq, n)
    osh = xo.native_expert_grouped(xo.layout(8, 8, H, F), [t2n(sh_arena[0])], np.array([0, 1], np.int32),
                                   np.zeros(1, np.int32), np.zeros(1, np.int32), oxq, 1)
    want = (t2n(res) + xo.combine(oparts, rw, osh, None, H, k, T)).astype(np.float32)
    assert np.array_equal(t2n(out).view(np.uint32), want.view(np.uint32)), xo.rel_max(t2n(out), want)


def test_decode_workspace_reuse(xm, xo, c2_arena):
    """One workspace, sized for 16 tokens and zeroed once, serves calls of 16, 1, 4 and 16 tokens in a row (the
    persistent layer's counters return to zero after every call): each call bit for bit the oracle, status word 0."""
    arena, L = c2_arena
    layer = xm.MoeLayer(L, arena, 128, 8, 16)
    ol = xo.layout(L.gu_type, L.d_type, L.n_embd, L.n_ff)
    for i, T in enumerate([16, 1, 4, 16]):
        g = torch.Generator(device=DEV).manual_seed(300 + i)
        logits = torch.randn(T, 128, device=DEV, generator=g)
        x = torch.randn(T, L.n_embd, device=DEV, generator=g)
        res = torch.randn(T, L.n_embd, device=DEV, generator=g)
        out = torch.empty_like(res)
        layer(x, logits, res, out)
        torch.cuda.synchronize()
        assert layer.status() == 0
        ids, _ = xo.router_top10(t2n(logits), k=8)
        used = set(ids.ravel().tolist())
        by_expert = [t2n(arena[e]) if e in used else np.zeros(16, np.uint8) for e in range(128)]
        want = xo.moe_layer_decode(ol, by_expert, 8, t2n(x), t2n(logits), t2n(res), n_threads=8)
        assert np.array_equal(t2n(out).view(np.uint32), want.view(np.uint32)), (T, xo.rel_max(t2n(out), want))


def test_decode_graph_replays(xm, c2_arena):
    """The decode layer captured in a HIP graph: every replay (with eager work and waits between them) gives the
    eager call's bits."""
    arena, L = c2_arena
    T = 4
    g = torch.Generator(device=DEV).manual_seed(77)
    logits = torch.randn(T, 128, device=DEV, generator=g)
    x = torch.randn(T, L.n_embd, device=DEV, generator=g)
    res = torch.randn(T, L.n_embd, device=DEV, generator=g)
    layer = xm.MoeLayer(L, arena, 128, 8, T)
    eager = torch.empty_like(res)
    layer(x, logits, res, eager)
    torch.cuda.synchronize()
    out = torch.zeros_like(res)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        layer(x, logits, res, out, stream=s)   # warm-up on the capture stream
        s.synchronize()
        with torch.cuda.graph(graph, stream=s):
            layer(x, logits, res, out, stream=s)
    torch.cuda.synchronize()
    for r in range(4):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), eager.view(torch.int32)), r
    assert layer.status() == 0


@pytest.fixture(scope="module")
def c2_shared(xm):
    """A Q8_0 shared expert beside config 2's routed ones (hidden 2048, F 512), and a gate vector."""
    sh_arena, SL = xm.build_arena(1, 2048, 512, 8, 8, seed=22)
    g = torch.Generator(device=DEV).manual_seed(23)
    w_gate = torch.randn(2048, device=DEV, generator=g) * 0.02
    return sh_arena, SL, w_gate


def test_prefill_shared_graph_replays(xm, c2_arena, c2_shared):
    """The prompt layer with a (gated) shared expert captured in a HIP graph: the shared expert's work runs on a side
    stream forked from the caller's and joined before the combine, so the graph holds two branches.  Every replay
    (with eager work and waits between them) gives the eager call's bits."""
    arena, L = c2_arena
    sh_arena, SL, w_gate = c2_shared
    T = 64
    g = torch.Generator(device=DEV).manual_seed(78)
    logits = torch.randn(T, 128, device=DEV, generator=g)
    x = torch.randn(T, L.n_embd, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, L.n_embd, device=DEV, generator=g)
    layer = xm.MoeLayer(L, arena, 128, 8, T, prefill=True, shared=(SL, sh_arena, w_gate))
    eager = torch.empty_like(res)
    print("[case] prefill + shared expert, graph replays", flush=True)
    layer(x, logits, res, eager)
    torch.cuda.synchronize()
    out = torch.zeros_like(res)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        layer(x, logits, res, out, stream=s)   # warm-up on the capture stream
        s.synchronize()
        with torch.cuda.graph(graph, stream=s):
            layer(x, logits, res, out, stream=s)
    torch.cuda.synchronize()
    for r in range(4):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), eager.view(torch.int32)), r
    assert not torch.equal(eager, res)   # the layer added something


def test_shared_expert_decode(xm, xo, c2_shared):
    """xs_shared_expert_decode: every token through the one expert, rows bit for bit the oracle's (the same canonical
    rows as the routed experts); the gate logit within 1e-5 of a float64 dot (the router-logit GEMV's bound)."""
    sh_arena, SL, w_gate = c2_shared
    T = 5
    g = torch.Generator(device=DEV).manual_seed(24)
    x = torch.randn(T, 2048, device=DEV, generator=g).to(torch.bfloat16).float()
    shared, gate = xm.shared_expert_decode(SL, sh_arena[0], x, w_gate)
    torch.cuda.synchronize()
    want = xo.shared_expert(xo.layout(8, 8, 2048, 512), t2n(sh_arena[0]), t2n(x))
    assert np.array_equal(t2n(shared).view(np.uint32), want.view(np.uint32))
    ref = t2n(x).astype(np.float64) @ t2n(w_gate).astype(np.float64)
    assert np.max(np.abs(t2n(gate) - ref)) <= 1e-5 * np.max(np.abs(t2n(x)) @ np.abs(t2n(w_gate)))


@pytest.mark.parametrize("T", [1, 4, 16, 80])
@pytest.mark.parametrize("gated", [False, True])
def test_decode_shared_expert_layer(xm, xo, c2_arena, c2_shared, T, gated):
    """xs_moe_layer_decode_shared at config 2 + a Q8_0 shared expert (one persistent launch up to 16 tokens, the
    chained launches at 80): the routed combine, then the shared row once (times the sigmoid of its gate), then the
    residual.  Ungated: bit for bit the oracle.  Gated: the gate's sigmoid uses each side's own expf, so within an ulp
    or two (the gate logits given to the oracle are the device's, from xs_shared_expert_decode)."""
    arena, L = c2_arena
    sh_arena, SL, w_gate = c2_shared
    E, k = 128, 8
    g = torch.Generator(device=DEV).manual_seed(300 + T)
    logits = torch.randn(T, E, device=DEV, generator=g)
    x = torch.randn(T, 2048, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, 2048, device=DEV, generator=g)
    wg = w_gate if gated else None
    layer = xm.MoeLayer(L, arena, E, k, T, shared=(SL, sh_arena[0], wg))
    out = torch.empty_like(res)
    layer(x, logits, res, out)
    gate = xm.shared_expert_decode(SL, sh_arena[0], x, wg)[1] if gated else None
    torch.cuda.synchronize()
    assert layer.status() == 0
    want = xo.moe_layer_decode_shared(xo.layout(12, 14, 2048, 768), [t2n(arena[e]) for e in range(E)], k, t2n(x),
                                      t2n(logits), t2n(res), xo.layout(8, 8, 2048, 512), t2n(sh_arena[0]),
                                      None if gate is None else t2n(gate))
    got = t2n(out)
    if gated:
        assert np.max(np.abs(got - want)) <= 1e-6 * np.max(np.abs(want)), xo.rel_max(got, want)
    else:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), xo.rel_max(got, want)


def test_decode_one_token_probability_tie(xm, xo, c2_arena):
    """One token whose two best experts have logits one float ulp apart (the larger at the higher index) and
    probabilities that round to one float: the exact routing ranks the lower index first (router.cpp's tie rule), the
    logits' order the other one, so the one-token kernel's speculative fetch misses and is redone.  Bit for bit the
    oracle, and the ids in the exact order."""
    arena, L = c2_arena
    E, k = 128, 8
    rng = np.random.default_rng(5)
    lg = (np.full((1, E), -10.0) + rng.standard_normal((1, E)) * 0.1).astype(np.float32)
    lg[0, 12] = np.float32(0.25)
    lg[0, 37] = np.nextafter(np.float32(0.25), np.float32(1))
    rids, _ = xo.router_top10(lg, k)
    assert rids[0, 0] == 12 and rids[0, 1] == 37          # the tie the test is about
    logits = torch.from_numpy(lg).to(DEV)
    rel, moe_rel = decode_case(xm, xo, arena, L, E, k, 1, logits, 5)
    assert rel <= 1e-3 and moe_rel <= 1e-3, (rel, moe_rel)


def test_decode_one_token_nan_routing(xm, c2_arena):
    """One token with fewer than k numbers among its logits: the router leaves ranks unwritten, the layer writes no
    output and sets bit 2 (value 4) of the status word."""
    arena, L = c2_arena
    E, k = 128, 8
    logits = torch.full((1, E), float("nan"), device=DEV)
    logits[0, :5] = torch.arange(5, device=DEV, dtype=torch.float32)
    x = torch.randn(1, L.n_embd, device=DEV)
    res = torch.randn(1, L.n_embd, device=DEV)
    out = torch.full_like(res, 7.0)
    layer = xm.MoeLayer(L, arena, E, k, 1)
    layer(x, logits, res, out)
    torch.cuda.synchronize()
    assert layer.status() & 4
    assert torch.all(out == 7.0)
    with pytest.raises(xm.XsError, match="fewer than k experts"):   # the checked contract: raises, then clears
        layer.check()
    assert layer.status() == 0
    layer.check()


def test_prefill_f16_copy_in_the_permutation_launch(xm):
    """The prompt layer's f16 copy of x is built by the permutation launch's work-groups past its own, one 8-value
    chunk a thread, at most 2,048 work-groups and a stride beyond: at 4,096 tokens of hidden 7,168 (3.7 M chunks) the
    stride loop runs, every chunk is converted (the output within 2e-2 of the fp32 reference), and a saturating value
    in the last chunk of the last token - the stride's last visit - still sets status bit 8."""
    from test_gpu_experts import torch_reference_prefill
    E, k, T, H, F = 8, 2, 4096, 7168, 256
    arena, L = xm.build_arena(E, H, F, xm.Q8_0, xm.Q8_0, seed=21)
    g = torch.Generator(device=DEV).manual_seed(22)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, H, device=DEV, generator=g)
    logits = torch.randn(T, E, device=DEV, generator=g)
    out = torch.empty_like(res)
    layer = xm.MoeLayer(L, arena, E, k, T, prefill=True)
    print(f"[case] prefill T={T} H={H} (the conversion's stride loop)", flush=True)
    layer(x, logits, res, out)
    torch.cuda.synchronize()
    layer.check()
    ids, w = xm.router_top10(logits, k)
    moe = (torch_reference_prefill(xm, arena, L, x, ids, E).reshape(T, k, -1) * w[:, :, None]).sum(1)
    rel = float(((out - res) - moe).abs().max() / moe.abs().max())
    assert rel <= 2e-2, rel
    x2 = x.clone()
    x2[T - 1, H - 1] = 1e6
    layer(x2, logits, res, out)
    torch.cuda.synchronize()
    assert layer.status() & 8
    with pytest.raises(xm.XsError, match="f16 range"):
        layer.check()
