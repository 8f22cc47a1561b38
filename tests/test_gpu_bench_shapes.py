"""GPU parity at exactly the kernel instances bench.py times, against the CPU oracle (decode, bit for bit) and a plain
PyTorch fp32 reference (prefill, max|a - b| / max|ref| <= 2e-2, the f16 MFMA path's bar).

The fused decode kernel is instantiated per (gate/up type, down type, tokens class NE, mode, experts a routing lane
PER): these cases run the instances of config 4 at 128 experts (IQ4_XS, T = 1 and 8), config 5 at 256 experts with
and without its Q8_0 shared expert, the 2-3 token class (NE = 2) and the 17-64 token class (NE = 4 without the token
table).  The prefill cases cover Q6_K gate/up rows, the Q6_K down loop at n_ff = 1536, and config 5's prompt shapes
(hidden 7168, F 2048: the routed Q4_K layer and the Q8_0 shared expert) at the bench's 1024 tokens, and Q4_K at a
small Zipf-routed batch (mostly partial tiles, the head groups over several)."""
import numpy as np
import pytest
import torch

from test_gpu_experts import torch_reference_prefill

pytestmark = pytest.mark.gpu
DEV = "cuda"


def t2n(t):
    return t.detach().cpu().numpy()


def boosted_logits(T, E, k, s, seed):
    """The bench's routing (set_logits): i.i.d. N(0,1) logits plus 8 on the T*k experts s*T*k .. (mod E)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    lg = torch.randn(T, E, device=DEV, generator=g)
    lg[:, (torch.arange(T * k, device=DEV) + s * T * k) % E] += 8.0
    return lg


def used_blobs(arena, E, ids):
    used = set(np.asarray(ids).ravel().tolist())
    return [t2n(arena[e]) if e in used else np.zeros(16, np.uint8) for e in range(E)]


def decode_layer_case(xm, xo, arena, L, E, k, T, logits, seed, shared=None):
    """One layer call against the oracle's layer; shared = (SL, blob, w_gate or None).  Returns (got, want)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(T, L.n_embd, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, L.n_embd, device=DEV, generator=g)
    layer = xm.MoeLayer(L, arena, E, k, T, shared=shared)
    out = torch.empty_like(res)
    print(f"[case] decode E={E} k={k} T={T} H={L.n_embd} F={L.n_ff} types={L.gu_type}/{L.d_type} "
          f"shared={shared is not None}", flush=True)
    layer(x, logits, res, out)
    gate = None
    if shared is not None and shared[2] is not None:
        gate = xm.shared_expert_decode(shared[0], shared[1], x, shared[2])[1]
    torch.cuda.synchronize()
    assert layer.status() == 0
    ids, _ = xo.router_top10(t2n(logits), k)
    blobs = used_blobs(arena, E, ids)
    ol = xo.layout(L.gu_type, L.d_type, L.n_embd, L.n_ff)
    if shared is None:
        want = xo.moe_layer_decode(ol, blobs, k, t2n(x), t2n(logits), t2n(res), n_threads=8)
    else:
        SL = shared[0]
        want = xo.moe_layer_decode_shared(ol, blobs, k, t2n(x), t2n(logits), t2n(res),
                                          xo.layout(SL.gu_type, SL.d_type, SL.n_embd, SL.n_ff), t2n(shared[1]),
                                          None if gate is None else t2n(gate))
    return t2n(out), want


# ------------------------------------------------------------------------------------------------ config 4, 128 experts

@pytest.fixture(scope="module")
def c4_arena(xm):
    return xm.build_arena(128, 4096, 1536, 23, 23, seed=4)


@pytest.mark.parametrize("T", [1, 8])
def test_config4_decode_128_experts(xm, xo, c4_arena, T):
    """Config 4 as benched: IQ4_XS both sides, hidden 4096, F 1536, 128 experts, top-8, the bench's boosted disjoint
    routing (T=8: the pipelined 4-16 token instance; T=1: the one-token instance).  Bit for bit."""
    arena, L = c4_arena
    got, want = decode_layer_case(xm, xo, arena, L, 128, 8, T, boosted_logits(T, 128, 8, 1, 40 + T), T)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), xo.rel_max(got, want)


# ------------------------------------------------------------------------------------------------ config 5, 256 experts

@pytest.fixture(scope="module")
def c5_arena(xm):
    arena, L = xm.build_arena(256, 7168, 2048, 12, 12, seed=5)
    sh, SL = xm.build_arena(1, 7168, 2048, 8, 8, seed=55)
    g = torch.Generator(device=DEV).manual_seed(56)
    w_gate = torch.randn(7168, device=DEV, generator=g) * 0.02
    return arena, L, sh, SL, w_gate


@pytest.mark.parametrize("gated", [None, False, True])
def test_config5_decode_256_experts(xm, xo, c5_arena, gated):
    """Config 5's shapes as benched: 256 routed Q4_K experts (hidden 7168, F 2048, top-8; the one-token direct form
    with 4 routing experts a lane), alone (None) and through xs_moe_layer_decode_shared with the 7168 x 2048 Q8_0
    shared expert, ungated (bit for bit) and gated (within 1e-6 relative: each side's own expf in the sigmoid)."""
    arena, L, sh, SL, w_gate = c5_arena
    shared = None if gated is None else (SL, sh[0], w_gate if gated else None)
    got, want = decode_layer_case(xm, xo, arena, L, 256, 8, 1, boosted_logits(1, 256, 8, 3, 57), 58, shared)
    if gated:
        assert np.max(np.abs(got - want)) <= 1e-6 * np.max(np.abs(want)), xo.rel_max(got, want)
    else:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), xo.rel_max(got, want)


def test_config5_decode_256_experts_four_tokens(xm, xo, c5_arena):
    """256 experts at 4 tokens: the 4-16 token instance with 4 routing experts a lane."""
    arena, L, _, _, _ = c5_arena
    g = torch.Generator(device=DEV).manual_seed(59)
    logits = torch.randn(4, 256, device=DEV, generator=g)
    got, want = decode_layer_case(xm, xo, arena, L, 256, 8, 4, logits, 60)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), xo.rel_max(got, want)


# ------------------------------------------------------------------------------------------------ token classes

@pytest.fixture(scope="module")
def c2_arena(xm):
    return xm.build_arena(128, 2048, 768, 12, 14, seed=2)


@pytest.mark.parametrize("T,k", [(2, 8), (3, 8), (5, 8), (8, 8), (12, 8), (24, 8), (32, 8), (64, 4)])
def test_config2_decode_token_classes(xm, xo, c2_arena, T, k):
    """The fused layer's other token classes at config 2: 2-3 tokens (NE = 2); 5, 8 and 12 tokens (the pipelined
    instance with its token table sized to the call, 8 and 12 tokens, and at 5-8 tokens 8-row h-slabs, two work-groups
    a CU); 17-64 tokens (NE = 4 without the LDS token table: T = 24, 32 at top-8, T = 64 at top-4, 256 entries, the
    persistent layer's largest call)."""
    arena, L = c2_arena
    g = torch.Generator(device=DEV).manual_seed(500 + T)
    logits = torch.randn(T, 128, device=DEV, generator=g)
    got, want = decode_layer_case(xm, xo, arena, L, 128, k, T, logits, 600 + T)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), xo.rel_max(got, want)


# ------------------------------------------------------------------------------------------------ prefill

def zipf_ids(xm, T, E, k, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    p = 1.0 / torch.arange(1, E + 1, device=DEV, dtype=torch.float32) ** 1.2
    logits = torch.log(p)[None, :] - torch.log(-torch.log(torch.rand(T, E, device=DEV, generator=g)))
    return logits.contiguous()


def prefill_experts_case(xm, arena, L, E, k, T, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(T, L.n_embd, device=DEV, generator=g).to(torch.bfloat16).float()
    ids, _ = xm.router_top10(zipf_ids(xm, T, E, k, seed + 1), k)
    r = xm.prefill_route(ids.reshape(-1), k, E, cache_base=arena.data_ptr(), blob=L.bytes, with_ptr=True)
    n = T * k
    scratch = torch.zeros(xm.moe_prefill_scratch_bytes(T, n, L.n_embd, L.n_ff), dtype=torch.uint8, device=DEV)
    parts = torch.zeros(n, L.n_embd, device=DEV)
    print(f"[case] prefill experts E={E} k={k} T={T} H={L.n_embd} F={L.n_ff} types={L.gu_type}/{L.d_type}",
          flush=True)
    xm.moe_prefill_experts(L, x, r["src"], r["entry"], r["bounds"], r["n_groups"], r["grp_ptr"], min(n, E), n,
                           scratch, parts)
    torch.cuda.synchronize()
    want = torch_reference_prefill(xm, arena, L, x, ids, E)
    return float((parts - want).abs().max() / want.abs().max())


@pytest.mark.parametrize("gu,dt,H,F", [(14, 14, 2048, 768), (12, 14, 2048, 1536), (14, 14, 4096, 1536)])
def test_prefill_q6_k_forms(xm, gu, dt, H, F):
    """Q6_K gate/up rows, and the Q6_K down loop at a run-time n_ff (1536, not the unrolled 768)."""
    E, k, T = 16, 8, 256
    arena, L = xm.build_arena(E, H, F, gu, dt, seed=gu + F)
    rel = prefill_experts_case(xm, arena, L, E, k, T, 71)
    assert rel <= 2e-2, rel


@pytest.mark.parametrize("T", [256, 512])
def test_prefill_q4_k_zipf_small_batch(xm, T):
    """Q4_K gate/up and down at a small prompt batch with Zipf routing: groups from a few rows to T rows (several
    128-row tiles), most of them partial tiles."""
    E, k = 64, 8
    arena, L = xm.build_arena(E, 2048, 768, 12, 12, seed=T)
    rel = prefill_experts_case(xm, arena, L, E, k, T, 91)
    assert rel <= 2e-2, rel


def test_config5_prefill_routed_layer(xm, c5_arena):
    """Config 5's prompt layer as benched: 1024 tokens through the 256 routed Q4_K experts (hidden 7168, F 2048,
    softmax top-8) with the f16 MFMA GEMMs; the layer output minus the residual against the fp32 reference's
    weighted parts."""
    arena, L, _, _, _ = c5_arena
    E, k, T = 256, 8, 1024
    g = torch.Generator(device=DEV).manual_seed(81)
    x = torch.randn(T, L.n_embd, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, L.n_embd, device=DEV, generator=g)
    logits = torch.randn(T, E, device=DEV, generator=g)
    layer = xm.MoeLayer(L, arena, E, k, T, prefill=True)
    out = torch.empty_like(res)
    print(f"[case] config 5 prefill layer T={T}", flush=True)
    layer(x, logits, res, out)
    ids, w = xm.router_top10(logits, k)
    parts = torch_reference_prefill(xm, arena, L, x, ids, E)
    moe = (parts.reshape(T, k, -1) * w[:, :, None]).sum(1)
    rel = float(((out - res) - moe).abs().max() / moe.abs().max())
    assert rel <= 2e-2, rel


def test_config5_prefill_shared_expert(xm, c5_arena):
    """Config 5's Q8_0 shared expert (7168 x 2048) over 1024 tokens as the bench runs it: one group of every token
    through xs_moe_prefill_experts."""
    _, _, sh, SL, _ = c5_arena
    T, H = 1024, 7168
    g = torch.Generator(device=DEV).manual_seed(82)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16).float()
    i32 = dict(dtype=torch.int32, device=DEV)
    src = torch.arange(T, **i32)
    bounds = torch.tensor([0, T], **i32)
    ng = torch.ones(1, **i32)
    ptr = torch.tensor([sh[0].data_ptr()], dtype=torch.int64, device=DEV)
    scratch = torch.zeros(xm.moe_prefill_scratch_bytes(T, T, H, SL.n_ff), dtype=torch.uint8, device=DEV)
    out = torch.zeros(T, H, device=DEV)
    print(f"[case] config 5 shared expert prefill T={T}", flush=True)
    xm.moe_prefill_experts(SL, x, src, src, bounds, ng, ptr, 1, T, scratch, out)
    ids = torch.zeros(T, 1, **i32)
    want = torch_reference_prefill(xm, sh, SL, x, ids, 1)
    rel = float((out - want).abs().max() / want.abs().max())
    assert rel <= 2e-2, rel


# ------------------------------------------------------------------------------------------------ config 5 in one call

def oracle_grouped_layer(xo, arena, L, E, k, x, logits, bias, res, shared=None, gate=None, n_group=8, topk_group=4,
                         scale=2.5):
    """The oracle's composition of a decode layer routed by the grouped sigmoid router: router, plan, grouped experts,
    the shared expert as one group of every token, the combine (+ the shared row, times sigmoid(gate) if given),
    the residual."""
    T, H = x.shape
    rids, rw = xo.router_grouped_sigmoid(logits, bias, n_group, topk_group, k, scale)
    p = xo.decode_plan(rids, k)
    oxq = xo.quantize_q8_1_rows(x)
    blobs = [t2n(arena[e]) for e in p["experts"]]
    oparts = xo.native_expert_grouped(xo.layout(L.gu_type, L.d_type, H, L.n_ff), blobs, p["start"], p["dst"], p["tok"],
                                      oxq, T * k)
    osh = None
    if shared is not None:
        SL, sblob = shared
        idx = np.arange(T, dtype=np.int32)
        osh = xo.native_expert_grouped(xo.layout(SL.gu_type, SL.d_type, H, SL.n_ff), [t2n(sblob)],
                                       np.array([0, T], np.int32), idx, idx, oxq, T)
    return rids, (res + xo.combine(oparts, rw, osh, gate, H, k, T)).astype(np.float32)


@pytest.mark.parametrize("T,gated", [(1, False), (1, True), (4, False)])
def test_config5_decode_one_call(xm, xo, c5_arena, T, gated):
    """Config 5's whole decode layer as one call (xs_moe_layer_decode_ex): the group-limited sigmoid router with bias
    (8 groups, top-4, k 8, routed scale 2.5) over 256 Q4_K experts plus the Q8_0 shared expert.  Ungated: bit for bit
    the oracle's composition; gated: within 1e-6 relative (each side's own expf in the sigmoid)."""
    arena, L, sh, SL, w_gate = c5_arena
    E, k, H = 256, 8, 7168
    g = torch.Generator(device=DEV).manual_seed(70 + T)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, H, device=DEV, generator=g)
    logits = torch.randn(T, E, device=DEV, generator=g)
    bias = torch.randn(E, device=DEV, generator=g) * 0.1
    router = xm.grouped_sigmoid_router(bias, 8, 4, 2.5)
    wg = w_gate if gated else None
    layer = xm.MoeLayer(L, arena, E, k, T, shared=(SL, sh[0], wg), router=router)
    out = torch.empty_like(res)
    print(f"[case] config 5 decode one call T={T} gated={gated}", flush=True)
    layer(x, logits, res, out)
    gate = xm.shared_expert_decode(SL, sh[0], x, wg)[1] if gated else None
    torch.cuda.synchronize()
    layer.check()
    _, want = oracle_grouped_layer(xo, arena, L, E, k, t2n(x), t2n(logits), t2n(bias), t2n(res), (SL, sh[0]),
                                   None if gate is None else t2n(gate))
    got = t2n(out)
    if gated:
        assert np.max(np.abs(got - want)) <= 1e-6 * np.max(np.abs(want)), xo.rel_max(got, want)
    else:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), xo.rel_max(got, want)


def test_grouped_router_chained_decode(xm, xo, c2_arena):
    """The grouped sigmoid router on config 2's experts (128 = 8 groups of 16, top-4 groups, k 8) at 40 tokens: 320
    entries, past the persistent kernel, so the chained path plans the given ids (resident plan) and runs the grouped
    kernels and the combine.  Bit for bit the oracle's composition, no shared expert."""
    arena, L = c2_arena
    E, k, T, H = 128, 8, 40, 2048
    g = torch.Generator(device=DEV).manual_seed(77)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, H, device=DEV, generator=g)
    logits = torch.randn(T, E, device=DEV, generator=g)
    bias = torch.randn(E, device=DEV, generator=g) * 0.1
    layer = xm.MoeLayer(L, arena, E, k, T, router=xm.grouped_sigmoid_router(bias, 8, 4, 1.0))
    out = torch.empty_like(res)
    layer(x, logits, res, out)
    torch.cuda.synchronize()
    layer.check()
    _, want = oracle_grouped_layer(xo, arena, L, E, k, t2n(x), t2n(logits), t2n(bias), t2n(res), scale=1.0)
    got = t2n(out)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), xo.rel_max(got, want)


@pytest.mark.parametrize("gated", [False, True])
def test_config5_prefill_one_call(xm, c5_arena, gated):
    """Config 5's prompt layer as one call (xs_moe_layer_prefill_ex): 1024 tokens, the grouped sigmoid router, the 256
    routed Q4_K experts and the Q8_0 shared expert through the f16 MFMA GEMMs, the shared row added by the combine
    (times sigmoid(w_gate . x) when gated).  Against the fp32 reference: max|a - b| / max|ref| <= 2e-2."""
    arena, L, sh, SL, w_gate = c5_arena
    E, k, T, H = 256, 8, 1024, 7168
    g = torch.Generator(device=DEV).manual_seed(90)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, H, device=DEV, generator=g)
    logits = torch.randn(T, E, device=DEV, generator=g)
    bias = torch.randn(E, device=DEV, generator=g) * 0.1
    wg = w_gate if gated else None
    layer = xm.MoeLayer(L, arena, E, k, T, prefill=True, shared=(SL, sh[0], wg),
                        router=xm.grouped_sigmoid_router(bias, 8, 4, 2.5))
    out = torch.empty_like(res)
    print(f"[case] config 5 prefill one call gated={gated}", flush=True)
    layer(x, logits, res, out)
    ids, w = xm.router_grouped_sigmoid(logits, bias, 8, 4, k, 2.5)
    parts = torch_reference_prefill(xm, arena, L, x, ids, E)
    shared = torch_reference_prefill(xm, sh, SL, x, torch.zeros(T, 1, dtype=torch.int32, device=DEV), 1)
    if gated:
        shared = shared * torch.sigmoid(x @ w_gate)[:, None]
    moe = (parts.reshape(T, k, -1) * w[:, :, None]).sum(1) + shared
    rel = float(((out - res) - moe).abs().max() / moe.abs().max())
    assert rel <= 2e-2, rel
