"""Mixed layers - gate rows of one type, up rows of another, each read as a gate/up matrix of its own type (the
reference's native_expert_supported / native_expert_layout with up_type, src/kernels/xe/iq_kernels.cpp:2003-2005,
2021-2036) - against the CPU oracle, whose restatement reads each row by its own type.

The grouped decode product (xs_native_expert_grouped: the gate rows and the up rows as two launches of their own
types) and the decode layer at 1 and 4 tokens (the chained path: the one-token and persistent kernels take one
gate/up type and refuse a mixed layer) bit for bit; the prompt layer (its generic f16 GEMM path, which dequantizes each
row by its own type) within the f16 path's 2e-2 of a PyTorch fp32 reference over the exactly dequantized weights."""
import numpy as np
import pytest
import torch

from test_gpu_bench_shapes import used_blobs
from test_gpu_experts import group_case, torch_reference_prefill

pytestmark = pytest.mark.gpu
DEV = "cuda"
MIXED = [(12, 14, 14, 2048, 768), (14, 8, 12, 1024, 512), (8, 23, 8, 1024, 256)]   # gate, up, down, H, F


def t2n(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("gu,up,dt,H,F", MIXED)
def test_native_expert_grouped_mixed(xm, xo, gu, up, dt, H, F):
    rng = np.random.default_rng(H + F + 7 * up)
    E = 4
    arena, L = xm.build_arena(E, H, F, gu, dt, seed=gu * 13 + up, up_type=up)
    assert (L.gu_type, L.up_type) == (gu, up)
    blobs = t2n(arena)
    sizes = [2, 5, 1, 3]
    experts = [1, 0, 3, 1]
    T = 5
    start, tok, dst = group_case(len(sizes), sizes, T, rng)
    n = int(start[-1])
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).float()
    xq = xm.quantize_q8_1_rows(x.to(DEV))
    grp_ptr = torch.tensor([arena[e].data_ptr() for e in experts], dtype=torch.int64, device=DEV)
    scratch = torch.zeros(xm.native_expert_scratch_bytes(n, F), dtype=torch.uint8, device=DEV)
    out = torch.zeros(n, H, device=DEV)
    print(f"[case] grouped mixed {gu}/{up}/{dt} H={H} F={F}", flush=True)
    xm.native_expert_grouped(L, grp_ptr, torch.from_numpy(start).to(DEV),
                             torch.tensor([len(sizes)], dtype=torch.int32, device=DEV), torch.from_numpy(dst).to(DEV),
                             torch.from_numpy(tok).to(DEV), len(sizes), n, xq, scratch, out)
    torch.cuda.synchronize()
    ol = xo.layout(gu, dt, H, F, up)
    want, gate, upr, hq = xo.native_expert_grouped(ol, [blobs[e] for e in experts], start, dst, tok, t2n(xq), n,
                                                   want_inner=True)
    fa = (n * F * 4 + 255) & ~255
    assert np.array_equal(t2n(scratch[:n * F * 4].view(torch.float32)).reshape(n, F).view(np.uint32),
                          gate.view(np.uint32))
    assert np.array_equal(t2n(scratch[fa:fa + n * F * 4].view(torch.float32)).reshape(n, F).view(np.uint32),
                          upr.view(np.uint32))
    assert np.array_equal(t2n(scratch[3 * fa:3 * fa + n * (F // 32) * 36]), hq)
    assert np.array_equal(t2n(out).view(np.uint32), want.view(np.uint32))
    # the up rows read by their own type: the same blobs read as a same-type layer give other up rows
    same = xo.layout(gu, dt, H, F)
    if same.down_off != ol.down_off:
        assert ol.up_row != same.gu_row


@pytest.mark.parametrize("T", [1, 4])
@pytest.mark.parametrize("gu,up,dt,H,F", MIXED[:2])
def test_decode_layer_mixed(xm, xo, gu, up, dt, H, F, T):
    E, k = 16, 4
    arena, L = xm.build_arena(E, H, F, gu, dt, seed=3 * T + up, up_type=up)
    g = torch.Generator(device=DEV).manual_seed(40 + T)
    logits = torch.randn(T, E, device=DEV, generator=g)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, H, device=DEV, generator=g)
    out = torch.empty_like(res)
    layer = xm.MoeLayer(L, arena, E, k, T)
    print(f"[case] decode mixed {gu}/{up}/{dt} T={T}", flush=True)
    layer(x, logits, res, out)
    torch.cuda.synchronize()
    assert layer.status() == 0
    ids, _ = xo.router_top10(t2n(logits), k)
    want = xo.moe_layer_decode(xo.layout(gu, dt, H, F, up), used_blobs(arena, E, ids), k, t2n(x), t2n(logits),
                               t2n(res), n_threads=8)
    assert np.array_equal(t2n(out).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("gu,up,dt,H,F", MIXED[:2])
def test_prefill_layer_mixed(xm, gu, up, dt, H, F):
    E, k, T = 8, 2, 96
    arena, L = xm.build_arena(E, H, F, gu, dt, seed=5 + up, up_type=up)
    g = torch.Generator(device=DEV).manual_seed(77)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, H, device=DEV, generator=g)
    logits = torch.randn(T, E, device=DEV, generator=g)
    out = torch.full_like(res, float("nan"))
    layer = xm.MoeLayer(L, arena, E, k, T, prefill=True)
    print(f"[case] prefill mixed {gu}/{up}/{dt} T={T}", flush=True)
    layer(x, logits, res, out)
    torch.cuda.synchronize()
    layer.check()
    ids, w = xm.router_top10(logits, k)
    parts = torch_reference_prefill(xm, arena, L, x, ids, E)
    moe = (parts.reshape(T, k, -1) * w[:, :, None]).sum(1)
    rel = float(((out - res) - moe).abs().max() / moe.abs().max())
    assert rel <= 2e-2, rel


@pytest.mark.parametrize("T", [1, 3])
def test_decode_mixed_shared_and_noalloc(xm, xo, T):
    """A mixed routed layer with a mixed shared expert (its own one-group chain: the persistent one-expert layer takes
    one gate/up type), against the oracle bit for bit; and the allocation-free entry point on the mixed layer equals
    the workspace entry point bit for bit."""
    E, k, H, F = 16, 4, 1024, 512
    arena, L = xm.build_arena(E, H, F, 14, 12, seed=11 + T, up_type=8)
    sarena, SL = xm.build_arena(1, H, 256, 12, 8, seed=12 + T, up_type=14)
    g = torch.Generator(device=DEV).manual_seed(60 + T)
    logits = torch.randn(T, E, device=DEV, generator=g)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, H, device=DEV, generator=g)
    out = torch.empty_like(res)
    print(f"[case] decode mixed + shared T={T}", flush=True)
    layer = xm.MoeLayer(L, arena, E, k, T, shared=(SL, sarena[0], None))
    layer(x, logits, res, out)
    torch.cuda.synchronize()
    assert layer.status() == 0
    ids, _ = xo.router_top10(t2n(logits), k)
    want = xo.moe_layer_decode_shared(xo.layout(14, 12, H, F, 8), used_blobs(arena, E, ids), k, t2n(x), t2n(logits),
                                      t2n(res), xo.layout(12, 8, H, 256, 14), t2n(sarena[0]), None)
    assert np.array_equal(t2n(out).view(np.uint32), want.view(np.uint32))
    got = torch.full_like(res, float("nan"))
    ref = torch.empty_like(res)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    xm.MoeLayer(L, arena, E, k, T)(x, logits, res, ref)
    xm.moe_layer_decode_noalloc(L, arena, E, k, x, logits, res, got, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    assert torch.equal(got.view(torch.int32), ref.view(torch.int32))
