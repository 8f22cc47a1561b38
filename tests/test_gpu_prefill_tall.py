"""The prompt layer's tall-tile split (xs_moe_set_prefill_tall): every whole 256-row tile of an expert's rows runs on
the tall-tile GEMMs (8 waves over 256 rows x 256 or 128 weight rows, the weights dequantized once a step into LDS) and
the other rows on the 128-row GEMMs on a side stream.  Both kinds of tile feed each output value the same f16
fragments in the same K order into the same MFMA instruction, so the layer's output with the split - side by side or
its chains one after the other - equals the output without it bit for bit; it is also within the f16 path's 2e-2 of
the fp32 torch reference over exactly dequantized weights.

Cases: config 3 (Q4_K gate/up, Q6_K down, 2048 tokens, Zipf routing: 33 tall tiles beside 128 remainders); both
pairs of the tall GEMMs' formats (Q4_K / Q6_K either way round) at group sizes around the tile edge (0, 1, 255, 256,
257, 511, 512 and 768 rows); and the split under graph capture (its side stream becomes a branch of the graph),
replayed three times with eager work between the replays."""
import numpy as np
import pytest
import torch

from test_gpu_experts import torch_reference_prefill
from test_gpu_layer import zipf_logits

pytestmark = pytest.mark.gpu
DEV = "cuda"


def run_layer(xm, layer, x, logits, res, tall):
    """tall: 0 off, 1 the split side by side (the default), 2 the split's chains one after the other."""
    out = torch.full_like(res, float("nan"))
    xm.lib().xs_moe_set_prefill_tall(int(tall))
    try:
        layer(x, logits, res, out)
        torch.cuda.synchronize()
    finally:
        xm.lib().xs_moe_set_prefill_tall(1)
    return out


def reference_rel(xm, arena, L, E, k, x, logits, res, out):
    ids, w = xm.router_top10(logits, k)
    parts = torch_reference_prefill(xm, arena, L, x, ids, E)
    moe = (parts.reshape(x.shape[0], k, -1) * w[:, :, None]).sum(1)
    return float(((out - res) - moe).abs().max() / moe.abs().max())


def inputs(T, H, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, H, device=DEV, generator=g)
    return x, res


def edge_logits(counts, T, E, seed):
    """Top-2 logits giving expert e exactly counts[e] of the 2 T routed rows (every count <= T): the ids sorted by
    expert, token t takes ids t and t + T (distinct, as no expert spans more than T places)."""
    assert sum(counts) == 2 * T and max(counts) <= T
    ids = np.repeat(np.arange(E), counts)
    g = torch.Generator(device=DEV).manual_seed(seed)
    logits = 0.1 * torch.randn(T, E, device=DEV, generator=g)
    t = torch.arange(T, device=DEV)
    logits[t, torch.from_numpy(ids[:T]).to(DEV)] = 10.0
    logits[t, torch.from_numpy(ids[T:]).to(DEV)] = 9.0
    return logits


@pytest.fixture(scope="module")
def c3(xm):
    return xm.build_arena(128, 2048, 768, xm.Q4_K, xm.Q6_K, seed=2)


def test_config3_split_equals_unsplit(xm, c3):
    arena, L = c3
    E, k, T = 128, 8, 2048
    x, res = inputs(T, L.n_embd, 33)
    logits = zipf_logits(T, E, 3)
    layer = xm.MoeLayer(L, arena, E, k, T, prefill=True)
    print("[case] config3 T=2048 tall on/off/serial", flush=True)
    off = run_layer(xm, layer, x, logits, res, 0)
    on = run_layer(xm, layer, x, logits, res, 1)
    serial = run_layer(xm, layer, x, logits, res, 2)
    assert torch.equal(on.view(torch.int32), off.view(torch.int32)), float((on - off).abs().max())
    assert torch.equal(serial.view(torch.int32), off.view(torch.int32)), float((serial - off).abs().max())
    rel = reference_rel(xm, arena, L, E, k, x, logits, res, on)
    assert rel <= 2e-2, rel


@pytest.mark.parametrize("gu,dt", [("Q4_K", "Q6_K"), ("Q6_K", "Q4_K")])
def test_tile_edges(xm, gu, dt):
    E, k, H, F = 8, 2, 1024, 512
    counts = [256, 257, 255, 511, 512, 1, 0, 768]
    T = sum(counts) // 2
    arena, L = xm.build_arena(E, H, F, getattr(xm, gu), getattr(xm, dt), seed=5)
    x, res = inputs(T, H, 44)
    logits = edge_logits(counts, T, E, 45)
    ids, _ = xm.router_top10(logits, k)
    assert np.array_equal(np.bincount(ids.reshape(-1).cpu().numpy(), minlength=E), counts)
    layer = xm.MoeLayer(L, arena, E, k, T, prefill=True)
    print(f"[case] tile edges {gu}/{dt} T={T}", flush=True)
    off = run_layer(xm, layer, x, logits, res, 0)
    on = run_layer(xm, layer, x, logits, res, 1)
    assert torch.equal(on.view(torch.int32), off.view(torch.int32)), float((on - off).abs().max())
    rel = reference_rel(xm, arena, L, E, k, x, logits, res, on)
    assert rel <= 2e-2, rel


def test_split_under_graph_capture(xm, c3):
    arena, L = c3
    E, k, T = 128, 8, 1024
    x, res = inputs(T, L.n_embd, 55)
    logits = zipf_logits(T, E, 56)
    layer = xm.MoeLayer(L, arena, E, k, T, prefill=True)
    want = run_layer(xm, layer, x, logits, res, 1)
    out = torch.full_like(res, float("nan"))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer(x, logits, res, out)   # warm-up on the capture stream
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer(x, logits, res, out)
    torch.cuda.synchronize()
    for i in range(3):
        print(f"[case] graph replay {i}", flush=True)
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), i
        other = run_layer(xm, layer, x, logits, res, 0)   # eager work between the replays
        assert torch.equal(other.view(torch.int32), want.view(torch.int32)), i
