"""The persistent decode layers' hand-over contract, forced from the host:

* a bounded wait that expires: xs_moe_set_wait_bound(-1) makes every hand-over wait expire at once (the host's way
  of forcing the path a wait running out takes), every work-group still ends (the calls return and the device
  synchronises), the status word reports it and the checked contract (MoeLayer.check -> xs_moe_status_check) raises
  and clears it; with the default bound restored the next calls on the same workspace are bit for bit the reference
  again;
* the call tag near its wrap: the call counters preset so that the epoch reaches 2^32 - 2, 2^32 - 1 and 2^32 on a
  freshly zeroed workspace - the tag is never 0 (the value of a hand-over word never written), so every call equals a
  fresh workspace's output bit for bit."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def c2(xm):
    return xm.build_arena(128, 2048, 768, xm.Q4_K, xm.Q6_K, seed=2)


def inputs(T, H, E, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, H, device=DEV, generator=g)
    logits = torch.randn(T, E, device=DEV, generator=g)
    return x, res, logits


def reference_out(xm, arena, L, E, k, T, x, logits, res):
    out = torch.empty_like(res)
    layer = xm.MoeLayer(L, arena, E, k, T)
    layer(x, logits, res, out)
    layer.check()
    return out


@pytest.mark.parametrize("T", [1, 4, 16])
def test_expired_waits_are_reported(xm, c2, T):
    """Config 2 at 1 (the one-token kernel), 4 and 16 tokens (the persistent multi-token layer)."""
    arena, L = c2
    E, k = 128, 8
    x, res, logits = inputs(T, L.n_embd, E, 500 + T)
    want = reference_out(xm, arena, L, E, k, T, x, logits, res)
    layer = xm.MoeLayer(L, arena, E, k, T)
    out = torch.empty_like(res)
    print(f"[case] forced wait bound T={T}", flush=True)
    xm.lib().xs_moe_set_wait_bound(-1)
    try:
        for _ in range(4):
            layer(x, logits, res, out)
        torch.cuda.synchronize()   # every work-group ended
    finally:
        xm.lib().xs_moe_set_wait_bound(0)
    with pytest.raises(xm.XsError, match="bound|wait"):
        layer.check()
    assert layer.status() == 0   # cleared by the check
    for _ in range(2):
        layer(x, logits, res, out)
        layer.check()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32))


@pytest.mark.parametrize("T", [1, 4])
def test_call_tag_wrap(xm, c2, T):
    arena, L = c2
    E, k = 128, 8
    x, res, logits = inputs(T, L.n_embd, E, 600 + T)
    want = reference_out(xm, arena, L, E, k, T, x, logits, res)
    layer = xm.MoeLayer(L, arena, E, k, T)
    off = layer.ws_ptr - layer.ws.data_ptr()
    # counter 0 of the 16 (bytes 128 + 128 i of the workspace, 64-bit): the epoch is the counters' sum >> 20
    ctr = layer.ws[off + 128:off + 136].view(torch.int64)
    ctr.fill_((2 ** 32 - 2) << 20)
    torch.cuda.synchronize()
    out = torch.empty_like(res)
    for i in range(3):
        print(f"[case] tag wrap T={T} epoch=2^32-2+{i}", flush=True)
        out.fill_(float("nan"))
        layer(x, logits, res, out)
        layer.check()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), i


@pytest.mark.parametrize("cfg", ["config2", "config1"])
def test_help_path_bit_exact(xm, c2, cfg):
    """The path a waiter takes for a unit whose owner has not started (it computes the unit itself from the rows in
    HBM), forced for every unit from the host (xs_moe_set_wait_bound(-2)): the output equals the normal path's bit for
    bit, and the status stays clean."""
    if cfg == "config2":
        arena, L = c2
        E, k = 128, 8
    else:
        arena, L = xm.build_arena(8, 1024, 512, xm.Q8_0, xm.Q8_0, seed=0)
        E, k = 8, 2
    x, res, logits = inputs(1, L.n_embd, E, 800)
    want = reference_out(xm, arena, L, E, k, 1, x, logits, res)
    layer = xm.MoeLayer(L, arena, E, k, 1)
    out = torch.full_like(res, float("nan"))
    print(f"[case] help path forced, {cfg}", flush=True)
    xm.lib().xs_moe_set_wait_bound(-2)
    try:
        layer(x, logits, res, out)
        torch.cuda.synchronize()
    finally:
        xm.lib().xs_moe_set_wait_bound(0)
    layer.check()
    assert torch.equal(out.view(torch.int32), want.view(torch.int32)), float((out - want).abs().max())


@pytest.mark.parametrize("T", [1])
def test_layer_beside_other_work(xm, c2, T):
    """Half the compute units held by other work on another stream (xs_bench_occupy: one work-group a CU with all of
    its LDS, for 100 ms of the wall clock, then it ends) while the layer runs: the layer's grid cannot be resident at
    once, so its units must be taken in dependency order (gate/up before down before combine) for its waits to end.
    It must finish with a clean status (no wait ran into its 50 ms bound) and the reference's output bit for bit."""
    import time
    arena, L = c2
    E, k = 128, 8
    x, res, logits = inputs(T, L.n_embd, E, 700 + T)
    want = reference_out(xm, arena, L, E, k, T, x, logits, res)
    layer = xm.MoeLayer(L, arena, E, k, T)
    out = torch.full_like(res, float("nan"))
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.zeros(n_cu, dtype=torch.int32, device=DEV)
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    print(f"[case] layer T={T} beside {n_cu // 2} occupied CUs", flush=True)
    xm._check(xm.lib().xs_bench_occupy(n_cu // 2, 160 * 1024, 10_000_000, sink.data_ptr(), side.cuda_stream))
    time.sleep(0.005)   # the occupier's work-groups are placed
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    layer(x, logits, res, out)
    e1.record()
    torch.cuda.synchronize()
    print(f"[case] layer beside the occupier: {e0.elapsed_time(e1):.3f} ms", flush=True)
    layer.check()
    assert torch.equal(out.view(torch.int32), want.view(torch.int32))
