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
