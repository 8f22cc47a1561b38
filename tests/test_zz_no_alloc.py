"""xs_moe_layer_decode_noalloc (the decode layer in the library's own device scratch, no workspace) against
xs_moe_layer_decode (the same layer in a caller's workspace), through the C ABI, bit for bit: consecutive calls whose
inputs shrink, a call of another layout in between (the one scratch serves every layout), and the refusals past the
scratch's limits (checked before anything is launched)."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def both(xm, arena, L, E, k, T, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    logits = torch.randn(T, E, device=DEV, generator=g)
    x = torch.randn(T, L.n_embd, device=DEV, generator=g).to(torch.bfloat16).float()
    res = torch.randn(T, L.n_embd, device=DEV, generator=g)
    want = torch.empty_like(res)
    got = torch.full_like(res, float("nan"))
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    print(f"[case] noalloc E={E} k={k} T={T} H={L.n_embd} F={L.n_ff} seed={seed}", flush=True)
    xm.MoeLayer(L, arena, E, k, T)(x, logits, res, want)
    xm.moe_layer_decode_noalloc(L, arena, E, k, x, logits, res, got, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (T, float((got - want).abs().max()))


def test_noalloc_matches_workspace_entry(xm):
    """Config 2 (Q4_K / Q6_K, 128 experts, top-8) at 16 tokens, then 4, then 1 (each smaller than the last); then
    config 1's layout (Q8_0, 8 experts, top-2, 4 tokens: other offsets in the same scratch); then config 2 again."""
    arena, L = xm.build_arena(128, 2048, 768, 12, 14, seed=2)
    for i, T in enumerate([16, 4, 1]):
        both(xm, arena, L, 128, 8, T, 900 + i)
    arena1, L1 = xm.build_arena(8, 1024, 512, 8, 8, seed=0)
    both(xm, arena1, L1, 8, 2, 4, 910)
    both(xm, arena, L, 128, 8, 2, 911)


def test_noalloc_refuses_past_its_scratch(xm):
    """Sizes past the fixed scratch fail with XS_EINVAL before any launch: too many entries for the array at config
    5's expert shape, and a hidden size past the scratch's largest layout.  The arena is NULL, so a regression of the
    size checks is still refused on the host (the layer's own arena check) and launches nothing."""
    L5 = xm.native_expert_layout(12, 12, 7168, 2048)
    x = torch.zeros(128, 7168, device=DEV)
    lg = torch.zeros(128, 256, device=DEV)
    out = torch.zeros_like(x)
    with pytest.raises(xm.XsError, match="past the fixed"):
        xm.moe_layer_decode_noalloc(L5, None, 256, 8, x, lg, x, out, blob_bytes=L5.bytes)
    L9 = xm.native_expert_layout(12, 12, 9216, 512)
    x9 = torch.zeros(1, 9216, device=DEV)
    with pytest.raises(xm.XsError, match="past the fixed scratch"):
        xm.moe_layer_decode_noalloc(L9, None, 8, 2, x9, lg[:1, :8], x9, x9.clone(), blob_bytes=L9.bytes)


def test_noalloc_status_word_without_caller_status(xm):
    """With status=None the call ORs its bits into the fixed scratch's own status word, which
    xs_moe_layer_decode_noalloc_status exposes: a token whose logits are all NaN (its router finds fewer than k
    experts: bit 2, no output) is reported by noalloc_status_check, which then clears the word; a good call after it
    leaves the word clear."""
    arena, L = xm.build_arena(8, 1024, 512, 8, 8, seed=0)
    xm.noalloc_status_check()   # clear whatever earlier calls left
    x = torch.randn(1, 1024, device=DEV)
    res = torch.randn(1, 1024, device=DEV)
    out = torch.zeros_like(res)
    bad = torch.full((1, 8), float("nan"), device=DEV)
    print("[case] noalloc NaN logits, status=None", flush=True)
    xm.moe_layer_decode_noalloc(L, arena, 8, 2, x, bad, res, out)
    with pytest.raises(xm.XsError):
        xm.noalloc_status_check()
    xm.noalloc_status_check()   # cleared by the check above
    good = torch.randn(1, 8, device=DEV)
    xm.moe_layer_decode_noalloc(L, arena, 8, 2, x, good, res, out)
    xm.noalloc_status_check()
    assert torch.isfinite(out).all()
