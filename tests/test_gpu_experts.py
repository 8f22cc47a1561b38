"""GPU parity of the grouped expert products against the CPU oracle.

Decode / verify (xs_native_expert_grouped, the reference's native_expert_grouped contract: q8_1 activations, exact
integer block sums): gate / up within 1e-5 of each row's magnitude, the q8_1 of SwiGLU(gate, up) bit for bit for the
same gate / up, outputs within max|a - b| / max|ref| <= 1e-3 (fp32 accumulate).
Prefill (xs_moe_prefill_experts, f16 MFMA): against a plain PyTorch fp32 reference over the dequantized weights
(xs_iq_dequant_f32 is bit-exact with the reference's dequantizer), max-relative <= 2e-2."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def t2n(t):
    return t.detach().cpu().numpy()


PAIRS = [(8, 8, 1024, 512), (12, 14, 2048, 768), (23, 23, 4096, 1536), (12, 12, 7168, 2048), (8, 8, 7168, 2048),
         (14, 14, 2048, 512), (23, 23, 1024, 256)]


def group_case(n_groups, sizes, n_tok, rng):
    start = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    n = int(start[-1])
    tok = rng.integers(0, n_tok, n).astype(np.int32)
    dst = rng.permutation(n).astype(np.int32)
    return start, tok, dst


@pytest.mark.parametrize("gu,dt,H,F", PAIRS)
def test_native_expert_grouped(xm, xo, gu, dt, H, F):
    rng = np.random.default_rng(H * 7 + F + gu)
    E = 4
    arena, L = xm.build_arena(E, H, F, gu, dt, seed=gu * 31 + H)
    blobs = t2n(arena)
    sizes = [1, 3, 7, 2, 5]                      # groups of 1..7 entries, the last two on the same expert
    experts = [0, 2, 1, 3, 3]
    T = 6
    start, tok, dst = group_case(len(sizes), sizes, T, rng)
    n = int(start[-1])
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).float()
    xq = xm.quantize_q8_1_rows(x.to(DEV))
    grp_ptr = torch.tensor([arena[e].data_ptr() for e in experts], dtype=torch.int64, device=DEV)
    d_start = torch.from_numpy(start).to(DEV)
    ng = torch.tensor([len(sizes)], dtype=torch.int32, device=DEV)
    scratch = torch.zeros(xm.native_expert_scratch_bytes(n, F), dtype=torch.uint8, device=DEV)
    out = torch.zeros(n, H, device=DEV)
    xm.native_expert_grouped(L, grp_ptr, d_start, ng, torch.from_numpy(dst).to(DEV), torch.from_numpy(tok).to(DEV),
                             len(sizes), n, xq, scratch, out)
    torch.cuda.synchronize()
    ol = xo.layout(gu, dt, H, F)
    want, gate, up, hq = xo.native_expert_grouped(ol, [blobs[e] for e in experts], start, dst, tok, t2n(xq), n,
                                                  want_inner=True)
    fa = (n * F * 4 + 255) & ~255
    sg = t2n(scratch[:n * F * 4].view(torch.float32)).reshape(n, F)
    su = t2n(scratch[fa:fa + n * F * 4].view(torch.float32)).reshape(n, F)
    # the canonical row order is the oracle's: gate / up rows, their SwiGLU q8_1 and the down rows bit for bit
    assert np.array_equal(sg.view(np.uint32), gate.view(np.uint32))
    assert np.array_equal(su.view(np.uint32), up.view(np.uint32))
    hb = t2n(scratch[3 * fa:3 * fa + n * (F // 32) * 36])
    assert np.array_equal(hb, hq)
    assert np.array_equal(t2n(out).view(np.uint32), want.view(np.uint32))
    # and within the reference's float criterion of the exact dot of the dequantized operands
    q, d, _ = xo.q8_1_values(t2n(xq))
    a = (q.astype(np.float64) * d[:, None]).reshape(T, H)
    for e in range(n):
        scale = np.abs(a[tok[e]]).sum() * 0.02 * 4
        assert np.max(np.abs(sg[e] - gate[e])) <= 1e-5 * scale
    status = torch.from_numpy(np.zeros(1, np.int32))
    st = scratch[xm.native_expert_scratch_bytes(n, F) - 256:][:4].view(torch.int32)
    assert int(st[0]) == 0


def test_grid_groups_same_bits(xm):
    """grid_groups rows of work-groups striding over the groups give the same bits (reference iq_kernels.hpp:85-89)."""
    H, F = 2048, 768
    arena, L = xm.build_arena(6, H, F, 12, 14, seed=5)
    rng = np.random.default_rng(2)
    start, tok, dst = group_case(6, [1, 2, 1, 1, 3, 1], 4, rng)
    n = int(start[-1])
    x = torch.randn(4, H, device=DEV)
    xq = xm.quantize_q8_1_rows(x)
    grp_ptr = torch.tensor([arena[e].data_ptr() for e in range(6)], dtype=torch.int64, device=DEV)
    args = [torch.from_numpy(a).to(DEV) for a in (start, dst, tok)]
    ng = torch.tensor([6], dtype=torch.int32, device=DEV)
    outs = []
    for gg in (0, 1, 4):
        scratch = torch.zeros(xm.native_expert_scratch_bytes(n, F), dtype=torch.uint8, device=DEV)
        out = torch.zeros(n, H, device=DEV)
        xm.native_expert_grouped(L, grp_ptr, args[0], ng, args[1], args[2], 6, n, xq, scratch, out, grid_groups=gg)
        outs.append(out)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


def test_misaligned_blob_flagged(xm):
    """A blob address off a 16-byte boundary is skipped (never read) and flagged in the scratch status word."""
    H, F = 1024, 512
    arena, L = xm.build_arena(1, H, F, 8, 8, seed=1)
    grp_ptr = torch.tensor([arena[0].data_ptr() + 8], dtype=torch.int64, device=DEV)
    start = torch.tensor([0, 1], dtype=torch.int32, device=DEV)
    zero = torch.zeros(1, dtype=torch.int32, device=DEV)
    ng = torch.ones(1, dtype=torch.int32, device=DEV)
    xq = xm.quantize_q8_1_rows(torch.randn(1, H, device=DEV))
    scratch = torch.zeros(xm.native_expert_scratch_bytes(1, F), dtype=torch.uint8, device=DEV)
    out = torch.zeros(1, H, device=DEV)
    xm.native_expert_grouped(L, grp_ptr, start, ng, zero, zero, 1, 1, xq, scratch, out)
    torch.cuda.synchronize()
    st = scratch[xm.native_expert_scratch_bytes(1, F) - 256:][:4].view(torch.int32)
    assert int(st[0]) == 1


def torch_reference_prefill(xm, arena, L, x, ids, E):
    """fp32 PyTorch reference of the routed products: weights dequantized exactly (xs_iq_dequant_f32), fp32 matmuls,
    h = g / (1 + exp(-g)) * u; returns parts [T*k, H] in routing order."""
    T, H = x.shape
    F = L.n_ff
    k = ids.shape[1]
    parts = torch.zeros(T * k, H, device=DEV)
    flat = ids.reshape(-1)
    for e in torch.unique(flat).tolist():
        rows = torch.nonzero(flat == e).flatten()
        blob = arena[e]
        wg = xm.iq_dequant_f32(L.gu_type, blob[:F * L.gu_row], F * H).reshape(F, H)
        wu = xm.iq_dequant_f32(L.up_type, blob[L.up_off:L.up_off + F * L.up_row], F * H).reshape(F, H)
        wd = xm.iq_dequant_f32(L.d_type, blob[L.down_off:L.down_off + H * L.d_row], H * F).reshape(H, F)
        xs = x[rows // k]
        g = xs @ wg.t().contiguous()
        u = xs @ wu.t().contiguous()
        h = g / (1.0 + torch.exp(-g)) * u
        parts[rows] = h @ wd.t().contiguous()
    return parts


@pytest.mark.parametrize("gu,dt,H,F,T,E", [(12, 14, 2048, 768, 256, 32), (8, 8, 1024, 512, 64, 8),
                                           (23, 23, 4096, 1536, 64, 16), (12, 12, 2048, 512, 5, 16)])
def test_prefill_experts(xm, gu, dt, H, F, T, E):
    k = 8 if E >= 8 else 2
    arena, L = xm.build_arena(E, H, F, gu, dt, seed=gu + H)
    g = torch.Generator(device=DEV).manual_seed(T)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16).float()
    p = 1.0 / torch.arange(1, E + 1, device=DEV, dtype=torch.float32) ** 1.2
    logits = torch.log(p)[None, :] - torch.log(-torch.log(torch.rand(T, E, device=DEV, generator=g)))
    ids, w = xm.router_top10(logits.contiguous(), k)
    r = xm.prefill_route(ids.reshape(-1), k, E, cache_base=arena.data_ptr(), blob=L.bytes, with_ptr=True)
    n = T * k
    cap = min(n, E)
    scratch = torch.zeros(xm.moe_prefill_scratch_bytes(T, n, H, F), dtype=torch.uint8, device=DEV)
    parts = torch.zeros(n, H, device=DEV)
    xm.moe_prefill_experts(L, x, r["src"], r["entry"], r["bounds"], r["n_groups"], r["grp_ptr"], cap, n, scratch,
                           parts)
    torch.cuda.synchronize()
    want = torch_reference_prefill(xm, arena, L, x, ids, E)
    rel = float((parts - want).abs().max() / want.abs().max())
    assert rel <= 2e-2, rel


def test_prefill_experts_saturation_status(xm):
    """xs_moe_prefill_experts flags a value saturated to the f16 range in its scratch's status word
    (xs_moe_prefill_status): clear after a normal call on a zero-filled scratch, bit 8 after a 1e6 activation, and
    xs_moe_status_check raises and clears it."""
    H, F, E, k, T = 1024, 512, 8, 2, 32
    arena, L = xm.build_arena(E, H, F, xm.Q4_K, xm.Q6_K, seed=9)
    g = torch.Generator(device=DEV).manual_seed(9)
    x = torch.randn(T, H, device=DEV, generator=g)
    logits = torch.randn(T, E, device=DEV, generator=g)
    ids, _ = xm.router_top10(logits, k)
    r = xm.prefill_route(ids.reshape(-1), k, E, cache_base=arena.data_ptr(), blob=L.bytes, with_ptr=True)
    n = T * k
    scratch = torch.zeros(xm.moe_prefill_scratch_bytes(T, n, H, F), dtype=torch.uint8, device=DEV)
    status = xm.lib().xs_moe_prefill_status(scratch.data_ptr(), T, n, H, F)
    parts = torch.zeros(n, H, device=DEV)
    for bad in (False, True):
        xb = x.clone()
        if bad:
            xb[3, 7] = 1e6
        xm.moe_prefill_experts(L, xb, r["src"], r["entry"], r["bounds"], r["n_groups"], r["grp_ptr"], min(n, E), n,
                               scratch, parts)
        torch.cuda.synchronize()
        if bad:
            with pytest.raises(xm.XsError, match="f16 range"):
                xm._check(xm.lib().xs_moe_status_check(status, None))
        xm._check(xm.lib().xs_moe_status_check(status, None))   # clear (again)
