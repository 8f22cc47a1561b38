"""GPU parity of the drop-in surface around the path: the FP16 dequantizer, the int8 MMQ activations (gathered and
scattered), the prompt path's SwiGLU and iota rows, and the combine with the tier path's hit rows folded in.

Bars: bytes bit for bit (FP16 weights, int8 codes, scales and sums, the ungated combine); the SwiGLU and the gated
combine within 1e-6 relative (each side's own expf)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def t2n(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("t", [8, 12, 14, 23])
def test_iq_dequant_f16(xm, xo, t):
    """iq_dequant_f16: the oracle's fp32 dequantized values rounded to FP16 (nearest even), bit for bit."""
    g = torch.Generator().manual_seed(40 + t)
    x = (torch.randn(32, 1024, generator=g) * 0.05).to(DEV)
    blocks = xm.quantize_rows(t, x.reshape(-1))
    n = x.numel()
    got = t2n(xm.iq_dequant_f16(t, blocks, n))
    want = xo.dequant(t, t2n(blocks), n).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def _acts(rows, cols, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, cols)) * 0.3).astype(np.float32)
    x[0, :32] = 0.0
    x[-1, 7] = 2.0e5                 # an outlier block
    x[rows // 2, 64:96] = np.float32(0.5) * np.arange(-16, 16, dtype=np.float32) / np.float32(127.0 / 15.5)
    return x


@pytest.mark.parametrize("rows,cols,use_ids,sums,dup", [
    (1, 2048, False, True, False), (37, 7168, True, True, False), (64, 1536, True, False, False),
    (9, 256, False, True, True), (300, 4096, True, True, False)])
def test_mmq_quantize(xm, xo, rows, cols, use_ids, sums, dup):
    """iq_mmq_quantize against the oracle's restatement of the reference's, byte for byte over the whole buffer
    (codes, scales, sums; the sums part left as allocated when not asked for)."""
    n_src = rows + 5
    x = _acts(n_src, cols, rows)
    ids = np.random.default_rng(rows).integers(0, n_src, rows).astype(np.int32) if use_ids else None
    got = t2n(xm.iq_mmq_quantize(torch.from_numpy(x).to(DEV), torch.from_numpy(ids).to(DEV) if use_ids else None,
                                 cols, cols, rows, sums, dup))
    want = xo.mmq_quantize(x, ids, cols, rows, sums, dup)
    assert got.size == want.size == xm.iq_mmq_act_bytes(rows, 2 * cols if dup else cols)
    assert np.array_equal(got, want)


def test_mmq_quantize_strided_rows(xm, xo):
    """ld > cols: the first cols values of each ld-float row."""
    x = _acts(12, 1024 + 64, 3)
    got = t2n(xm.iq_mmq_quantize(torch.from_numpy(x).to(DEV), None, 1024, 1024 + 64, 12, True))
    assert np.array_equal(got, xo.mmq_quantize(np.ascontiguousarray(x[:, :1024]), None, 1024, 12, True))


@pytest.mark.parametrize("n_tok,k,n_expert,dup", [(5, 2, 8, False), (64, 8, 128, False), (33, 4, 16, True)])
def test_mmq_quantize_scatter(xm, xo, n_tok, k, n_expert, dup):
    """iq_mmq_quantize_scatter over the prompt permutation's slots writes the bytes iq_mmq_quantize writes over its
    rows' tokens (src), the oracle's bytes."""
    cols = 512
    rng = np.random.default_rng(n_tok)
    x = _acts(n_tok, cols, n_tok + 1)
    ids = np.stack([rng.permutation(n_expert)[:k] for _ in range(n_tok)]).astype(np.int32)
    pr = xo.prefill_route(ids, k, n_expert)
    src, slot = pr["src"], pr["slot"]
    rows = n_tok * k
    got = t2n(xm.iq_mmq_quantize_scatter(torch.from_numpy(x).to(DEV), torch.from_numpy(slot.astype(np.int32)).to(DEV),
                                         cols, cols, n_tok, k, True, dup))
    want = xo.mmq_quantize(x, src.astype(np.int64), cols, rows, True, dup)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("interleaved", [False, True])
def test_mmq_swiglu(xm, interleaved):
    rows, n_ff = 19, 768
    g = torch.Generator().manual_seed(11)
    gu = torch.randn(rows, 2 * n_ff, generator=g) * 4
    got = t2n(xm.mmq_swiglu(gu.to(DEV), rows, n_ff, interleaved)).astype(np.float64)
    a = gu.double().numpy()
    gate, up = (a[:, 0::2], a[:, 1::2]) if interleaved else (a[:, :n_ff], a[:, n_ff:])
    want = gate / (1 + np.exp(-gate)) * up
    assert np.max(np.abs(got - want)) <= 1e-6 * np.max(np.abs(want))


def test_mmq_iota(xm):
    assert np.array_equal(t2n(xm.mmq_iota(5000)), np.arange(5000, dtype=np.int32))


@pytest.mark.parametrize("k,n,shared,gated,n_hit", [(8, 5, False, False, 11), (4, 16, True, False, 64),
                                                   (8, 3, True, True, 7), (15, 2, False, False, 0)])
def test_combine_multi_hits(xm, xo, k, n, shared, gated, n_hit):
    """native_moe_combine_multi_hits: the entries listed in dst[0, *count) (any order) read parts + hits before
    their product - the oracle's combine over parts with those rows replaced by the float32 sums; the list's unused
    tail and out-of-range entries are ignored."""
    N = 1024
    g = torch.Generator().manual_seed(k * 10 + n)
    parts = torch.randn(n * k, N, generator=g)
    hits = torch.randn(n * k, N, generator=g)
    w = torch.randint(0, 1000, (n * k,), generator=g).float() / 1000
    sh = torch.randn(n, N, generator=g)
    gate = torch.randn(n, generator=g)
    rng = np.random.default_rng(n_hit)
    listed = rng.permutation(n * k)[:n_hit].astype(np.int32)
    stray = np.array([n * k + 3, -1], np.int32)                  # out of range: ignored
    dst = np.concatenate([listed, stray, np.array([0, 1] * 4, np.int32)])   # a tail past *count: never read
    count = np.array([n_hit + 2], np.int32)
    out = torch.empty(n, N, device=DEV)
    xm.native_moe_combine_multi_hits(parts.to(DEV), hits.to(DEV), torch.from_numpy(dst).to(DEV),
                                     torch.from_numpy(count).to(DEV), w.to(DEV), sh.to(DEV) if shared else None, out,
                                     N, k, n, shared_gate=gate.to(DEV) if gated else None)
    p = parts.numpy().copy()
    p[listed] = (p[listed] + hits.numpy()[listed]).astype(np.float32)
    want = xo.combine(p, w.numpy(), sh.numpy() if shared else None, gate.numpy() if gated else None, N, k, n)
    got = t2n(out)
    if gated:
        assert np.max(np.abs(got - want)) <= 1e-6 * np.max(np.abs(want))
    else:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------------------------------------ router projections

@pytest.mark.parametrize("n_tok,n_out,n_in", [(1, 128, 2048), (4, 256, 7168), (8, 128, 4096), (3, 5, 192),
                                              (1, 1, 2048), (2, 64, 64)])
def test_mmvf_bits(xm, xo, n_tok, n_out, n_in):
    """f32_gemv_fp32_mmvf_multi and its BF16-weight twin: the oracle's bits (the reference's decode order)."""
    rng = np.random.default_rng(n_in + n_out)
    x = rng.standard_normal((n_tok, n_in)).astype(np.float32)
    w = (rng.standard_normal((n_out, n_in)) * 0.02).astype(np.float32)
    got = t2n(xm.f32_gemv_fp32_mmvf_multi(torch.from_numpy(x).to(DEV), torch.from_numpy(w).to(DEV)))
    assert np.array_equal(got.view(np.uint32), xo.mmvf(x, w).view(np.uint32))
    wb = xo.bf16_from_f32(w)
    got = t2n(xm.f32_gemv_fp32_mmvf_multi(torch.from_numpy(x).to(DEV), torch.from_numpy(wb.view(np.int16)).to(DEV)))
    assert np.array_equal(got.view(np.uint32), xo.mmvf(x, wb).view(np.uint32))


@pytest.mark.parametrize("n_tok,n_out,n_in", [(1, 128, 2048), (100, 256, 7168), (300, 128, 2048), (70, 1, 1000),
                                              (9, 65, 48)])
def test_gemm_rows_bits(xm, xo, n_tok, n_out, n_in):
    """f32_gemm_rows: the oracle's bits (one FMA chain a logit, the prompt path's order)."""
    rng = np.random.default_rng(n_tok * n_in)
    x = rng.standard_normal((n_tok, n_in)).astype(np.float32)
    w = (rng.standard_normal((n_out, n_in)) * 0.02).astype(np.float32)
    got = t2n(xm.f32_gemm_rows(torch.from_numpy(x).to(DEV), torch.from_numpy(w).to(DEV)))
    assert np.array_equal(got.view(np.uint32), xo.gemm_rows(x, w).view(np.uint32))


def test_f32_to_bf16_reference_vectors(xm, golden):
    """f32_to_bf16_bulk against the reference's own bf16_from_f32 outputs (committed vectors: ties, carries,
    overflow to inf, NaNs kept quiet)."""
    ref, _ = golden
    got = t2n(xm.f32_to_bf16_bulk(torch.from_numpy(ref["bf16_x"]).to(DEV))).view(np.uint16)
    assert np.array_equal(got, ref["bf16_y"])


@pytest.mark.parametrize("n_out,n_in", [(128, 2048), (256, 7168), (40, 2048), (96, 1000)])
def test_bf16_projection_bits(xm, xo, n_out, n_in):
    """project_bf16 (f32 -> bf16 bits, then the 32-lane rows), its one-launch form, bf16_gemv (one chain a row below
    64 rows) and bf16_gemv_split at 64 and 256 threads: the oracle's bits."""
    rng = np.random.default_rng(n_out)
    x = rng.standard_normal(n_in).astype(np.float32)
    w = xo.bf16_from_f32((rng.standard_normal((n_out, n_in)) * 0.02).astype(np.float32))
    xd, wd = torch.from_numpy(x).to(DEV), torch.from_numpy(w.view(np.int16)).to(DEV)
    xb = xo.bf16_from_f32(x)
    for split, x_bf16 in ((True, torch.empty(n_in, dtype=torch.int16, device=DEV)), (True, None),
                          (False, torch.empty(n_in, dtype=torch.int16, device=DEV))):
        got = t2n(xm.project_bf16(xd, wd, split=split, x_bf16=x_bf16))
        want = xo.bf16_gemv(xb, w, 0 if split or n_out >= 64 else 1)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (split, x_bf16 is None)
    for tpr in (64, 256):
        got = t2n(xm.bf16_gemv(torch.from_numpy(xb.view(np.int16)).to(DEV), wd, threads_per_row=tpr))
        assert np.array_equal(got.view(np.uint32), xo.bf16_gemv(xb, w, 2, tpr).view(np.uint32))
    got = t2n(xm.project_bf16(xd, wd, native=True))       # the native form: bf16 weights against f32 x, mmvf order
    assert np.array_equal(got.view(np.uint32), xo.mmvf(x[None], w)[0].view(np.uint32))


@pytest.mark.parametrize("n_tok,n_expert,n_in,k", [(1, 128, 2048, 8), (8, 256, 7168, 8), (64, 128, 2048, 8),
                                                   (1024, 128, 4096, 8)])
def test_ids_from_own_logits(xm, xo, n_tok, n_expert, n_in, k):
    """The ids routed from this library's own router GEMV (xs_router_logits_f32: the decode order up to 8 tokens,
    the prompt order above) equal the ids the oracle routes from the reference-order logits - every token, every
    rank, and the weights' bits."""
    rng = np.random.default_rng(n_tok)
    x = rng.standard_normal((n_tok, n_in)).astype(np.float32)
    w = (rng.standard_normal((n_expert, n_in)) * 0.03).astype(np.float32)
    xd, wd = torch.from_numpy(x).to(DEV), torch.from_numpy(w).to(DEV)
    logits = xm.router_logits_f32(xd, wd)
    ids, wts = xm.router_top10(logits, k)
    want_logits = xo.mmvf(x, w) if n_tok <= 8 else xo.gemm_rows(x, w)
    assert np.array_equal(t2n(logits).view(np.uint32), want_logits.view(np.uint32))
    rids, rw = xo.router_top10(want_logits, k)
    assert np.array_equal(t2n(ids), rids)
    assert np.array_equal(t2n(wts).view(np.uint32), rw.view(np.uint32))


@pytest.mark.parametrize("t,w_rows,w_cols,counts,use_wtab", [
    (12, 512, 2048, [40, 0, 300, 7, 129, 64], False), (14, 2048, 768, [128, 1, 0, 257, 33], False),
    (8, 512, 1024, [5, 200, 77, 0], True), (23, 256, 4096, [65, 3, 130], False),
    (12, 768, 2048, [1, 2, 3, 150, 0, 0, 9, 31], True)])
def test_iq_mmq_grouped(xm, t, w_rows, w_cols, counts, use_wtab):
    """iq_mmq_grouped over xs_iq_mmq_quantize's int8 activations: expert e's rows bounds[e] .. bounds[e + 1] times its
    weights (contiguous, or through a device table in another order) into dst rows ids[row] of a wider dst, against an
    fp32 reference over the exactly dequantized weights and activations (q * d): within 2e-2 (the f16 MFMA path); the
    columns past w_rows untouched."""
    g = torch.Generator(device=DEV).manual_seed(t * 1000 + w_rows)
    n = len(counts)
    rb = xm.row_bytes(t, w_cols)
    eb = (w_rows * rb + 255) // 256 * 256 + 256          # expert_bytes: padded past the matrix
    wbuf = torch.zeros(n * eb, dtype=torch.uint8, device=DEV)
    W = []
    for e in range(n):
        w = torch.randn(w_rows, w_cols, generator=g, device=DEV) * 0.02
        xm.quantize_rows(t, w.reshape(-1), out=wbuf[e * eb:e * eb + w_rows * rb])
        W.append(xm.iq_dequant_f32(t, wbuf[e * eb:e * eb + w_rows * rb], w_rows * w_cols).reshape(w_rows, w_cols))
    total = sum(counts)
    bounds = torch.tensor(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32), device=DEV)
    x = torch.randn(total, w_cols, generator=g, device=DEV)
    xq = xm.iq_mmq_quantize(x, None, w_cols, w_cols, total, True)
    q = xq[:total * w_cols].view(torch.int8).reshape(total, w_cols).float()
    d = xq[total * w_cols:total * w_cols + total * (w_cols // 32) * 4].view(torch.float32).reshape(total, -1)
    a = q * d.repeat_interleave(32, dim=1)
    ids = torch.randperm(total, generator=torch.Generator().manual_seed(5)).to(torch.int32).to(DEV)
    ld = w_rows + 64
    dst = torch.full((total, ld), 7.0, device=DEV)
    order = list(range(n))
    table = None
    if use_wtab:                                          # expert e's weights: blob order[e]
        order = list(reversed(range(n)))
        table = torch.tensor([wbuf.data_ptr() + o * eb for o in order], dtype=torch.int64, device=DEV)
    xm.iq_mmq_grouped(t, None if use_wtab else wbuf, eb, w_rows, w_cols, n, xq, total, bounds, ids, dst, ld,
                      wtab=table)
    ref = torch.zeros(total, w_rows, device=DEV)
    for e in range(n):
        r0, r1 = int(bounds[e]), int(bounds[e + 1])
        if r1 > r0:
            ref[r0:r1] = a[r0:r1] @ W[order[e]].t().contiguous()
    got = dst[ids.long()]
    rel = float((got[:, :w_rows] - ref).abs().max() / ref.abs().max())
    assert rel <= 2e-2, rel
    assert bool((got[:, w_rows:] == 7.0).all())
