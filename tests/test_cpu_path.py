"""The CPU/host baseline (oracle/cpu_path.cpp, the reference's CPU decode path restated for AVX2) on the CPU.

Pins, since ggml (whose quantizers and float orders the reference's CPU path runs) is absent from this image:
- the activation quantizers by their closed forms (Q8_K: the signed max's -127 / max scale, nearest-even codes
  clamped at 127, 16-value sums; Q8_0: an fp16 amax / 127, nearest-even codes of x * 127 / amax), with exact ties
  and the first-largest-magnitude rule built in;
- the row dots against float64 sums of the dequantized weights times the dequantized activations (the integer part
  of every block is exact; only the float accumulation rounds);
- the whole layer against the float64 expert reference (fp32 activations) within the int8 activations' error.
The float accumulation order is this file's own and stays parity-unpinned against ggml's."""
import numpy as np
import pytest

from test_oracle import random_rows


def test_q8_k_closed_form(xo):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(256 * 6) * np.array([1, 1e-3, 1e4, 1, 1, 1]).repeat(256)).astype(np.float32)
    x[256 * 3:256 * 4] = 0.0                                  # a zero block
    x[256 * 4 + 3], x[256 * 4 + 100] = -5.0, 5.0              # the largest magnitude twice: the FIRST one's sign wins
    x[256 * 4:256 * 5] = np.clip(x[256 * 4:256 * 5], -4.0, 4.0)
    x[256 * 4 + 3], x[256 * 4 + 100] = -5.0, 5.0
    blk = x[256 * 5:256 * 6]
    blk[:] = 0.0
    blk[0], blk[1], blk[2], blk[3] = -127.0, 2.5, -2.5, 3.5   # max = -127: iscale 1, exact ties to even
    d, qs, bs, _ = xo.cpu_q8_k(x)
    v = x.reshape(6, 256)
    for b in range(6):
        if not np.any(v[b]):
            assert d[b] == 0 and not qs[b].any() and not bs[b].any()
            continue
        i = int(np.argmax(np.abs(v[b])))                       # the first largest magnitude
        iscale = np.float32(-127.0) / v[b, i]
        assert qs[b, i] == -127
        p = (iscale * v[b]).astype(np.float32).astype(np.float64)
        q = qs[b].astype(np.float64)
        assert np.all(np.abs(q - p) <= 0.5)
        ties = np.abs(np.abs(p - np.trunc(p)) - 0.5) == 0
        assert np.all(q[ties] % 2 == 0)
        assert d[b] == np.float32(1.0) / iscale
        np.testing.assert_array_equal(bs[b], qs[b].astype(np.int64).reshape(16, 16).sum(axis=1))
    assert qs[4, 3] == -127 and qs[4, 100] == 127             # -5 first: max = -5, iscale 25.4 (+5 first: -25.4)
    assert list(qs[5, :4]) == [-127, 2, -2, 4]                # max = -127: iscale 1, 2.5 -> 2, -2.5 -> -2, 3.5 -> 4


def test_q8_0_closed_form(xo):
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(32 * 8) * 3).astype(np.float32)
    x[32:64] = 0.0
    x[64:96] = 0.0
    x[64], x[65], x[66] = 127.0, 2.5, -3.5                     # amax 127: inverse 1, ties to even
    d, qs, _ = xo.cpu_q8_0(x)
    v = x.reshape(8, 32)
    for b in range(8):
        amax = np.float32(np.max(np.abs(v[b])))
        assert d[b] == np.float32(np.float16(amax / np.float32(127)))
        inv = np.float32(127) / amax if amax else np.float32(0)
        want = np.rint((v[b] * inv).astype(np.float32))        # numpy rint: nearest even
        np.testing.assert_array_equal(qs[b], want.astype(np.int8))
    assert list(qs[2, :3]) == [127, 2, -4]


@pytest.mark.parametrize("t,n", [(12, 2048), (14, 768), (8, 1024), (14, 2048)])
def test_row_dot_exact_integer_parts(xo, t, n):
    """One row against a quantized activation: within float rounding of the float64 sum of dequantized operands."""
    rng = np.random.default_rng(t * n)
    row = random_rows(xo, t, 1, n, rng)
    w = xo.dequant(t, row, n).astype(np.float64)
    x = rng.standard_normal(n).astype(np.float32)
    if t == 8:
        d, qs, raw = xo.cpu_q8_0(x)
        a = (qs.astype(np.float64) * d[:, None].astype(np.float64)).ravel()
    else:
        d, qs, _, raw = xo.cpu_q8_k(x)
        a = (qs.astype(np.float64) * d[:, None].astype(np.float64)).ravel()
    got = xo.cpu().xscpu_row_dot(t, xo._a(np.ascontiguousarray(row)), n, xo._a(raw))
    want = float(w @ a)
    assert abs(got - want) <= 1e-5 * float(np.abs(w) @ np.abs(a)) + 1e-30, (got, want)


def _layer(xo, gu, dn, H, F, E, seed):
    rng = np.random.default_rng(seed)
    L = xo.layout(gu, dn, H, F)
    blobs = []
    for _ in range(E):
        g = random_rows(xo, gu, F, H, rng)
        u = random_rows(xo, gu, F, H, rng)
        d = random_rows(xo, dn, H, F, rng)
        b = np.zeros(L.bytes, np.uint8)
        b[:g.size] = g
        b[L.up_off:L.up_off + u.size] = u
        b[L.down_off:L.down_off + d.size] = d
        blobs.append(b)
    return L, blobs, rng


@pytest.mark.parametrize("gu,dn,H,F,E,k,T", [(8, 8, 1024, 512, 8, 2, 4), (12, 14, 2048, 768, 16, 8, 1),
                                             (12, 14, 2048, 768, 16, 8, 3)])
def test_cpu_layer_close_to_float(xo, gu, dn, H, F, E, k, T):
    """The whole CPU layer (router, Q8 activations, rows, SwiGLU, down, combine, residual) against the float64
    expert reference with fp32 activations: within 3e-2 of the MoE part's largest magnitude (two int8 roundings
    of the activations); the residual added exactly."""
    L, blobs, rng = _layer(xo, gu, dn, H, F, E, gu * 100 + T)
    arena = np.concatenate(blobs)
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    res = rng.standard_normal((T, H)).astype(np.float32)
    xo.cpu().xscpu_init(4)
    got = xo.cpu_layer_decode(L, arena, L.bytes, E, k, x, logits, res)
    ids, w = xo.router_top10(logits, k)
    moe = np.zeros((T, H), np.float64)
    for t in range(T):
        outs = xo.expert_float(L, [blobs[e] for e in ids[t]], x, np.full(k, t, np.int32), n_threads=4)
        moe[t] = (outs.astype(np.float64) * w[t][:, None]).sum(axis=0)
    err = np.max(np.abs((got - res).astype(np.float64) - moe)) / np.max(np.abs(moe))
    assert err <= 3e-2, err
