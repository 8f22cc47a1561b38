"""ctypes loader of oracle/liboracle.so (the CPU restatement of the reference's MoE hot path) and of oracle/_ref's
shim over the reference's own host headers.  TEST INFRASTRUCTURE: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may load this module, and only as the checker."""
import ctypes
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF = HERE / "_ref" / "libxsref.so"
CPU = HERE / "libxscpu.so"

Q8_0, Q4_K, Q6_K, IQ4_XS = 8, 12, 14, 23
BLOCK_VALUES = {Q8_0: 32, Q4_K: 256, Q6_K: 256, IQ4_XS: 256}
BLOCK_BYTES = {Q8_0: 34, Q4_K: 144, Q6_K: 210, IQ4_XS: 136}

P = ctypes.c_void_p
I, I64, F = ctypes.c_int, ctypes.c_int64, ctypes.c_float


class Layout(ctypes.Structure):
    _fields_ = [("gu_type", I), ("d_type", I), ("n_embd", I64), ("n_ff", I64), ("gu_row", I64), ("d_row", I64),
                ("up_off", I64), ("down_off", I64), ("bytes", I64), ("up_type", I64), ("up_row", I64)]


_lib = None
_ref = None


def build():
    subprocess.run(["make", "-s", "-C", str(HERE), "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        L.xso_fp16_to_fp32.restype = F
        L.xso_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.xso_fp32_to_fp16.restype = ctypes.c_uint16
        L.xso_fp32_to_fp16.argtypes = [F]
        L.xso_row_bytes.restype = I64
        L.xso_vec_dot.restype = F
        L.xso_vec_dot.argtypes = [I, P, P, I64, I]
        L.xso_vec_dot_calls.restype = F
        L.xso_vec_dot_calls.argtypes = [I, P, P, I64, I]
        L.xso_canon_rcp.restype = F
        L.xso_canon_rcp.argtypes = [F]
        L.xso_canon_exp.restype = F
        L.xso_canon_exp.argtypes = [F]
        L.xso_decode_plan.restype = I
        L.xso_prefill_route.restype = I
        L.xso_prefill_route.argtypes = [P, I64, I, I, P, P, P, P, P, P]
        L.xso_dequant_row.argtypes = [I, P, I64, P]
        L.xso_quantize_q8_1_rows.argtypes = [P, I64, I64, P]
        L.xso_quantize_q8_1_per32.argtypes = [P, I64, P]
        L.xso_native_layout.argtypes = [I, I, I64, I64, ctypes.POINTER(Layout)]
        L.xso_native_layout_mixed.argtypes = [I, I, I64, I64, I, ctypes.POINTER(Layout)]
        L.xso_native_expert_grouped.argtypes = [ctypes.POINTER(Layout), P, P, I, P, P, P, P, P, P, P, I]
        L.xso_router_top10.argtypes = [P, I, I, I, P, P]
        L.xso_router_grouped_sigmoid.argtypes = [P, P, I, I, I, I, I, F, P, P]
        L.xso_decode_plan.argtypes = [P, I, I, P, P, P, P, P]
        L.xso_combine.argtypes = [P, P, P, P, P, I64, I, I]
        L.xso_expert_float.argtypes = [ctypes.POINTER(Layout), P, P, P, I, P, I]
        L.xso_moe_layer_decode.argtypes = [ctypes.POINTER(Layout), P, I, I, P, P, P, I, P, I]
        L.xso_shared_expert.argtypes = [ctypes.POINTER(Layout), P, P, I, P, I]
        L.xso_moe_layer_decode_shared.argtypes = [ctypes.POINTER(Layout), P, I, I, P, P, P, I, ctypes.POINTER(Layout),
                                                  P, P, P, I]
        L.xso_canon_silu_mul_n.argtypes = [P, P, I64, P]
        L.xso_canon_exp_n.argtypes = [P, I64, P]
        L.xso_canon_rcp_n.argtypes = [P, I64, P]
        L.xso_mmvf_block.argtypes = [I64]
        L.xso_mmvf.argtypes = [P, I64, P, P, P, I64, I64, I64, I]
        L.xso_gemm_rows.argtypes = [P, I64, P, P, I64, I64, I64, I64]
        L.xso_bf16_gemv.argtypes = [P, P, P, I64, I64, I, I]
        _lib = L
    return _lib


def ref():
    """oracle/_ref's shim over the reference's dequant.hpp / canon_math.hpp, or None where it is not built."""
    global _ref
    if _ref is None and REF.exists():
        R = ctypes.CDLL(str(REF))
        R.xsref_fp16_to_fp32.restype = F
        R.xsref_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        R.xsref_dequant.argtypes = [I, P, I64, P]
        R.xsref_canon_exp.argtypes = [P, I64, P]
        R.xsref_canon_rcp.argtypes = [P, I64, P]
        R.xsref_canon_silu_mul.argtypes = [P, P, I64, P]
        R.xsref_canon_q8.argtypes = [P, I64, P, P, P]
        R.xsref_bf16_from_f32.argtypes = [P, I64, P]
        _ref = R
    return _ref


_cpu = None


def cpu():
    """oracle/libxscpu.so: the reference's CPU decode path restated for AVX2 (bench.py's cpu_baseline)."""
    global _cpu
    if _cpu is None:
        if not CPU.exists():
            subprocess.run(["make", "-s", "-C", str(HERE), "libxscpu.so"], check=True)
        C = ctypes.CDLL(str(CPU))
        C.xscpu_init.argtypes = [I]
        C.xscpu_init.restype = I
        C.xscpu_quantize_q8_k.argtypes = [P, I64, P]
        C.xscpu_quantize_q8_0.argtypes = [P, I64, P]
        C.xscpu_row_dot.argtypes = [I, P, I64, P]
        C.xscpu_row_dot.restype = F
        lay = [I, I, I64, I64, I64, I64, I64, I64, P, I64, I, I]
        C.xscpu_layer_decode.argtypes = lay + [P, P, P, I, P]
        C.xscpu_layer_decode.restype = I
        C.xscpu_time.argtypes = lay + [P, P, I, P, I, P, I, I]
        C.xscpu_time.restype = ctypes.c_double
        _cpu = C
    return _cpu


def cpu_q8_k(x):
    """ggml's Q8_K blocks of x (292 bytes a 256 values) as (d f32 [nb], qs int8 [nb, 256], bsums int16 [nb, 16])."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    nb = x.size // 256
    y = np.zeros(nb * 292, np.uint8)
    cpu().xscpu_quantize_q8_k(_a(x), x.size, _a(y))
    b = y.reshape(nb, 292)
    return b[:, :4].copy().view(np.float32).ravel(), b[:, 4:260].copy().view(np.int8), \
        b[:, 260:].copy().view(np.int16), y


def cpu_q8_0(x):
    """Q8_0 activations (the fp16 scale as a float, 36 bytes a 32 values) as (d [nb], qs [nb, 32], raw bytes)."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    nb = x.size // 32
    y = np.zeros(nb * 36, np.uint8)
    cpu().xscpu_quantize_q8_0(_a(x), x.size, _a(y))
    b = y.reshape(nb, 36)
    return b[:, :4].copy().view(np.float32).ravel(), b[:, 4:].copy().view(np.int8), y


def _cpu_layout_args(L, arena, blob, n_expert, k):
    return (L.gu_type, L.d_type, L.n_embd, L.n_ff, L.gu_row, L.d_row, L.up_off, L.down_off, _a(arena), blob,
            n_expert, k)


def cpu_layer_decode(L, arena, blob, n_expert, k, x, logits, residual):
    """out = residual + MoE(x) on the CPU path (n_tok <= 8); arena: uint8 [n_expert * blob]."""
    x = np.ascontiguousarray(x, np.float32)
    logits = np.ascontiguousarray(logits, np.float32)
    residual = np.ascontiguousarray(residual, np.float32)
    out = np.zeros_like(residual)
    r = cpu().xscpu_layer_decode(*_cpu_layout_args(L, arena, blob, n_expert, k), _a(x), _a(logits), _a(residual),
                                 x.shape[0], _a(out))
    if r:
        raise ValueError("cpu path: unsupported layer")
    return out


def cpu_time(L, arena, blob, n_expert, k, x, logit_sets, residual, reps=10, trials=5):
    """Microseconds a layer call: the best of `trials` means of `reps` calls, logits rotating over the sets."""
    x = np.ascontiguousarray(x, np.float32)
    logit_sets = np.ascontiguousarray(logit_sets, np.float32)
    residual = np.ascontiguousarray(residual, np.float32)
    out = np.zeros_like(residual)
    n_sets = logit_sets.shape[0]
    return cpu().xscpu_time(*_cpu_layout_args(L, arena, blob, n_expert, k), _a(x), _a(logit_sets), n_sets,
                            _a(residual), x.shape[0], _a(out), reps, trials)


def _a(x):
    return x.ctypes.data_as(P)


def row_bytes(t, n):
    return n // BLOCK_VALUES[t] * BLOCK_BYTES[t]


def dequant(t, blocks, n):
    out = np.zeros(n, np.float32)
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    lib().xso_dequant_row(t, _a(b), n, _a(out))
    return out


def canon_exp(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().xso_canon_exp_n(_a(x), x.size, _a(y))
    return y


def canon_rcp(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().xso_canon_rcp_n(_a(x), x.size, _a(y))
    return y


def canon_silu_mul(g, u):
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    h = np.empty_like(g)
    lib().xso_canon_silu_mul_n(_a(g), _a(u), g.size, _a(h))
    return h


def quantize_q8_1_rows(x):
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    y = np.zeros(rows * cols // 32 * 36, np.uint8)
    lib().xso_quantize_q8_1_rows(_a(x), rows, cols, _a(y))
    return y


def quantize_q8_1_per32(x):
    x = np.ascontiguousarray(x, np.float32).ravel()
    y = np.zeros(x.size // 32 * 36, np.uint8)
    lib().xso_quantize_q8_1_per32(_a(x), x.size, _a(y))
    return y


def q8_1_values(y):
    """q8_1 bytes -> (int8 values, fp32 d per block, fp32 s per block)."""
    b = np.asarray(y, np.uint8).reshape(-1, 36)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    s = b[:, 2:4].copy().view(np.float16).astype(np.float32).ravel()
    q = b[:, 4:].copy().view(np.int8)
    return q, d, s


def vec_dot(t, row, xq, n, s256, calls=False):
    row = np.ascontiguousarray(row, np.uint8)
    xq = np.ascontiguousarray(xq, np.uint8)
    fn = lib().xso_vec_dot_calls if calls else lib().xso_vec_dot
    return fn(t, _a(row), _a(xq), n, int(s256))


def layout(gu, d, n_embd, n_ff, up=-1):
    """up >= 0 and not gu: a mixed layer (up rows of their own type)."""
    L = Layout()
    if not lib().xso_native_layout_mixed(gu, d, n_embd, n_ff, gu if up < 0 else up, ctypes.byref(L)):
        raise ValueError("unsupported layout")
    return L


def native_expert_grouped(L, blobs, start, ent_dst, ent_tok, x_q8_1, n_out_rows, n_threads=8, want_inner=False):
    """blobs: list of uint8 arrays (one per group).  Returns out [n_out_rows, n_embd] (and gate, up, hq)."""
    ng = len(blobs)
    keep = [np.ascontiguousarray(b, np.uint8) for b in blobs]
    arr = (ctypes.c_void_p * max(ng, 1))(*[b.ctypes.data for b in keep])
    start = np.ascontiguousarray(start, np.int32)
    ent_dst = np.ascontiguousarray(ent_dst, np.int32)
    ent_tok = np.ascontiguousarray(ent_tok, np.int32)
    x_q8_1 = np.ascontiguousarray(x_q8_1, np.uint8)
    out = np.zeros((n_out_rows, L.n_embd), np.float32)
    n_ent = int(start[ng] - start[0])
    gate = np.zeros((max(n_ent, 1), L.n_ff), np.float32)
    up = np.zeros_like(gate)
    hq = np.zeros(max(n_ent, 1) * (L.n_ff // 32) * 36, np.uint8)
    lib().xso_native_expert_grouped(ctypes.byref(L), ctypes.cast(arr, P), _a(start), ng, _a(ent_dst), _a(ent_tok),
                                    _a(x_q8_1), _a(out), _a(gate), _a(up), _a(hq), n_threads)
    if want_inner:
        return out, gate[:n_ent], up[:n_ent], hq[: n_ent * (L.n_ff // 32) * 36]
    return out


def expert_float(L, blobs, x, tok, n_threads=8):
    keep = [np.ascontiguousarray(b, np.uint8) for b in blobs]
    arr = (ctypes.c_void_p * len(keep))(*[b.ctypes.data for b in keep])
    x = np.ascontiguousarray(x, np.float32)
    tok = np.ascontiguousarray(tok, np.int32)
    out = np.zeros((len(keep), L.n_embd), np.float32)
    lib().xso_expert_float(ctypes.byref(L), ctypes.cast(arr, P), _a(x), _a(tok), len(keep), _a(out), n_threads)
    return out


def router_top10(logits, k, ids=None, weights=None):
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    ids = np.zeros((T, k), np.int32) if ids is None else ids.copy()
    w = np.zeros((T, k), np.float32) if weights is None else weights.copy()
    lib().xso_router_top10(_a(logits), T, E, k, _a(ids), _a(w))
    return ids, w


def router_grouped_sigmoid(logits, bias, n_group, topk_group, k, routed_scale):
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    ids = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().xso_router_grouped_sigmoid(_a(logits), None if b is None else _a(b), T, E, n_group, topk_group, k,
                                     routed_scale, _a(ids), _a(w))
    return ids, w


def decode_plan(ids, k):
    ids = np.ascontiguousarray(ids, np.int32).ravel()
    n = ids.size
    counts = np.zeros(4, np.int32)
    start = np.zeros(n + 1, np.int32)
    dst = np.zeros(n, np.int32)
    tok = np.zeros(n, np.int32)
    gexp = np.zeros(n, np.int32)
    g = lib().xso_decode_plan(_a(ids), n, k, _a(counts), _a(start), _a(dst), _a(tok), _a(gexp))
    return dict(counts=counts, start=start[: g + 1], dst=dst, tok=tok, experts=gexp[:g], groups=g)


def prefill_route(ids, k, n_expert):
    ids = np.ascontiguousarray(ids, np.int32).ravel()
    n = ids.size
    src = np.zeros(n, np.int32)
    slot = np.zeros(n, np.int32)
    entry = np.zeros(n, np.int32)
    bounds = np.zeros(n_expert + 1, np.int32)
    experts = np.zeros(n_expert, np.int32)
    counts = np.zeros(n_expert, np.int32)
    g = lib().xso_prefill_route(_a(ids), n, k, n_expert, _a(src), _a(slot), _a(entry), _a(bounds), _a(experts),
                                _a(counts))
    return dict(src=src, slot=slot, entry=entry, bounds=bounds[: g + 1], experts=experts[:g], counts=counts, groups=g)


def combine(parts, weights, shared=None, shared_gate=None, n_embd=None, k=None, n_tok=None):
    parts = np.ascontiguousarray(parts, np.float32)
    weights = np.ascontiguousarray(weights, np.float32)
    out = np.zeros((n_tok, n_embd), np.float32)
    sh = None if shared is None else np.ascontiguousarray(shared, np.float32)
    sg = None if shared_gate is None else np.ascontiguousarray(shared_gate, np.float32)
    lib().xso_combine(_a(parts), _a(weights), None if sh is None else _a(sh), None if sg is None else _a(sg), _a(out),
                      n_embd, k, n_tok)
    return out


def moe_layer_decode(L, blobs_by_expert, k, x, logits, residual, n_threads=1):
    keep = [np.ascontiguousarray(b, np.uint8) for b in blobs_by_expert]
    arr = (ctypes.c_void_p * len(keep))(*[b.ctypes.data for b in keep])
    x = np.ascontiguousarray(x, np.float32)
    logits = np.ascontiguousarray(logits, np.float32)
    residual = np.ascontiguousarray(residual, np.float32)
    out = np.zeros_like(residual)
    lib().xso_moe_layer_decode(ctypes.byref(L), ctypes.cast(arr, P), len(keep), k, _a(x), _a(logits), _a(residual),
                               x.shape[0], _a(out), n_threads)
    return out


def shared_expert(SL, blob, x, n_threads=8):
    """One shared expert over the tokens of x [T, n_embd] -> rows [T, n_embd]."""
    x = np.ascontiguousarray(x, np.float32)
    blob = np.ascontiguousarray(blob, np.uint8)
    out = np.zeros((x.shape[0], SL.n_embd), np.float32)
    lib().xso_shared_expert(ctypes.byref(SL), _a(blob), _a(x), x.shape[0], _a(out), n_threads)
    return out


def moe_layer_decode_shared(L, blobs_by_expert, k, x, logits, residual, SL, shared_blob, gate_logit=None,
                            n_threads=8):
    keep = [np.ascontiguousarray(b, np.uint8) for b in blobs_by_expert]
    arr = (ctypes.c_void_p * len(keep))(*[b.ctypes.data for b in keep])
    x = np.ascontiguousarray(x, np.float32)
    logits = np.ascontiguousarray(logits, np.float32)
    residual = np.ascontiguousarray(residual, np.float32)
    sb = np.ascontiguousarray(shared_blob, np.uint8)
    g = None if gate_logit is None else np.ascontiguousarray(gate_logit, np.float32)
    out = np.zeros_like(residual)
    lib().xso_moe_layer_decode_shared(ctypes.byref(L), ctypes.cast(arr, P), len(keep), k, _a(x), _a(logits),
                                      _a(residual), x.shape[0], ctypes.byref(SL), _a(sb),
                                      None if g is None else _a(g), _a(out), n_threads)
    return out


def bf16_from_f32(x):
    """include/strata/kernels/bf16_bits.hpp:39-45 (uint16 bits): nearest even on bit 16, a NaN kept with bit 6 set."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + ((u >> 16) & 1) + 0x7FFF) & 0xFFFF0000) >> 16
    return np.where(nan, (u >> 16) | 64, r).astype(np.uint16)


def mmvf(x, w, n_tok=None):
    """The decode GEMV's order (bf16_gemv.cpp:91-147): x [n_tok, n_in] f32, w [n_out, n_in] f32 or bf16 bits
    (uint16) -> [n_tok, n_out]."""
    x = np.ascontiguousarray(x, np.float32)
    n_tok = x.shape[0] if n_tok is None else n_tok
    n_out, n_in = w.shape
    y = np.zeros((n_tok, n_out), np.float32)
    if w.dtype == np.uint16:
        lib().xso_mmvf(_a(x), x.shape[1], None, _a(np.ascontiguousarray(w)), _a(y), n_out, n_in, n_out, n_tok)
    else:
        lib().xso_mmvf(_a(x), x.shape[1], _a(np.ascontiguousarray(w, np.float32)), None, _a(y), n_out, n_in, n_out,
                       n_tok)
    return y


def gemm_rows(x, w):
    """The prompt GEMM's order (bf16_gemv.cpp:475-502)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.zeros((x.shape[0], w.shape[0]), np.float32)
    lib().xso_gemm_rows(_a(x), x.shape[1], _a(w), _a(y), w.shape[0], x.shape[1], w.shape[0], x.shape[0])
    return y


def bf16_gemv(x_bits, w_bits, form, tpr=32):
    """bf16 x . bf16 rows in launch_warp (form 0), launch_naive (1) or the split tree (2) order."""
    w_bits = np.ascontiguousarray(w_bits, np.uint16)
    y = np.zeros(w_bits.shape[0], np.float32)
    lib().xso_bf16_gemv(_a(np.ascontiguousarray(x_bits, np.uint16)), _a(w_bits), _a(y), w_bits.shape[1],
                        w_bits.shape[0], form, tpr)
    return y


def mmq_quantize(x, ids, cols, rows, sums, dup=False):
    """The int8 MMQ activations (src/kernels/xe/iq_mmq.cpp:1264-1302, iq_mmq_act_bytes and iq_mmq_quantize) as the
    bytes the reference lays out: int8 q[rows][oc] | f32 d[rows][oc/32] | f32 d*sum(q)[rows][oc/32] (zeros where
    `sums` is off), oc = 2 cols with `dup` (each block twice).  Per block: d = amax / 127 and id = 1 / d (0 when
    amax == 0) in float32 (IEEE division), q = round half away from zero of fl(v * id) (sycl::round)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    src = np.arange(rows) if ids is None else np.asarray(ids, dtype=np.int64)
    v = x[src, :cols].reshape(rows, cols // 32, 32)
    amax = np.max(np.abs(v), axis=2)
    with np.errstate(divide="ignore"):
        d = (amax / np.float32(127.0)).astype(np.float32)
        idv = np.where(amax > 0, np.float32(1.0) / np.where(d > 0, d, np.float32(1.0)), np.float32(0.0))
    prod = (v * idv.astype(np.float32)[:, :, None]).astype(np.float32).astype(np.float64)
    q = (np.sign(prod) * np.floor(np.abs(prod) + 0.5)).astype(np.int64)
    s = (d * q.sum(axis=2).astype(np.float32)).astype(np.float32)
    rep = 2 if dup else 1
    q8 = np.repeat(q.astype(np.int8), rep, axis=1).reshape(rows, cols * rep)
    dd = np.repeat(d, rep, axis=1)
    ss = np.repeat(s, rep, axis=1) if sums else np.zeros_like(dd)
    return np.concatenate([q8.view(np.uint8).ravel(), dd.view(np.uint8).ravel(), ss.view(np.uint8).ravel()])


def mmq_quantize_parts(buf, rows, oc):
    """Split mmq_quantize's bytes into (q int8 [rows, oc], d f32 [rows, oc/32], s f32 [rows, oc/32])."""
    nb = oc // 32
    q = buf[:rows * oc].view(np.int8).reshape(rows, oc)
    d = buf[rows * oc:rows * oc + 4 * rows * nb].view(np.float32).reshape(rows, nb)
    s = buf[rows * oc + 4 * rows * nb:rows * oc + 8 * rows * nb].view(np.float32).reshape(rows, nb)
    return q, d, s


def rel_max(a, b):
    """The reference's relative error: max |a - b| / max |b| (src/kernels/iq_mmq_parity.cpp:126-134)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def rel_sum(a, b):
    """Sum-relative error: sum |a - b| / sum |b| (src/kernels/native_expert_parity.cpp:46-50)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.sum(np.abs(a - b)) / (np.sum(np.abs(b)) + 1e-30))
