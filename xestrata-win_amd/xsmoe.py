"""Host-side mirror of XeStrata's MoE kernel API over libxsmoe.so (include/xs_moe.h), for Python callers.

Device memory and streams are torch tensors on a HIP device and torch's current stream: plumbing only; every
computation runs in the library's HIP kernels.  Names and argument meanings follow the reference's
strata::kernels functions (router_top10, quantize_q8_1_rows, native_expert_grouped, resident_plan,
native_moe_combine_multi, ...); a failing call raises XsError with the library's message, as the reference's
entry points throw (std::invalid_argument / core::DeviceError).

There is no fallback: when libxsmoe.so is missing every call raises.
"""
import ctypes
import pathlib

import torch

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libxsmoe.so"

Q8_0, Q4_K, Q6_K, IQ4_XS = 8, 12, 14, 23
BLOCK_VALUES = {Q8_0: 32, Q4_K: 256, Q6_K: 256, IQ4_XS: 256}
BLOCK_BYTES = {Q8_0: 34, Q4_K: 144, Q6_K: 210, IQ4_XS: 136}
XS_OK, XS_EINVAL, XS_EDEVICE = 0, 1, 2


class XsError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


class Layout(ctypes.Structure):
    """xs_expert_layout_t: the reference's NativeExpertLayout (include/strata/kernels/iq_kernels.hpp:66-75)."""
    _fields_ = [("gu_type", ctypes.c_int), ("d_type", ctypes.c_int), ("up_type", ctypes.c_int),
                ("n_embd", ctypes.c_int64), ("n_ff", ctypes.c_int64),
                ("gu_row", ctypes.c_size_t), ("d_row", ctypes.c_size_t), ("up_row", ctypes.c_size_t),
                ("up_off", ctypes.c_size_t), ("down_off", ctypes.c_size_t), ("bytes", ctypes.c_size_t)]


_lib = None
class PackInfo(ctypes.Structure):
    """xs_pack_info_t: a pack's ExpertLayout totals (include/strata/kernels/cpu/expert_layout.hpp:21-49)."""
    _fields_ = [("version", ctypes.c_int), ("has_gguf_off", ctypes.c_int), ("n_layers", ctypes.c_int64),
                ("n_expert", ctypes.c_int64), ("max_blob", ctypes.c_uint64), ("total", ctypes.c_uint64)]


class PackLayer(ctypes.Structure):
    """xs_pack_layer_t: one layer's row of ExpertLayout (expert_layout.hpp:22-44)."""
    _fields_ = [("gu_type", ctypes.c_int), ("d_type", ctypes.c_int), ("up_type", ctypes.c_int),
                ("block", ctypes.c_int64), ("offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64),
                ("up_off", ctypes.c_uint64), ("down_off", ctypes.c_uint64), ("gguf_off", ctypes.c_uint64 * 3),
                ("gguf_file", ctypes.c_char_p * 3)]


class RouterCfg(ctypes.Structure):
    """xs_router_cfg_t: how a layer routes (XS_ROUTER_SOFTMAX, or XS_ROUTER_GROUPED_SIGMOID with its bias, groups and
    routed scale)."""
    _fields_ = [("kind", ctypes.c_int), ("bias", ctypes.c_void_p), ("n_group", ctypes.c_int),
                ("topk_group", ctypes.c_int), ("routed_scale", ctypes.c_float)]


ROUTER_SOFTMAX, ROUTER_GROUPED_SIGMOID = 0, 1


def grouped_sigmoid_router(bias, n_group, topk_group, routed_scale):
    """DeepSeek-V3's routing for a layer: (RouterCfg, bias tensor kept alive with it)."""
    cfg = RouterCfg(ROUTER_GROUPED_SIGMOID, None if bias is None else bias.data_ptr(), n_group, topk_group,
                    float(routed_scale))
    cfg._keep = bias
    return cfg


class PackLoadStats(ctypes.Structure):
    _fields_ = [("bytes", ctypes.c_uint64), ("layers", ctypes.c_uint64), ("seconds", ctypes.c_double)]


P, I, I64, SZ, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float
LP = ctypes.POINTER(Layout)
RP = ctypes.c_void_p
LL = ctypes.c_longlong
U32 = ctypes.c_uint32
U64 = ctypes.c_uint64
S = ctypes.c_char_p

_SIGS = {
    "xs_last_error": (ctypes.c_char_p, []),
    "xs_abi_version": (I, []),
    "xs_iq_row_bytes": (SZ, [I, I64]),
    "xs_native_expert_supported": (I, [I, I, I64, I64, I]),
    "xs_native_expert_layout": (I, [I, I, I64, I64, I, LP]),
    "xs_native_expert_scratch_bytes": (SZ, [I64, I64]),
    "xs_native_expert_status": (P, [P, I64, I64]),
    "xs_native_expert_gate_up": (I, [LP, P, P, P, P, I64, I64, P, P, P, I64]),
    "xs_native_expert_down": (I, [LP, P, P, P, P, I64, I64, P, P, P, I64]),
    "xs_quantize_q8_1_rows": (I, [P, I64, I64, P, P]),
    "xs_native_expert_grouped": (I, [LP, P, P, P, P, P, I64, I64, P, P, P, P, I64]),
    "xs_iq_dequant_f32": (I, [I, P, I64, P, P]),
    "xs_iq_dequant_bf16": (I, [I, P, I64, P, P]),
    "xs_iq_dequant_f16": (I, [I, P, I64, P, P]),
    "xs_moe_status_check": (I, [P, P]),
    "xs_moe_set_wait_bound": (None, [LL]),
    "xs_moe_set_prefill_tall": (None, [I]),
    "xs_bench_hbm_read": (I, [P, SZ, P, I, P]),
    "xs_bench_mfma_f16": (I, [I, I, P, P]),
    "xs_bench_occupy": (I, [I, I, LL, P, P]),
    "xs_bench_lds_read": (I, [I, I, P, P]),
    "xs_f32_gemv_fp32_mmvf_multi": (I, [P, I64, P, P, I64, I64, I64, I, P]),
    "xs_bf16_gemv_fp32_mmvf_multi": (I, [P, I64, P, P, I64, I64, I64, I, P]),
    "xs_f32_gemm_rows": (I, [P, I64, P, P, I64, I64, I64, I64, P]),
    "xs_f32_to_bf16_bulk": (I, [P, P, I64, P]),
    "xs_bf16_gemv": (I, [P, P, P, I64, I64, P]),
    "xs_bf16_gemv_split": (I, [P, P, P, I64, I64, I, P]),
    "xs_project_bf16": (I, [P, P, P, P, I64, I64, I, I, P]),
    "xs_iq_mmq_act_bytes": (ctypes.c_size_t, [I64, I64]),
    "xs_iq_mmq_type_sums": (I, [I]),
    "xs_iq_mmq_type_dup": (I, [I]),
    "xs_iq_mmq_quantize": (I, [P, P, P, I64, I64, I64, I, I, P]),
    "xs_iq_mmq_quantize_scatter": (I, [P, P, P, I64, I64, I64, I, I, I, P]),
    "xs_mmq_swiglu": (I, [P, P, I64, I64, I, P]),
    "xs_iq_mmq_grouped": (I, [I, P, SZ, I64, I64, I, P, I64, P, I64, P, P, I64, P, SZ, I64, P]),
    "xs_mmq_iota": (I, [P, I64, P]),
    "xs_quantize_rows": (I, [I, P, I64, P, P]),
    "xs_router_top10": (I, [P, I, I, I, P, P, P]),
    "xs_router_grouped_sigmoid": (I, [P, P, I, I, I, I, I, F, P, P, P]),
    "xs_router_logits_f32": (I, [P, P, P, I, I64, I, P]),
    "xs_resident_plan": (I, [P, I, I, P, I, P, P, LL, P, LL, P, U32, P]),
    "xs_plan_offsets": (None, [LL, P, P, P, P, P]),
    "xs_prefill_route": (I, [P, I64, I, I, P, P, P, P, P, P, P, LL, P, P]),
    "xs_moe_prefill_experts": (I, [LP, P, I64, P, P, P, P, P, I64, I64, P, P, P]),
    "xs_moe_prefill_scratch_bytes": (SZ, [I64, I64, I64, I64]),
    "xs_moe_prefill_status": (P, [P, I64, I64, I64, I64]),
    "xs_native_moe_combine": (I, [P, P, P, P, I64, I64, P]),
    "xs_native_moe_combine_multi": (I, [P, P, P, P, I64, I64, I, P, P]),
    "xs_moe_combine_residual": (I, [P, P, P, P, P, P, I64, I64, I, P]),
    "xs_native_moe_combine_multi_hits": (I, [P, P, P, P, P, P, P, I64, I64, I, P, P]),
    "xs_add_inplace": (I, [P, P, I64, P]),
    "xs_moe_layer_decode": (I, [LP, P, SZ, I, I, P, P, P, P, I, P, SZ, P]),
    "xs_moe_layer_decode_workspace_bytes": (SZ, [LP, I, I, I]),
    "xs_moe_layer_decode_status": (P, [P]),
    "xs_moe_layer_prefill_status": (P, [P]),
    "xs_moe_layer_decode_noalloc": (I, [LP, P, SZ, I, I, P, P, P, P, I, P, P]),
    "xs_moe_layer_decode_noalloc_status": (P, []),
    "xs_moe_layer_prefill": (I, [LP, P, SZ, I, I, P, P, P, P, I, P, SZ, P]),
    "xs_shared_expert_decode": (I, [LP, P, P, I, P, P, P, P, SZ, P]),
    "xs_shared_expert_decode_workspace_bytes": (SZ, [LP, I]),
    "xs_moe_layer_decode_shared": (I, [LP, P, SZ, I, I, P, P, P, P, I, LP, P, P, P, SZ, P]),
    "xs_moe_layer_decode_shared_workspace_bytes": (SZ, [LP, I, I, I, LP]),
    "xs_moe_layer_prefill_workspace_bytes": (SZ, [LP, I, I, I]),
    "xs_moe_layer_decode_ex": (I, [LP, P, SZ, I, I, P, P, P, P, I, RP, LP, P, P, P, SZ, P]),
    "xs_moe_layer_decode_ex_workspace_bytes": (SZ, [LP, I, I, I, LP]),
    "xs_moe_layer_prefill_ex": (I, [LP, P, SZ, I, I, P, P, P, P, I, RP, LP, P, P, P, SZ, P]),
    "xs_moe_layer_prefill_ex_workspace_bytes": (SZ, [LP, I, I, I, LP]),
    # include/xs_pack.h
    "xs_pack_layout_load": (I, [S, I64, I64, I64, I64, ctypes.POINTER(P)]),
    "xs_pack_layout_from_gguf": (I, [S, ctypes.POINTER(I64), I64, I64, I64, I64, ctypes.POINTER(P)]),
    "xs_pack_free": (None, [P]),
    "xs_pack_info": (I, [P, ctypes.POINTER(PackInfo)]),
    "xs_pack_layer": (I, [P, I64, ctypes.POINTER(PackLayer)]),
    "xs_pack_blob_offset": (U64, [P, I64, I64]),
    "xs_pack_check_gguf": (I, [P, S]),
    "xs_pack_load_gguf": (I, [P, S, P, U64, I, ctypes.POINTER(PackLoadStats)]),
    "xs_pack_load_gguf_layers": (I, [P, S, ctypes.POINTER(P), I, ctypes.POINTER(PackLoadStats)]),
    # include/xs_tiers.h
    "xs_wait_flag_ge": (I, [P, U32, I64, P, P]),
    "xs_copy_i32_from_mapped": (I, [P, P, I64, P]),
    "xs_copy_rows_from_mapped": (I, [P, P, I64, I64, P, P, P]),
    "xs_fetch_blobs": (I, [P, P, P, I64, I, P]),
    "xs_rebase_ptrs": (I, [P, P, P, I64, P]),
    "xs_moe_hit_add": (I, [P, P, P, P, I64, I64, P]),
}


def lib():
    """The loaded libxsmoe.so; raises when it is not built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `python xestrata-win_amd/build.py`")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(code):
    if code != XS_OK:
        raise XsError(code, lib().xs_last_error().decode())


def _p(t):
    """Device address of a tensor (None -> NULL)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream=None):
    if stream is not None:
        return getattr(stream, "cuda_stream", stream)   # a torch stream or a raw handle
    return torch.cuda.current_stream().cuda_stream


# ------------------------------------------------------------------------------------------------ formats

def row_bytes(t, n):
    return lib().xs_iq_row_bytes(t, n)


def native_expert_supported(gu, d, n_embd, n_ff, up=-1):
    return bool(lib().xs_native_expert_supported(gu, d, n_embd, n_ff, up))


def native_expert_layout(gu, d, n_embd, n_ff, up=-1):
    L = Layout()
    _check(lib().xs_native_expert_layout(gu, d, n_embd, n_ff, up, ctypes.byref(L)))
    return L


def native_expert_scratch_bytes(cap_entries, n_ff):
    return lib().xs_native_expert_scratch_bytes(cap_entries, n_ff)


def quantize_rows(t, x, out=None, stream=None):
    """Float rows (device fp32, a whole number of blocks) -> `t` blocks (uint8 device tensor)."""
    n = x.numel()
    if out is None:
        out = torch.empty(n // BLOCK_VALUES[t] * BLOCK_BYTES[t], dtype=torch.uint8, device=x.device)
    _check(lib().xs_quantize_rows(t, _p(x), n, _p(out), _stream(stream)))
    return out


def iq_dequant_f32(t, src, n, out=None, stream=None):
    if out is None:
        out = torch.empty(n, dtype=torch.float32, device=src.device)
    _check(lib().xs_iq_dequant_f32(t, _p(src), n, _p(out), _stream(stream)))
    return out


def iq_dequant_bf16(t, src, n, out=None, stream=None):
    if out is None:
        out = torch.empty(n, dtype=torch.int16, device=src.device)
    _check(lib().xs_iq_dequant_bf16(t, _p(src), n, _p(out), _stream(stream)))
    return out


def iq_dequant_f16(t, src, n, out=None, stream=None):
    if out is None:
        out = torch.empty(n, dtype=torch.float16, device=src.device)
    _check(lib().xs_iq_dequant_f16(t, _p(src), n, _p(out), _stream(stream)))
    return out


# ------------------------------------------------------------------------------------------------ activations

def quantize_q8_1_rows(x, out=None, stream=None):
    """x [rows, cols] fp32 -> q8_1 blocks, rows * cols / 32 * 36 bytes (reference quantize_q8_1_rows)."""
    rows, cols = x.shape
    if out is None:
        out = torch.empty(rows * cols // 32 * 36, dtype=torch.uint8, device=x.device)
    _check(lib().xs_quantize_q8_1_rows(_p(x), rows, cols, _p(out), _stream(stream)))
    return out


# ------------------------------------------------------------------------------------------------ routing

def router_top10(logits, k, ids=None, weights=None, stream=None):
    """logits [T, E] fp32 -> (ids [T, k] int32, weights [T, k] fp32) (reference router_top10)."""
    T, E = logits.shape
    if ids is None:
        ids = torch.empty(T, k, dtype=torch.int32, device=logits.device)
    if weights is None:
        weights = torch.empty(T, k, dtype=torch.float32, device=logits.device)
    _check(lib().xs_router_top10(_p(logits), T, E, k, _p(ids), _p(weights), _stream(stream)))
    return ids, weights


def router_grouped_sigmoid(logits, bias, n_group, topk_group, k, routed_scale, stream=None):
    T, E = logits.shape
    ids = torch.empty(T, k, dtype=torch.int32, device=logits.device)
    weights = torch.empty(T, k, dtype=torch.float32, device=logits.device)
    _check(lib().xs_router_grouped_sigmoid(_p(logits), _p(bias), T, E, n_group, topk_group, k, float(routed_scale),
                                           _p(ids), _p(weights), _stream(stream)))
    return ids, weights


def router_logits_f32(x, w, stream=None):
    T, H = x.shape
    E = w.shape[0]
    logits = torch.empty(T, E, dtype=torch.float32, device=x.device)
    _check(lib().xs_router_logits_f32(_p(x), _p(w), _p(logits), T, H, E, _stream(stream)))
    return logits


def plan_offsets(capx):
    v = [ctypes.c_longlong() for _ in range(5)]
    lib().xs_plan_offsets(capx, *[ctypes.byref(x) for x in v])
    return dict(zip(("start", "dst", "tok", "ptr", "start2"), (x.value for x in v)))


def plan_words(capx):
    o = plan_offsets(capx)
    return o["start2"] + capx + 2


def resident_plan(ids, k, res, n_expert, cache_base, slot_off, blob, plan, capx, skip, ring, stream=None):
    n = ids.numel()
    _check(lib().xs_resident_plan(_p(ids), n, k, _p(res), n_expert, cache_base, _p(slot_off), blob, _p(plan), capx,
                                  _p(skip), ring, _stream(stream)))


def prefill_route(ids, k, n_expert, cache_base=None, blob=0, with_ptr=False, stream=None):
    """ids [T*k] -> dict(src, slot, entry, bounds, experts, n_groups, grp_ptr) (reference plain_prompt.cpp:576-637)."""
    n = ids.numel()
    dev = ids.device
    o = dict(src=torch.empty(n, dtype=torch.int32, device=dev), slot=torch.empty(n, dtype=torch.int32, device=dev),
             entry=torch.empty(n, dtype=torch.int32, device=dev),
             bounds=torch.empty(n_expert + 1, dtype=torch.int32, device=dev),
             experts=torch.empty(n_expert, dtype=torch.int32, device=dev),
             n_groups=torch.empty(1, dtype=torch.int32, device=dev),
             grp_ptr=torch.empty(n_expert, dtype=torch.int64, device=dev) if with_ptr else None)
    _check(lib().xs_prefill_route(_p(ids), n, k, n_expert, _p(o["src"]), _p(o["slot"]), _p(o["entry"]),
                                  _p(o["bounds"]), _p(o["experts"]), _p(o["n_groups"]), cache_base, blob,
                                  _p(o["grp_ptr"]), _stream(stream)))
    return o


# ------------------------------------------------------------------------------------------------ experts

def native_expert_grouped(L, grp_ptr, grp_start, n_groups, ent_dst, ent_tok, cap_groups, cap_entries, x_q8_1, scratch,
                          out, grid_groups=0, stream=None):
    _check(lib().xs_native_expert_grouped(ctypes.byref(L), _p(grp_ptr), _p(grp_start), _p(n_groups), _p(ent_dst),
                                          _p(ent_tok), cap_groups, cap_entries, _p(x_q8_1), _p(scratch), _p(out),
                                          _stream(stream), grid_groups))


def native_expert_gate_up(L, grp_ptr, grp_start, n_groups, ent_tok, cap_groups, cap_entries, x_q8_1, scratch,
                          grid_groups=0, stream=None):
    _check(lib().xs_native_expert_gate_up(ctypes.byref(L), _p(grp_ptr), _p(grp_start), _p(n_groups), _p(ent_tok),
                                          cap_groups, cap_entries, _p(x_q8_1), _p(scratch), _stream(stream),
                                          grid_groups))


def native_expert_down(L, grp_ptr, grp_start, n_groups, ent_dst, cap_groups, cap_entries, scratch, out, grid_groups=0,
                       stream=None):
    _check(lib().xs_native_expert_down(ctypes.byref(L), _p(grp_ptr), _p(grp_start), _p(n_groups), _p(ent_dst),
                                       cap_groups, cap_entries, _p(scratch), _p(out), _stream(stream), grid_groups))


def native_expert_status(scratch, cap_entries, n_ff):
    return lib().xs_native_expert_status(_p(scratch), cap_entries, n_ff)


def moe_prefill_scratch_bytes(n_tok, rows, n_embd, n_ff):
    return lib().xs_moe_prefill_scratch_bytes(n_tok, rows, n_embd, n_ff)


def moe_prefill_experts(L, x, src, entry, bounds, n_groups, grp_ptr, cap_groups, rows, scratch, parts, stream=None):
    _check(lib().xs_moe_prefill_experts(ctypes.byref(L), _p(x), x.shape[0], _p(src), _p(entry), _p(bounds),
                                        _p(n_groups), _p(grp_ptr), cap_groups, rows, _p(scratch), _p(parts),
                                        _stream(stream)))


# ------------------------------------------------------------------------------------------------ router projections

def f32_gemv_fp32_mmvf_multi(x, w, n_tok=None, out=None, stream=None):
    """logits [n_tok, n_out] = x [n_tok, n_in] . w [n_out, n_in]^T in the decode GEMV's order (1..8 tokens)."""
    n_tok = x.shape[0] if n_tok is None else n_tok
    n_out, n_in = w.shape
    if out is None:
        out = torch.empty(n_tok, n_out, dtype=torch.float32, device=x.device)
    fn = lib().xs_bf16_gemv_fp32_mmvf_multi if w.dtype in (torch.int16, torch.bfloat16) else \
        lib().xs_f32_gemv_fp32_mmvf_multi
    _check(fn(_p(x), x.stride(0), _p(w), _p(out), out.stride(0), n_in, n_out, n_tok, _stream(stream)))
    return out


def f32_gemm_rows(x, w, out=None, stream=None):
    """The prompt path's GEMM order: one FMA chain a logit."""
    n_tok, n_in = x.shape
    n_out = w.shape[0]
    if out is None:
        out = torch.empty(n_tok, n_out, dtype=torch.float32, device=x.device)
    _check(lib().xs_f32_gemm_rows(_p(x), x.stride(0), _p(w), _p(out), out.stride(0), n_in, n_out, n_tok,
                                  _stream(stream)))
    return out


def f32_to_bf16_bulk(x, out=None, stream=None):
    if out is None:
        out = torch.empty(x.numel(), dtype=torch.int16, device=x.device)
    _check(lib().xs_f32_to_bf16_bulk(_p(x), _p(out), x.numel(), _stream(stream)))
    return out


def bf16_gemv(x, w, out=None, threads_per_row=None, stream=None):
    """x bf16 bits [n_in], w bf16 bits [n_out, n_in]: bf16_gemv, or bf16_gemv_split at threads_per_row."""
    n_out, n_in = w.shape
    if out is None:
        out = torch.empty(n_out, dtype=torch.float32, device=w.device)
    if threads_per_row is None:
        _check(lib().xs_bf16_gemv(_p(x), _p(w), _p(out), n_in, n_out, _stream(stream)))
    else:
        _check(lib().xs_bf16_gemv_split(_p(x), _p(w), _p(out), n_in, n_out, threads_per_row, _stream(stream)))
    return out


def project_bf16(x, w, split=True, native=False, x_bf16=None, out=None, stream=None):
    n_out, n_in = w.shape
    if out is None:
        out = torch.empty(n_out, dtype=torch.float32, device=w.device)
    _check(lib().xs_project_bf16(_p(x), _p(x_bf16), _p(w), _p(out), n_in, n_out, int(split), int(native),
                                 _stream(stream)))
    return out


# ------------------------------------------------------------------------------------------------ int8 MMQ staging

def iq_mmq_act_bytes(rows, cols):
    return lib().xs_iq_mmq_act_bytes(rows, cols)


def iq_mmq_type_sums(t):
    return bool(lib().xs_iq_mmq_type_sums(t))


def iq_mmq_type_dup(t):
    return bool(lib().xs_iq_mmq_type_dup(t))


def iq_mmq_quantize(x, ids, cols, ld, rows, sums, dup=False, out=None, stream=None):
    """int8 MMQ activations (xs_iq_mmq_quantize): a uint8 device tensor of iq_mmq_act_bytes(rows, oc) bytes."""
    if out is None:
        out = torch.zeros(iq_mmq_act_bytes(rows, 2 * cols if dup else cols), dtype=torch.uint8, device=x.device)
    _check(lib().xs_iq_mmq_quantize(_p(x), _p(ids), _p(out), cols, ld, rows, int(sums), int(dup), _stream(stream)))
    return out


def iq_mmq_grouped(type_, w, expert_bytes, w_rows, w_cols, n, xq, total_rows, bounds, ids, dst, ld_dst, wtab=None,
                   woff=0, rows=0, max_rows=0, stream=None):
    """n experts' [w_rows, w_cols] products over the int8 MMQ activations xq into dst rows ids[row]
    (xs_iq_mmq_grouped).  w: the first expert's weights (experts expert_bytes apart) or, with wtab (a device int64
    tensor of n addresses), ignored."""
    _check(lib().xs_iq_mmq_grouped(type_, _p(w), expert_bytes, w_rows, w_cols, n, _p(xq),
                                   total_rows, _p(bounds), max_rows, _p(ids), _p(dst), ld_dst, _p(wtab), woff, rows,
                                   _stream(stream)))
    return dst


def iq_mmq_quantize_scatter(x, slot, cols, ld, tokens, k_used, sums, dup=False, out=None, stream=None):
    if out is None:
        out = torch.zeros(iq_mmq_act_bytes(tokens * k_used, 2 * cols if dup else cols), dtype=torch.uint8,
                          device=x.device)
    _check(lib().xs_iq_mmq_quantize_scatter(_p(x), _p(slot), _p(out), cols, ld, tokens, k_used, int(sums), int(dup),
                                            _stream(stream)))
    return out


def mmq_swiglu(gu, rows, n_ff, interleaved, out=None, stream=None):
    if out is None:
        out = torch.empty(rows, n_ff, dtype=torch.float32, device=gu.device)
    _check(lib().xs_mmq_swiglu(_p(gu), _p(out), rows, n_ff, int(interleaved), _stream(stream)))
    return out


def mmq_iota(n, out=None, device="cuda", stream=None):
    if out is None:
        out = torch.empty(n, dtype=torch.int32, device=device)
    _check(lib().xs_mmq_iota(_p(out), n, _stream(stream)))
    return out


# ------------------------------------------------------------------------------------------------ combine

def native_moe_combine_multi(parts, weights, shared, output, n_embd, k, n_tok, shared_gate=None, stream=None):
    _check(lib().xs_native_moe_combine_multi(_p(parts), _p(weights), _p(shared), _p(output), n_embd, k, n_tok,
                                             _stream(stream), _p(shared_gate)))


def native_moe_combine_multi_hits(parts, hits, dst, count, weights, shared, output, n_embd, k, n_tok,
                                  shared_gate=None, stream=None):
    _check(lib().xs_native_moe_combine_multi_hits(_p(parts), _p(hits), _p(dst), _p(count), _p(weights), _p(shared),
                                                  _p(output), n_embd, k, n_tok, _stream(stream), _p(shared_gate)))


def moe_combine_residual(parts, weights, residual, output, n_embd, k, n_tok, shared=None, shared_gate=None,
                         stream=None):
    _check(lib().xs_moe_combine_residual(_p(parts), _p(weights), _p(shared), _p(shared_gate), _p(residual),
                                         _p(output), n_embd, k, n_tok, _stream(stream)))


# ------------------------------------------------------------------------------------------------ whole layers

def moe_layer_decode_noalloc(L, arena, n_expert, k, x, logits, residual, out, status=None, blob_bytes=None,
                             stream=None):
    """The decode layer in the library's own device scratch (xs_moe_layer_decode_noalloc): no workspace, nothing
    allocated.  status: an optional int32 device tensor the call ORs its error bits into."""
    _check(lib().xs_moe_layer_decode_noalloc(ctypes.byref(L), _p(arena), L.bytes if blob_bytes is None else blob_bytes,
                                             n_expert, k, _p(x), _p(logits), _p(residual), _p(out), x.shape[0],
                                             _p(status), _stream(stream)))
    return out


def noalloc_status_check(stream=None):
    """Synchronize and raise XsError when the fixed scratch's own status word (where xs_moe_layer_decode_noalloc ORs
    its bits when called with status=None) is set; the word is then cleared."""
    st = lib().xs_moe_layer_decode_noalloc_status()
    if not st:
        raise XsError(XS_EDEVICE, lib().xs_last_error().decode())
    _check(lib().xs_moe_status_check(st, _stream(stream)))


def shared_expert_decode(SL, blob, x, w_gate=None, stream=None):
    """One shared expert over the tokens of x [T, n_embd] (blob: the expert's native bytes on the device) -> (shared
    rows [T, n_embd], gate logits [T] or None)."""
    T = x.shape[0]
    ws_bytes = lib().xs_shared_expert_decode_workspace_bytes(ctypes.byref(SL), T)
    ws = torch.zeros(ws_bytes + 256, dtype=torch.uint8, device=x.device)
    shared = torch.empty(T, SL.n_embd, dtype=torch.float32, device=x.device)
    gate = torch.empty(T, dtype=torch.float32, device=x.device) if w_gate is not None else None
    _check(lib().xs_shared_expert_decode(ctypes.byref(SL), _p(blob), _p(x), T, _p(w_gate), _p(shared), _p(gate),
                                         (ws.data_ptr() + 255) & ~255, ws_bytes, _stream(stream)))
    return shared, gate


class MoeLayer:
    """One MoE layer whose experts live in one HBM arena (expert e's native blob at arena + e * blob_bytes), with its
    workspace allocated once, so calls allocate nothing (graph-capturable).  shared = (SL, blob, w_gate or None): a
    shared expert added by the combine; router: None (the softmax top-k) or a RouterCfg (grouped_sigmoid_router)."""

    def __init__(self, L, arena, n_expert, k, max_tokens, prefill=False, device="cuda", shared=None, router=None):
        self.L, self.arena, self.n_expert, self.k, self.max_tokens = L, arena, n_expert, k, max_tokens
        self.blob = L.bytes
        self.prefill = prefill
        self.shared = shared
        self.router = router
        # the _ex entry points take a router and a shared expert on either path; the plain ones keep their own
        self.ex = router is not None or (prefill and shared is not None)
        SLp = ctypes.byref(shared[0]) if shared is not None else None
        if self.ex:
            fn = lib().xs_moe_layer_prefill_ex_workspace_bytes if prefill else lib().xs_moe_layer_decode_ex_workspace_bytes
            self.ws_bytes = fn(ctypes.byref(L), n_expert, k, max_tokens, SLp)
        elif shared is not None:
            self.ws_bytes = lib().xs_moe_layer_decode_shared_workspace_bytes(ctypes.byref(L), n_expert, k, max_tokens,
                                                                             SLp)
        else:
            fn = lib().xs_moe_layer_prefill_workspace_bytes if prefill else lib().xs_moe_layer_decode_workspace_bytes
            self.ws_bytes = fn(ctypes.byref(L), n_expert, k, max_tokens)
        # zeroed once: the decode layer's counters start at zero and every call leaves them there
        self.ws = torch.zeros(self.ws_bytes + 256, dtype=torch.uint8, device=device)
        self.ws_ptr = (self.ws.data_ptr() + 255) & ~255

    def status(self):
        """The workspace's status word (0: every call so far was good; the prompt layer's word is its workspace's first
        too: bit 8, a value saturated to the f16 range).  Synchronizes the device."""
        off = self.ws_ptr - self.ws.data_ptr()
        torch.cuda.synchronize(self.ws.device)
        return int(self.ws[off:off + 4].view(torch.int32).item())

    def check(self):
        """Synchronize and raise XsError when the status word is not 0 (decode: a bounded wait of the persistent layer
        ran out - its output is not valid - or a token's router produced fewer than k experts; prompt: a value passed
        the f16 range and was saturated); the word is cleared."""
        fn = lib().xs_moe_layer_prefill_status if self.prefill else lib().xs_moe_layer_decode_status
        _check(lib().xs_moe_status_check(fn(self.ws_ptr), None))

    def __call__(self, x, logits, residual, out, n_tok=None, arena=None, stream=None, shared_blob=None):
        """shared_blob: this call's shared-expert blob in place of the one given at construction (same layout)."""
        n_tok = x.shape[0] if n_tok is None else n_tok
        arena = self.arena if arena is None else arena
        if self.ex:
            SL, sblob, w_gate = self.shared if self.shared is not None else (None, None, None)
            sblob = sblob if shared_blob is None else shared_blob
            fn = lib().xs_moe_layer_prefill_ex if self.prefill else lib().xs_moe_layer_decode_ex
            _check(fn(ctypes.byref(self.L), _p(arena), self.blob, self.n_expert, self.k, _p(x), _p(logits),
                      _p(residual), _p(out), n_tok, None if self.router is None else ctypes.addressof(self.router),
                      None if SL is None else ctypes.byref(SL), _p(sblob), _p(w_gate), self.ws_ptr, self.ws_bytes,
                      _stream(stream)))
            return out
        if self.shared is not None:
            SL, sblob, w_gate = self.shared
            sblob = sblob if shared_blob is None else shared_blob
            _check(lib().xs_moe_layer_decode_shared(
                ctypes.byref(self.L), _p(arena), self.blob, self.n_expert, self.k, _p(x), _p(logits), _p(residual),
                _p(out), n_tok, ctypes.byref(SL), _p(sblob), _p(w_gate), self.ws_ptr, self.ws_bytes, _stream(stream)))
            return out
        fn = lib().xs_moe_layer_prefill if self.prefill else lib().xs_moe_layer_decode
        _check(fn(ctypes.byref(self.L), _p(arena), self.blob, self.n_expert, self.k, _p(x), _p(logits),
                  _p(residual), _p(out), n_tok, self.ws_ptr, self.ws_bytes, _stream(stream)))
        return out


# ------------------------------------------------------------------------------------------------ tier protocol
# Host buffers are pinned torch tensors (pin_memory=True: hipHostMalloc, device-accessible at the same address);
# device buffers are torch tensors on the GPU or raw addresses (ints).

def wait_flag_ge(flag, value, limit_us=0, status=None, stream=None):
    """Spin (bounded) until flag[0] >= value (include/xs_tiers.h; reference verify_kernels.cpp:783-788)."""
    _check(lib().xs_wait_flag_ge(_p(flag), value, limit_us, _p(status), _stream(stream)))


def copy_i32_from_mapped(dst, src, n, stream=None):
    _check(lib().xs_copy_i32_from_mapped(_p(dst), _p(src), n, _stream(stream)))


def copy_rows_from_mapped(dst, src, rows, width, hit_rows, count, stream=None):
    _check(lib().xs_copy_rows_from_mapped(_p(dst), _p(src), rows, width, _p(hit_rows), _p(count), _stream(stream)))


def fetch_blobs(src, n, dst, blob_bytes, cap, stream=None):
    _check(lib().xs_fetch_blobs(_p(src), _p(n), _p(dst), blob_bytes, cap, _stream(stream)))


def rebase_ptrs(ptr, n, base, blob_bytes, stream=None):
    _check(lib().xs_rebase_ptrs(_p(ptr), _p(n), _p(base), blob_bytes, _stream(stream)))


def moe_hit_add(parts, hit_out, dst, count, cap, n_embd, stream=None):
    _check(lib().xs_moe_hit_add(_p(parts), _p(hit_out), _p(dst), _p(count), cap, n_embd, _stream(stream)))


# ------------------------------------------------------------------------------------------------ native packs

class Pack:
    """A native pack's expert layout (include/xs_pack.h), the reference's ExpertLayout with expert_layout_load,
    expert_layout_from_gguf, check_experts_gguf and load_experts_gguf (src/kernels/cpu/expert_layout.cpp:278-393,
    src/core/expert_source.cpp:2706-2916).  The table lives in the library; load_gguf fills an HBM arena from the
    model's shards in place."""

    def __init__(self, handle):
        self._h = P(handle)

    @classmethod
    def load(cls, pack_dir, n_layers, n_expert, n_embd, n_ff):
        """native_experts.txt of pack_dir (expert_layout_load)."""
        h = P()
        _check(lib().xs_pack_layout_load(str(pack_dir).encode(), n_layers, n_expert, n_embd, n_ff, ctypes.byref(h)))
        return cls(h.value)

    @classmethod
    def from_gguf(cls, gguf, moe_blocks, n_expert, n_embd, n_ff):
        """The routed experts of a GGUF model read in place (expert_layout_from_gguf)."""
        blocks = (I64 * len(moe_blocks))(*moe_blocks)
        h = P()
        _check(lib().xs_pack_layout_from_gguf(str(gguf).encode(), blocks, len(moe_blocks), n_expert, n_embd, n_ff,
                                              ctypes.byref(h)))
        return cls(h.value)

    def __del__(self):
        if getattr(self, "_h", None) and self._h.value and _lib is not None:
            _lib.xs_pack_free(self._h)
            self._h = P()

    def info(self):
        v = PackInfo()
        _check(lib().xs_pack_info(self._h, ctypes.byref(v)))
        return dict(version=v.version, has_gguf_off=bool(v.has_gguf_off), n_layers=v.n_layers, n_expert=v.n_expert,
                    max_blob=v.max_blob, total=v.total)

    def layer(self, l):
        v = PackLayer()
        _check(lib().xs_pack_layer(self._h, l, ctypes.byref(v)))
        return dict(gu_type=v.gu_type, d_type=v.d_type, up_type=v.up_type, block=v.block, offset=v.offset,
                    bytes=v.bytes, up_off=v.up_off, down_off=v.down_off, gguf_off=list(v.gguf_off),
                    gguf_file=[f.decode() for f in v.gguf_file])

    def blob_offset(self, l, e):
        return lib().xs_pack_blob_offset(self._h, l, e)

    def check_gguf(self, native_shard):
        _check(lib().xs_pack_check_gguf(self._h, str(native_shard).encode()))

    def load_gguf(self, native_shard, arena, threads=0):
        """Fill `arena` (a uint8 tensor of at least info()['total'] bytes, on the GPU) from the shards."""
        st = PackLoadStats()
        _check(lib().xs_pack_load_gguf(self._h, str(native_shard).encode(), _p(arena), arena.numel() * arena.element_size(),
                                       threads, ctypes.byref(st)))
        return dict(bytes=st.bytes, layers=st.layers, seconds=st.seconds)

    def load_gguf_layers(self, native_shard, layer_dst, threads=0):
        """Fill one destination per layer (uint8 tensors of n_expert blobs each)."""
        ptrs = (P * len(layer_dst))(*[_p(t) for t in layer_dst])
        st = PackLoadStats()
        _check(lib().xs_pack_load_gguf_layers(self._h, str(native_shard).encode(), ptrs, threads, ctypes.byref(st)))
        return dict(bytes=st.bytes, layers=st.layers, seconds=st.seconds)


# ------------------------------------------------------------------------------------------------ synthetic experts

def fill_layer(out, L, seed, std=0.02, chunk=16):
    """One layer's experts (out: uint8 [n_expert, blob], blob >= L.bytes) from random fp32 N(0, std) weights drawn on
    out's device with a generator seeded by `seed`, quantized with this library's quantizer: each matrix of `chunk`
    experts at once (one draw, one quantization, one strided copy into the blobs).  Same format as build_arena, other
    draws (the weights of `chunk` experts come out of one stream); for building many distinct layers fast."""
    n_expert = out.shape[0]
    g = torch.Generator(device=out.device)
    g.manual_seed(seed)
    for e0 in range(0, n_expert, chunk):
        c = min(chunk, n_expert - e0)
        for off, rows, cols, t in ((0, L.n_ff, L.n_embd, L.gu_type), (L.up_off, L.n_ff, L.n_embd, L.up_type),
                                   (L.down_off, L.n_embd, L.n_ff, L.d_type)):
            w = torch.randn(c * rows, cols, generator=g, device=out.device, dtype=torch.float32) * std
            nbytes = rows * row_bytes(t, cols)
            q = quantize_rows(t, w.reshape(-1))
            out[e0:e0 + c, off:off + nbytes].copy_(q.view(c, nbytes))
            del w, q


def build_arena(n_expert, n_embd, n_ff, gu_type, d_type, seed=0, std=0.02, device="cuda", gen_device="cuda",
                copies=1, up_type=-1):
    """Random fp32 N(0, std) expert weights quantized with this library's quantizer into the native in-place pack
    layout: `copies` x n_expert blobs of [gate rows | up rows | down rows] back to back in one HBM arena (uint8
    [copies * n_expert, blob]).  Weights are drawn with a torch generator seeded by `seed` on `gen_device` ("cpu"
    gives the same bits everywhere); copy c > 0 repeats copy 0's bytes at other addresses (for rotating past the
    caches in timing loops).  up_type >= 0 (not gu_type): a mixed layer, its up rows of that type.  Returns (arena,
    layout)."""
    L = native_expert_layout(gu_type, d_type, n_embd, n_ff, up_type)
    blob = L.bytes
    arena = torch.empty(copies * n_expert, blob, dtype=torch.uint8, device=device)
    g = torch.Generator(device=gen_device)
    g.manual_seed(seed)
    for e in range(n_expert):
        for off, rows, cols, t in ((0, n_ff, n_embd, gu_type), (L.up_off, n_ff, n_embd, L.up_type),
                                   (L.down_off, n_embd, n_ff, d_type)):
            w = torch.randn(rows, cols, generator=g, device=gen_device, dtype=torch.float32) * std
            w = w.to(device)
            nbytes = rows * row_bytes(t, cols)
            quantize_rows(t, w.reshape(-1), out=arena[e, off:off + nbytes])
    for c in range(1, copies):
        arena[c * n_expert:(c + 1) * n_expert].copy_(arena[:n_expert])
    torch.cuda.synchronize()
    return arena, L
