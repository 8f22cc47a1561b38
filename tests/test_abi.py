"""The C ABI without a GPU: libxsmoe.so loads and exports every symbol include/xs_moe.h declares; geometry helpers
agree with the reference's formulas; argument checks fail with the reference's messages before any launch."""
import ctypes
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def xm():
    import xsmoe
    return xsmoe


def declared_symbols():
    text = "".join(h.read_text() for h in sorted((ROOT / "include").glob("*.h")))
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(xs_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol(xm):
    lib = xm.lib()
    names = declared_symbols()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_header(xm):
    assert set(declared_symbols()) == set(xm._SIGS)


# the native blob sizes of the five BASELINE configs (gate | up | down, raw GGUF blocks)
@pytest.mark.parametrize("gu,d,H,F,blob", [(8, 8, 1024, 512, 1_671_168), (12, 14, 2048, 768, 3_059_712),
                                           (23, 23, 4096, 1536, 10_027_008), (12, 12, 7168, 2048, 24_772_608),
                                           (8, 8, 7168, 2048, 46_792_704)])
def test_layout(xm, gu, d, H, F, blob):
    L = xm.native_expert_layout(gu, d, H, F)
    assert L.bytes == blob
    assert L.gu_row == H // xm.BLOCK_VALUES[gu] * xm.BLOCK_BYTES[gu]
    assert L.up_off == F * L.gu_row and L.down_off == 2 * F * L.gu_row
    assert L.bytes % 16 == 0


def test_supported(xm):
    assert xm.native_expert_supported(12, 14, 2048, 768)
    assert not xm.native_expert_supported(12, 14, 2048 + 32, 768)       # n_embd not a whole number of 256s
    assert not xm.native_expert_supported(12, 14, 2048, 700)             # down rows not whole Q6_K blocks
    assert not xm.native_expert_supported(2, 14, 2048, 768)              # Q4_0: not one of the four formats
    # a mixed layer: gate and up each a gate/up type of its own (iq_kernels.cpp:2003-2005)
    assert xm.native_expert_supported(12, 14, 2048, 768, up=14)
    assert xm.native_expert_supported(14, 14, 2048, 768, up=8)
    assert not xm.native_expert_supported(12, 14, 2048, 768, up=2)       # Q4_0 up rows: not one of the formats
    assert not xm.native_expert_supported(8, 14, 1024 + 32, 768, up=12)  # n_embd not whole Q4_K blocks for the up rows


def test_mixed_layout(xm, xo):
    """The mixed layout (native_expert_layout with up_type, iq_kernels.cpp:2021-2036): gate rows of the gate's row
    bytes, then up rows of the up type's, then down rows; the same offsets as the oracle's restatement."""
    for gu, up, d, H, F in ((12, 14, 14, 2048, 768), (14, 8, 12, 1024, 512), (8, 23, 8, 4096, 256)):
        L = xm.native_expert_layout(gu, d, H, F, up)
        assert (L.gu_type, L.up_type, L.d_type) == (gu, up, d)
        assert L.gu_row == xm.row_bytes(gu, H) and L.up_row == xm.row_bytes(up, H) and L.d_row == xm.row_bytes(d, F)
        assert L.up_off == F * L.gu_row and L.down_off == L.up_off + F * L.up_row and L.bytes == L.down_off + H * L.d_row
        O = xo.layout(gu, d, H, F, up)
        assert (O.up_off, O.down_off, O.bytes, O.up_row) == (L.up_off, L.down_off, L.bytes, L.up_row)
    same = xm.native_expert_layout(12, 14, 2048, 768)
    assert same.up_type == 12 and same.up_row == same.gu_row


def test_scratch_bytes(xm):
    # the reference's gate | up | h | hq areas (iq_kernels.cpp:2037-2040) plus the 256-byte status area
    cap, F = 8, 768
    f = cap * F * 4
    up = lambda v: (v + 255) & ~255
    assert xm.native_expert_scratch_bytes(cap, F) == 3 * up(f) + up(cap * (F // 32) * 36) + 256


def test_plan_offsets(xm):
    capx = 80
    o = xm.plan_offsets(capx)
    ptr_off = ((4 + (capx + 1) + 2 * capx) + 1) & ~1      # verify_kernels.cpp:860-866
    assert o == dict(start=4, dst=4 + capx + 1, tok=4 + 2 * capx + 1, ptr=ptr_off, start2=ptr_off + 4 * capx)


def test_argument_errors(xm):
    lib = xm.lib()
    # k past 64, checked before any launch (router.cpp:294)
    assert lib.xs_router_top10(8, 1, 128, 65, 8, 8, None) == xm.XS_EINVAL
    assert b"exceeds the kernel's 64" in lib.xs_last_error()
    # the combine's k range is 1..15
    assert lib.xs_native_moe_combine_multi(8, 8, None, 8, 2048, 16, 1, 8, None) == xm.XS_EINVAL
    # an unsupported layout
    L = xm.Layout()
    L.gu_type, L.d_type, L.up_type, L.n_embd, L.n_ff = 2, 14, -1, 2048, 768
    assert lib.xs_native_expert_grouped(ctypes.byref(L), 8, 8, 8, 8, 8, 1, 1, 8, 16, 8, None, 0) == xm.XS_EINVAL
    # resident_plan: more entries than a work-group
    assert lib.xs_resident_plan(8, 2000, 8, None, 128, None, None, 16, 8, 4000, 8, 1, 8) == xm.XS_EINVAL


def test_mmq_grouped_refusals(xm):
    """iq_mmq_grouped refuses, before any device call, the types its products do not decode, widths its tiles do not
    cover, a dst row narrower than the weights' rows and missing spans; n = 0 or no rows is a no-op."""
    lib = xm.lib()
    E = xm.XS_EINVAL
    args = dict(w=16, eb=4096, wr=512, wc=2048, n=4, xq=16, tot=64, b=16, mr=64, ids=16, dst=16, ld=512, wt=None,
                wo=0, rows=0)

    def call(t, **kw):
        a = dict(args, **kw)
        return lib.xs_iq_mmq_grouped(t, a["w"], a["eb"], a["wr"], a["wc"], a["n"], a["xq"], a["tot"], a["b"], a["mr"],
                                     a["ids"], a["dst"], a["ld"], a["wt"], a["wo"], a["rows"], None)
    assert call(10) == E                        # Q2_K: not among this build's products
    assert "ggml type 10" in lib.xs_last_error().decode()
    assert call(12, wc=2000) == E               # columns not a multiple of 256
    assert call(12, wr=384) == E                # Q4_K rows: tiles of 256
    assert call(12, ld=256) == E                # dst rows narrower than the weights' rows
    assert call(12, ids=None) == E
    assert call(12, w=None) == E                # neither w nor wtab
    assert call(12, n=0) == xm.XS_OK
    assert call(12, tot=0) == xm.XS_OK
