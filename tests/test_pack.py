"""The native-pack arena without a GPU (include/xs_pack.h): native_experts.txt tables, the GGUF check, the layout of a
GGUF model's experts, against the CPU restatement (oracle/xs_pack_oracle.py) and the reference's own files.

Mirrors the reference's tests/core/expert_layout_test.cpp: (1) the real packs' tables (tests/golden/native_experts,
copies of the reference's tests/data/native_experts) parse to every field of a plain reading and to the header's
totals; (2) the shard column's forms and refusals; (3) synthetic GGUF shards at the real 2560 x 640 dimensions with a
layer split over two files, then the refusals: an offset that is not the tensor's, a file that does not hold the
tensor, a missing or truncated shard, another type, another shape."""
import ctypes
import pathlib

import pytest

import gguf_fixture as gf
import xs_pack_oracle as po

ROOT = pathlib.Path(__file__).resolve().parent.parent
GOLD = ROOT / "tests" / "golden" / "native_experts"
PACKS = ["q2_0", "iq2_xs", "iq3_xxs", "iq3_s", "coder-iq1_m", "swift-iq2_xs"]
H, FF = 2560, 640
Q4_K, Q5_1, Q5_K, Q8_0, Q3_K, IQ3_S = 12, 7, 13, 8, 11, 21


@pytest.fixture(scope="module")
def xm():
    import xsmoe
    xsmoe.lib()
    return xsmoe


def ref_lib():
    p = ROOT / "oracle" / "_ref" / "libxsref.so"
    if not p.exists():
        pytest.skip("oracle/_ref (the reference's own GGUF reader) is not built here")
    L = ctypes.CDLL(str(p))
    if not hasattr(L, "xsref_gguf_dir"):
        pytest.skip("oracle/_ref predates the GGUF reader entry points")
    L.xsref_type_name.restype = ctypes.c_char_p
    L.xsref_gguf_dir.restype = ctypes.c_int64
    L.xsref_payload_bytes.restype = ctypes.c_uint64
    return L


def plain_reading(text):
    """Each data line split on whitespace (the pre-v4 rules: one shard name for all three roles) and the header's
    "(n_expert N, total T" numbers."""
    rows, hdr = {}, None
    for line in text.splitlines():
        if not line:
            continue
        if line.startswith("#"):
            i = line.find("(n_expert ")
            if i >= 0:
                n, rest = line[i + 10:].split(",", 1)
                hdr = (int(n), int(rest.split()[1].rstrip(";)")))
            continue
        v = line.split()
        rows[int(v[0])] = ([int(x) for x in v[1:8]], v[8] if len(v) > 8 else "")
    return rows, hdr


@pytest.mark.parametrize("pack", PACKS)
def test_real_pack_tables(xm, tmp_path, pack):
    text = (GOLD / f"{pack}.txt").read_text()
    rows, (hdr_n, hdr_total) = plain_reading(text)
    pk = po.parse_manifest(text, 48, 512, H, FF)   # raises when a blob is not what its types make
    assert pk["n_expert"] == hdr_n and pk["total"] == hdr_total
    assert pk["max_blob"] == max(r[0][3] for r in rows.values())
    (tmp_path / "native_experts.txt").write_text(text)
    P = xm.Pack.load(tmp_path, 48, 512, H, FF)
    info = P.info()
    assert (info["n_layers"], info["n_expert"], info["total"], info["max_blob"]) == (48, hdr_n, hdr_total, pk["max_blob"])
    assert info["has_gguf_off"] and info["version"] == int(text.split(" v", 1)[1].split(":")[0])
    for l in range(48):
        (gt, dt, off, blob, go, uo, do), shard = rows[l]
        got = P.layer(l)
        assert (got["gu_type"], got["d_type"], got["up_type"], got["offset"], got["bytes"]) == (gt, dt, gt, off, blob)
        assert got["gguf_off"] == [go, uo, do] and got["gguf_file"] == [shard] * 3
        L = pk["layers"][l]
        assert (got["up_off"], got["down_off"]) == (L["up_off"], L["down_off"])
        assert P.blob_offset(l, 3) == off + 3 * blob
    assert P.blob_offset(48, 0) == 2 ** 64 - 1 and P.blob_offset(0, hdr_n) == 2 ** 64 - 1


def test_type_table_is_the_references():
    L = ref_lib()
    e, b = ctypes.c_int(), ctypes.c_int()
    for t in range(256):
        known = L.xsref_block_geometry(t, ctypes.byref(e), ctypes.byref(b)) == 1
        assert known == (t in po.TYPES), t
        if known:
            assert (e.value, b.value) == po.TYPES[t][:2], t
            assert L.xsref_type_name(t).decode() in (po.TYPES[t][2], "?"), t


def manifest(version, col1, blob, n_expert=2):
    s = (f"# strata native experts v{version}: layer gu_type d_type offset blob_bytes gate_off up_off down_off "
         f"[shard | gate,up,down] (n_expert {n_expert}, total {2 * blob * n_expert})\n")
    s += f"0 12 7 0 {blob} 100 200 300\n"
    s += f"1 12 7 {blob * n_expert} {blob} 400 500 600" + (f" {col1}" if col1 else "") + "\n"
    return s


def load_err(xm, d, text, n_layers=2):
    (d / "native_experts.txt").write_text(text)
    with pytest.raises(xm.XsError) as e:
        xm.Pack.load(d, n_layers, 512, H, FF)
    return str(e.value)


def test_shard_columns(xm, tmp_path):
    blob = po.blob_format(Q4_K, Q5_1, Q4_K, H, FF)["bytes"]
    assert blob == 3_072_000
    (tmp_path / "native_experts.txt").write_text(manifest(4, "B.gguf,B.gguf,", blob))
    P = xm.Pack.load(tmp_path, 2, 512, H, FF)
    assert P.info()["version"] == 4 and P.info()["n_expert"] == 2
    assert P.layer(0)["gguf_file"] == ["", "", ""]
    assert P.layer(1)["gguf_file"] == ["B.gguf", "B.gguf", ""] and P.layer(1)["gguf_off"][2] == 600
    (tmp_path / "native_experts.txt").write_text(manifest(3, "A.gguf", blob))
    assert xm.Pack.load(tmp_path, 2, 512, H, FF).layer(1)["gguf_file"] == ["A.gguf"] * 3
    (tmp_path / "native_experts.txt").write_text(manifest(4, "a - c", blob))
    assert xm.Pack.load(tmp_path, 2, 512, H, FF).layer(1)["gguf_file"] == ["a", "", "c"]
    xs1 = manifest(4, "", blob).replace("# strata native experts v4", "# xestrata native experts xs1")
    (tmp_path / "native_experts.txt").write_text(xs1)
    assert xm.Pack.load(tmp_path, 2, 512, H, FF).info()["version"] == 4
    assert "v5" in load_err(xm, tmp_path, manifest(5, "", blob))
    assert "xs2" in load_err(xm, tmp_path, xs1.replace("xs1", "xs2"))
    assert "gate,up,down" in load_err(xm, tmp_path, manifest(4, "a,b,c,d", blob))
    assert "gate,up,down" in load_err(xm, tmp_path, manifest(4, "a,b", blob))
    assert "gate,up,down" in load_err(xm, tmp_path, manifest(4, "a extra", blob))
    assert "formats make" in load_err(xm, tmp_path, manifest(4, "", blob + 16))
    assert "not contiguous" in load_err(xm, tmp_path, manifest(4, "", blob), n_layers=3)
    assert "malformed" in load_err(xm, tmp_path, manifest(4, "", blob).replace("1 12 7", "2 12 7"))
    for text in (manifest(5, "", blob), manifest(4, "a,b", blob), manifest(4, "", blob + 16)):
        with pytest.raises(po.PackError):
            po.parse_manifest(text, 2, 512, H, FF)
    (tmp_path / "native_experts.txt").unlink()
    with pytest.raises(xm.XsError, match="not a native pack"):
        xm.Pack.load(tmp_path, 2, 512, H, FF)


# ---- synthetic shards: A holds layer 0 and layer 1's down, B layer 1's gate and up
NE = 2
TA = [("blk.0.ffn_gate_exps.weight", [H, FF, NE], Q4_K, 11), ("blk.0.ffn_up_exps.weight", [H, FF, NE], Q4_K, 12),
      ("blk.0.ffn_down_exps.weight", [FF, H, NE], Q5_1, 13), ("blk.1.ffn_down_exps.weight", [FF, H, NE], Q8_0, 23)]
TB = [("blk.1.ffn_gate_exps.weight", [H, FF, NE], Q5_K, 21), ("blk.1.ffn_up_exps.weight", [H, FF, NE], Q5_K, 22)]
KV = [("general.architecture", 8, "qwen4exp"), ("split.no", 2, 1), ("tokenizer.ggml.tokens", 9, (8, ["a", "bc", "def"])),
      ("tokenizer.ggml.scores", 9, (4, [1, 2, 3, 4])), ("split.tensors.count", 5, 6)]


def shards(d, cut_b=0):
    wa = gf.write(d / "M-00002-of-00003.gguf", TA, kv=KV)
    wb = gf.write(d / "M-00003-of-00003.gguf", TB, kv=KV[:1], align=64, cut=cut_b)
    gf.write(d / "M-00001-of-00003.gguf", [], kv=KV)
    return wa, wb


def split_text(wa, wb, down1=None, col1="M-00003-of-00003.gguf,M-00003-of-00003.gguf,"):
    at = lambda w, i: w["data_start"] + w["offsets"][i]
    f0 = po.blob_format(Q4_K, Q5_1, Q4_K, H, FF)["bytes"]
    f1 = po.blob_format(Q5_K, Q8_0, Q5_K, H, FF)["bytes"]
    total = (f0 + f1) * NE
    return (f"# strata native experts v4: layer gu_type d_type offset blob_bytes gate_off up_off down_off "
            f"[shard | gate,up,down] (n_expert {NE}, total {total})\n"
            f"0 12 7 0 {f0} {at(wa, 0)} {at(wa, 1)} {at(wa, 2)}\n"
            f"1 13 8 {f0 * NE} {f1} {at(wb, 0)} {at(wb, 1)} {down1 if down1 is not None else at(wa, 3)} {col1}\n")


def expected_arena(pk):
    """Blob (l, e) = [gate | up | down] of expert e: bytes e * per .. (e + 1) * per of each role's seeded tensor."""
    import numpy as np
    seeds = [(11, 12, 13), (21, 22, 23)]
    out = np.full(pk["total"], 0xEE, dtype=np.uint8)
    for l, L in enumerate(pk["layers"]):
        per, at = po.per_role(L), po.at_role(L)
        for e in range(NE):
            for r in range(3):
                o = L["offset"] + e * L["bytes"] + at[r]
                out[o:o + per[r]] = gf.pattern(seeds[l][r], e * per[r], per[r])
    return out


@pytest.fixture()
def split_pack(tmp_path):
    wa, wb = shards(tmp_path)
    pack = tmp_path / "pack"
    pack.mkdir()
    (pack / "native_experts.txt").write_text(split_text(wa, wb))
    return tmp_path, pack, wa, wb


def test_split_layer_checks_and_assembles(xm, split_pack):
    import numpy as np
    d, pack, wa, wb = split_pack
    native = str(d / "M-00002-of-00003.gguf")
    P = xm.Pack.load(pack, 2, 512, H, FF)
    P.check_gguf(native)
    pk = po.parse_manifest((pack / "native_experts.txt").read_text(), 2, 512, H, FF)
    assert po.check(pk, native) is None
    assert P.info()["total"] == pk["total"] == 2 * 3_072_000 + 2 * po.blob_format(Q5_K, Q8_0, Q5_K, H, FF)["bytes"]
    assert np.array_equal(po.assemble(pk, native), expected_arena(pk))


def test_gguf_directory_is_the_references(split_pack):
    L = ref_lib()
    d = split_pack[0]
    for name in ("M-00001-of-00003.gguf", "M-00002-of-00003.gguf", "M-00003-of-00003.gguf"):
        p = str(d / name).encode()
        ds, size, err = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.create_string_buffer(256)
        n = L.xsref_gguf_dir(p, ctypes.byref(ds), ctypes.byref(size), err, 256)
        mine = po.gguf_directory(d / name)
        assert n == len(mine[2]) and (ds.value, size.value) == mine[:2], err.value
        for i in range(n):
            nm, t, nd = ctypes.create_string_buffer(128), ctypes.c_uint32(), ctypes.c_uint32()
            shape, off = (ctypes.c_uint64 * 4)(), ctypes.c_uint64()
            assert L.xsref_gguf_tensor(p, i, nm, 128, ctypes.byref(t), ctypes.byref(nd), shape, ctypes.byref(off)) == 0
            want = mine[2][nm.value.decode()]
            assert (t.value, list(shape)[:nd.value], off.value) == (want[0], want[1], want[2])
            assert L.xsref_payload_bytes(t, shape, nd) == po.payload_bytes(want[0], want[1])
        out = ctypes.create_string_buffer(4096)
        assert L.xsref_split_paths(p, out, 4096) == 0
        assert out.value.decode().split() == po.split_paths(str(d / name))


def refused(xm, pack, native, text):
    (pack / "native_experts.txt").write_text(text)
    P = xm.Pack.load(pack, 2, 512, H, FF)
    with pytest.raises(xm.XsError) as e:
        P.check_gguf(native)
    pk = po.parse_manifest(text, 2, 512, H, FF)
    return str(e.value), po.check(pk, native)


def test_refusals(xm, split_pack):
    d, pack, wa, wb = split_pack
    native = str(d / "M-00002-of-00003.gguf")
    both = "M-00003-of-00003.gguf,M-00003-of-00003.gguf,"
    lib_msg, ora = refused(xm, pack, native, split_text(wa, wb, down1=wa["data_start"] + wa["offsets"][3] + 32))
    assert "starts at byte" in lib_msg and "starts at byte" in ora
    lib_msg, ora = refused(xm, pack, native, split_text(wa, wb, col1=""))
    assert "blk.1.ffn_gate_exps.weight" in lib_msg and "is not in it" in lib_msg and "is not in it" in ora
    lib_msg, ora = refused(xm, pack, native, split_text(wa, wb, col1="missing.gguf,missing.gguf,"))
    assert "cannot open" in lib_msg and "cannot open" in ora
    (pack / "native_experts.txt").write_text(split_text(wa, wb, col1=both + ",x"))
    with pytest.raises(xm.XsError, match="gate,up,down"):
        xm.Pack.load(pack, 2, 512, H, FF)
    shards(d, cut_b=100)
    lib_msg, ora = refused(xm, pack, native, split_text(wa, wb))
    assert "past the end" in lib_msg and "past the end" in ora
    # the load refuses the same table before it reads a byte (no arena is touched: a NULL-free dummy address)
    P = xm.Pack.load(pack, 2, 512, H, FF)
    with pytest.raises(xm.XsError, match="past the end"):
        st = xm.PackLoadStats()
        xm._check(xm.lib().xs_pack_load_gguf(P._h, native.encode(), 1 << 40, P.info()["total"], 1, ctypes.byref(st)))


def test_type_and_shape_refusals(xm, tmp_path):
    # Q3_K and IQ3_S are both 110 B a 256 values, so only the type differs
    f2 = po.blob_format(Q3_K, Q5_1, Q3_K, H, FF)["bytes"]
    c = tmp_path / "C.gguf"
    pack = tmp_path / "pack"
    pack.mkdir()

    def table(w):
        o = [w["data_start"] + x for x in w["offsets"]]
        return f"# strata native experts v3: (n_expert 2, total {f2 * NE})\n0 11 7 0 {f2} {o[0]} {o[1]} {o[2]}\n"

    w = gf.write(c, [("blk.0.ffn_gate_exps.weight", [H, FF, NE], IQ3_S, 31),
                     ("blk.0.ffn_up_exps.weight", [H, FF, NE], Q3_K, 32),
                     ("blk.0.ffn_down_exps.weight", [FF, H, NE + 1], Q5_1, 33)])
    (pack / "native_experts.txt").write_text(table(w))
    P = xm.Pack.load(pack, 1, 512, H, FF)
    with pytest.raises(xm.XsError, match="is IQ3_S"):
        P.check_gguf(str(c))
    assert "is IQ3_S" in po.check(po.parse_manifest(table(w), 1, 512, H, FF), str(c))
    w = gf.write(c, [("blk.0.ffn_gate_exps.weight", [H, FF, NE], Q3_K, 31),
                     ("blk.0.ffn_up_exps.weight", [H, FF, NE], Q3_K, 32),
                     ("blk.0.ffn_down_exps.weight", [FF, H, NE + 1], Q5_1, 33)])
    (pack / "native_experts.txt").write_text(table(w))
    P = xm.Pack.load(pack, 1, 512, H, FF)
    with pytest.raises(xm.XsError, match=r"is not \[640, 2560, 2\]"):
        P.check_gguf(str(c))
    assert "is not [640, 2560, 2]" in po.check(po.parse_manifest(table(w), 1, 512, H, FF), str(c))


def test_layout_from_gguf(xm, split_pack):
    d, pack, wa, wb = split_pack
    ref = xm.Pack.load(pack, 2, 512, H, FF)
    for any_shard in ("M-00001-of-00003.gguf", "M-00003-of-00003.gguf"):
        P = xm.Pack.from_gguf(d / any_shard, [0, 1], NE, H, FF)
        pk = po.from_gguf(str(d / any_shard), [0, 1], NE, H, FF)
        assert P.info()["total"] == ref.info()["total"] == pk["total"]
        assert P.info()["version"] == 0 and P.info()["has_gguf_off"]
        for l in range(2):
            got, want = P.layer(l), ref.layer(l)
            for k in ("gu_type", "d_type", "up_type", "offset", "bytes", "up_off", "down_off", "gguf_off", "block"):
                assert got[k] == want[k], (l, k)
            assert got["gguf_off"] == pk["gguf_off"][3 * l:3 * l + 3]
            assert got["gguf_file"] == pk["gguf_file"][3 * l:3 * l + 3]
        assert P.layer(1)["gguf_file"] == ["M-00003-of-00003.gguf", "M-00003-of-00003.gguf", "M-00002-of-00003.gguf"]
        P.check_gguf(d / "M-00002-of-00003.gguf")
    # layer 1 is block 1; asking for a block the model does not have, a shape it does not have, or a missing shard
    with pytest.raises(xm.XsError, match=r"blk\.2\.ffn_gate_exps\.weight is missing"):
        xm.Pack.from_gguf(d / "M-00002-of-00003.gguf", [0, 2], NE, H, FF)
    with pytest.raises(xm.XsError, match=r"is missing or not \[2560, 640, 3\]"):
        xm.Pack.from_gguf(d / "M-00002-of-00003.gguf", [0, 1], NE + 1, H, FF)
    (d / "M-00003-of-00003.gguf").unlink()
    with pytest.raises(xm.XsError, match="missing model shard"):
        xm.Pack.from_gguf(d / "M-00002-of-00003.gguf", [0, 1], NE, H, FF)
