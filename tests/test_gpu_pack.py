"""The native-pack arena filled in HBM (include/xs_pack.h's xs_pack_load_gguf and _layers) from synthetic GGUF shards,
byte for byte against the CPU restatement's assembly (oracle/xs_pack_oracle.py: load_experts_gguf's layout, blob
[gate | up | down] of expert e from byte e * per of each role's tensor) and against the seeded payloads themselves.

Config 2's dimensions (hidden 2048, n_ff 768, Q4_K gate/up, Q6_K down) with 128 experts: each gate and up tensor is
113 MB, more than one 64 MiB staging chunk, so every tensor is read in two chunks; layer 1's gate and up sit in another
shard than its down, as in a split model."""
import pytest
import torch

import gguf_fixture as gf
import xs_pack_oracle as po

pytestmark = pytest.mark.gpu

H, FF, E = 2048, 768, 128
Q4_K, Q6_K, Q8_0 = 12, 14, 8
SEEDS = [(41, 42, 43), (51, 52, 53)]


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    d = tmp_path_factory.mktemp("pack")
    a = gf.write(d / "X-00001-of-00002.gguf", [("blk.0.ffn_gate_exps.weight", [H, FF, E], Q4_K, 41),
                                               ("blk.0.ffn_up_exps.weight", [H, FF, E], Q4_K, 42),
                                               ("blk.0.ffn_down_exps.weight", [FF, H, E], Q6_K, 43),
                                               ("blk.1.ffn_down_exps.weight", [FF, H, E], Q8_0, 53)],
                 kv=[("general.architecture", 8, "qwen4exp")])
    b = gf.write(d / "X-00002-of-00002.gguf", [("blk.1.ffn_gate_exps.weight", [H, FF, E], Q4_K, 51),
                                               ("blk.1.ffn_up_exps.weight", [H, FF, E], Q4_K, 52)], align=64)
    f0 = po.blob_format(Q4_K, Q6_K, Q4_K, H, FF)["bytes"]
    f1 = po.blob_format(Q4_K, Q8_0, Q4_K, H, FF)["bytes"]
    o = lambda w, i: w["data_start"] + w["offsets"][i]
    text = (f"# xestrata native experts xs1: layer gu_type d_type offset blob_bytes gate_off up_off down_off "
            f"[gate,up,down] (n_expert {E}, total {(f0 + f1) * E})\n"
            f"0 12 14 0 {f0} {o(a, 0)} {o(a, 1)} {o(a, 2)}\n"
            f"1 12 8 {f0 * E} {f1} {o(b, 0)} {o(b, 1)} {o(a, 3)} X-00002-of-00002.gguf,X-00002-of-00002.gguf,\n")
    pack = d / "pack"
    pack.mkdir()
    (pack / "native_experts.txt").write_text(text)
    native = str(d / "X-00001-of-00002.gguf")
    pk = po.parse_manifest(text, 2, E, H, FF)
    want = po.assemble(pk, native)
    return pack, native, pk, torch.from_numpy(want)


def test_seeded_payloads_land_in_their_blobs(model):
    pack, native, pk, want = model
    for l, L in enumerate(pk["layers"]):
        per, at = po.per_role(L), po.at_role(L)
        for e in (0, 1, 74, 75, E - 1):   # 75 experts of a gate/up slice fill the first 64 MiB chunk
            for r in range(3):
                o = L["offset"] + e * L["bytes"] + at[r]
                assert torch.equal(want[o:o + per[r]], torch.from_numpy(gf.pattern(SEEDS[l][r], e * per[r], per[r])))


@pytest.mark.parametrize("threads", [1, 3])
def test_load_gguf_into_hbm(xm, model, threads):
    pack, native, pk, want = model
    P = xm.Pack.load(pack, 2, 512, H, FF)
    assert P.info()["n_expert"] == E and P.info()["total"] == want.numel()
    arena = torch.full((want.numel() + 4096,), 0xEE, dtype=torch.uint8, device="cuda")
    st = P.load_gguf(native, arena, threads=threads)
    torch.cuda.synchronize()
    assert st["bytes"] == want.numel() and st["layers"] == 2
    got = arena.cpu()
    assert torch.equal(got[:want.numel()], want), "arena differs from the oracle's assembly"
    assert bool((got[want.numel():] == 0xEE).all()), "the load wrote past the pack's total"
    print(f"\n[pack] {threads} thread(s): {st['bytes'] / 1e6:.0f} MB in {st['seconds'] * 1e3:.1f} ms, "
          f"{st['bytes'] / st['seconds'] / 1e9:.2f} GB/s (page cache to HBM, check included)")


def test_load_gguf_layers_and_from_gguf(xm, model):
    pack, native, pk, want = model
    P = xm.Pack.from_gguf(native, [0, 1], E, H, FF)   # the same table from the model's tensors, no manifest
    assert P.info()["total"] == want.numel()
    dst = [torch.full((L["bytes"] * E,), 0x5A, dtype=torch.uint8, device="cuda") for L in pk["layers"]]
    P.load_gguf_layers(native, dst, threads=2)
    torch.cuda.synchronize()
    for l, L in enumerate(pk["layers"]):
        assert torch.equal(dst[l].cpu(), want[L["offset"]:L["offset"] + L["bytes"] * E]), l


def test_load_refuses_a_small_arena(xm, model):
    pack, native, pk, want = model
    P = xm.Pack.load(pack, 2, 512, H, FF)
    arena = torch.empty(want.numel() - 1, dtype=torch.uint8, device="cuda")
    with pytest.raises(xm.XsError, match="the arena is"):
        P.load_gguf(native, arena)
