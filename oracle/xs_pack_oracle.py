"""CPU restatement of the reference's native-pack arena: native_experts.txt's table, the GGUF tensor directory, the
check of the table against the model's shards, and the arena assembled from them.  TEST INFRASTRUCTURE: only tests/
may import this module, and only as the checker of include/xs_pack.h's library calls.

Restates, in plain Python:
  - parse_manifest: expert_layout_load (src/kernels/cpu/expert_layout.cpp:278-393);
  - gguf_directory: GgufFile::parse (include/strata/artifact/gguf_reader.hpp:427-474) and gguf_split_paths
    (include/strata/artifact/gguf_split.hpp:26-53);
  - check: check_experts_gguf (src/core/expert_source.cpp:2784-2841);
  - from_gguf: expert_layout_from_gguf (src/core/expert_source.cpp:2706-2782);
  - assemble: load_experts_gguf (src/core/expert_source.cpp:2843-2916): every blob [gate | up | down], expert e's slice
    of a role taken from byte e * per of that role's tensor.
Pinned by the reference's own pack tables (tests/golden/native_experts: every blob size against the types, every
field against a plain whitespace reading of the line, totals against the header) and, where oracle/_ref builds, by
the reference's GGUF reader and block geometry on the same files.
"""
import os
import re
import struct

import numpy as np

# ggml type id -> (values per block, bytes per block, name); 42 is Strata's Q2_0.  The set the reference's GGUF reader
# gives a block geometry (include/strata/artifact/gguf_reader.hpp:124-260).
TYPES = {
    0: (1, 4, "F32"), 1: (1, 2, "F16"), 2: (32, 18, "Q4_0"), 3: (32, 20, "Q4_1"), 6: (32, 22, "Q5_0"),
    7: (32, 24, "Q5_1"), 8: (32, 34, "Q8_0"), 9: (32, 36, "Q8_1"), 10: (256, 84, "Q2_K"), 11: (256, 110, "Q3_K"),
    12: (256, 144, "Q4_K"), 13: (256, 176, "Q5_K"), 14: (256, 210, "Q6_K"), 16: (256, 66, "IQ2_XXS"),
    17: (256, 74, "IQ2_XS"), 18: (256, 98, "IQ3_XXS"), 20: (32, 18, "IQ4_NL"), 21: (256, 110, "IQ3_S"),
    22: (256, 82, "IQ2_S"), 23: (256, 136, "IQ4_XS"), 24: (1, 1, "I8"), 29: (256, 56, "IQ1_M"), 30: (1, 2, "BF16"),
    42: (64, 18, "Q2_0"),
}
ROLES = ("gate", "up", "down")


class PackError(ValueError):
    pass


def row_bytes(t, n):
    if t not in TYPES or n <= 0 or n % TYPES[t][0]:
        return 0
    return n // TYPES[t][0] * TYPES[t][1]


def payload_bytes(t, shape):
    if t not in TYPES or not shape or shape[0] % TYPES[t][0] or any(d == 0 for d in shape):
        return 0
    n = 1
    for d in shape:
        n *= d
    return n // TYPES[t][0] * TYPES[t][1]


def blob_format(gu, d, up, n_embd, n_ff):
    """[n_ff gate rows | n_ff up rows | n_embd down rows] of raw blocks (native_fmt's offsets)."""
    gr, ur, dr = row_bytes(gu, n_embd), row_bytes(up, n_embd), row_bytes(d, n_ff)
    if not (gr and ur and dr):
        raise PackError(f"no block geometry for types {gu}/{up}/{d} at {n_embd} x {n_ff}")
    up_off = n_ff * gr
    down_off = up_off + n_ff * ur
    return dict(gu_type=gu, d_type=d, up_type=up, up_off=up_off, down_off=down_off, bytes=down_off + n_embd * dr)


def per_role(layer):
    return (layer["up_off"], layer["down_off"] - layer["up_off"], layer["bytes"] - layer["down_off"])


def at_role(layer):
    return (0, layer["up_off"], layer["down_off"])


def parse_manifest(text, n_layers, n_expert, n_embd, n_ff):
    """native_experts.txt -> dict(version, n_expert, layers[], gguf_off (3 per layer or None), gguf_file, total,
    max_blob).  Follows expert_layout.cpp:278-393."""
    pk = dict(version=0, n_expert=n_expert, layers=[None] * n_layers, gguf_off=None, gguf_file=None)
    max_blob = 0
    for line in text.split("\n"):
        line = line.rstrip("\r")
        if not line:
            continue
        if line.startswith("#"):
            m = re.match(r"# strata native experts v(\d+)", line)
            x = re.match(r"# xestrata native experts xs(\d+)", line)
            if m or x:
                v = int((m or x).group(1))
                pk["version"] = v if m else 4
                if v > (4 if m else 1):
                    raise PackError(f"native_experts.txt is {'v' if m else 'xs'}{v}")
            at = line.find("(n_expert ")
            if at >= 0:
                pk["n_expert"] = int(re.match(r"\d+", line[at + 10:]).group(0))
            continue
        tok = line.split()
        try:
            l, gt, dt, off, blob = (int(v) for v in tok[:5])
        except ValueError:
            raise PackError("a malformed line: " + line)
        if len(tok) < 5 or not 0 <= l < n_layers:
            raise PackError("a malformed line: " + line)
        f = blob_format(gt, dt, gt, n_embd, n_ff)
        if f["bytes"] != blob:
            raise PackError(f"layer {l} blob is {blob} B but its formats make {f['bytes']}")
        rest = tok[5:]
        if len(rest) >= 3 and all(v.isdigit() for v in rest[:3]):
            if pk["gguf_off"] is None:
                pk["gguf_off"] = [0] * (3 * n_layers)
            pk["gguf_off"][3 * l:3 * l + 3] = [int(v) for v in rest[:3]]
            files = rest[3:]
            if len(files) == 1 and "," in files[0]:
                files = files[0].split(",")
            files = ["" if v == "-" else v for v in files]
            if len(files) == 1:
                files = files * 3
            if files and len(files) != 3:
                raise PackError(f"layer {l}: the shard column is one name, gate,up,down or three names")
            if files:
                if pk["gguf_file"] is None:
                    pk["gguf_file"] = [""] * (3 * n_layers)
                pk["gguf_file"][3 * l:3 * l + 3] = files
        f.update(block=l, offset=off)
        pk["layers"][l] = f
        max_blob = max(max_blob, blob)
    at = 0
    for l, L in enumerate(pk["layers"]):
        if L is None or L["offset"] != at:
            raise PackError(f"layer {l} is missing or not contiguous")
        at += L["bytes"] * pk["n_expert"]
    pk.update(total=at, max_blob=max_blob, n_embd=n_embd, n_ff=n_ff)
    return pk


def gguf_directory(path):
    """(data_start, file_size, {name: (type, shape, offset)}) of a GGUF v3 file (header and directory only)."""
    with open(path, "rb") as f:
        size = os.fstat(f.fileno()).st_size

        def rd(fmt):
            n = struct.calcsize(fmt)
            b = f.read(n)
            if len(b) != n:
                raise PackError(f"{path}: the header runs past the end of the file")
            return struct.unpack("<" + fmt, b)[0]

        def rstr():
            return f.read(rd("Q")).decode()

        scal = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "B", 10: "Q", 11: "q", 12: "d"}

        def value(t):
            if t == 8:
                return rstr()
            if t == 9:
                et, n = rd("I"), rd("Q")
                return [value(et) for _ in range(n)]
            return rd(scal[t])

        if rd("I") != 0x46554747:
            raise PackError(f"{path}: not a GGUF file")
        if rd("I") != 3:
            raise PackError(f"{path}: not GGUF v3")
        n_t, n_kv = rd("Q"), rd("Q")
        align = 32
        for _ in range(n_kv):
            key = rstr()
            v = value(rd("I"))
            if key == "general.alignment" and isinstance(v, int) and v:
                align = v
        tensors = {}
        for _ in range(n_t):
            name = rstr()
            nd = rd("I")
            shape = [rd("Q") for _ in range(nd)]
            tensors[name] = (rd("I"), shape, rd("Q"))
        data_start = (f.tell() + align - 1) // align * align
        if data_start > size:
            if n_t:
                raise PackError(f"{path}: the data section starts past the end")
            data_start = size
    return data_start, size, tensors


def split_paths(any_shard):
    m = re.match(r"^(.*-)(\d{5})(-of-)(\d{5})(\.gguf)$", any_shard)
    if not m or not 1 <= int(m.group(2)) <= int(m.group(4)):
        return [any_shard]
    n = int(m.group(4))
    return [f"{m.group(1)}{i:05d}{m.group(3)}{m.group(4)}{m.group(5)}" for i in range(1, n + 1)]


def file_of(pk, native, l, r):
    if not pk["gguf_file"] or not pk["gguf_file"][3 * l + r]:
        return native
    return os.path.join(os.path.dirname(native), pk["gguf_file"][3 * l + r])


def check(pk, native):
    """None when every (layer, role) tensor matches the table, else the reason (check_experts_gguf's order)."""
    if pk["gguf_off"] is None:
        return "no GGUF offsets"
    dirs = {}
    for l, L in enumerate(pk["layers"]):
        per = per_role(L)
        for r in range(3):
            path = file_of(pk, native, l, r)
            if path not in dirs:
                if not os.path.exists(path):
                    return f"cannot open {path}"
                dirs[path] = gguf_directory(path)
            ds, size, ts = dirs[path]
            name = f"blk.{L['block']}.ffn_{ROLES[r]}_exps.weight"
            want_t = (L["gu_type"], L["up_type"], L["d_type"])[r]
            cols, rows = (pk["n_embd"], pk["n_ff"]) if r < 2 else (pk["n_ff"], pk["n_embd"])
            nbytes = per[r] * pk["n_expert"]
            if name not in ts:
                return f"{name} is not in it"
            t, shape, off = ts[name]
            if t != want_t:
                return f"{name} is {TYPES[t][2] if t in TYPES else t}, the pack says type {want_t}"
            if shape != [cols, rows, pk["n_expert"]]:
                return f"{name} is not [{cols}, {rows}, {pk['n_expert']}]"
            if payload_bytes(t, shape) != nbytes:
                return f"{name} is not {per[r]} B per expert"
            if ds + off != pk["gguf_off"][3 * l + r]:
                return f"{name} starts at byte {ds + off}, the pack says {pk['gguf_off'][3 * l + r]}"
            if off > size - ds or nbytes > size - ds - off:
                return f"{name} runs past the end of the file"
    return None


def from_gguf(gguf, moe_blocks, n_expert, n_embd, n_ff):
    """The table of a GGUF model's expert tensors (expert_layout_from_gguf)."""
    where = {}
    dirs = []
    for p in split_paths(gguf):
        dirs.append((p, gguf_directory(p)))
        for name in dirs[-1][1][2]:
            if name in where:
                raise PackError(f"tensor {name} is in two shards")
            where[name] = len(dirs) - 1
    n = len(moe_blocks)
    pk = dict(version=0, n_expert=n_expert, layers=[], gguf_off=[0] * (3 * n), gguf_file=[""] * (3 * n),
              n_embd=n_embd, n_ff=n_ff)
    at = 0
    for l, b in enumerate(moe_blocks):
        found = []
        for r in range(3):
            name = f"blk.{b}.ffn_{ROLES[r]}_exps.weight"
            cols, rows = (n_embd, n_ff) if r < 2 else (n_ff, n_embd)
            if name not in where:
                raise PackError(f"{name} is missing")
            p, (ds, size, ts) = dirs[where[name]]
            t, shape, off = ts[name]
            if shape != [cols, rows, n_expert]:
                raise PackError(f"{name} is not [{cols}, {rows}, {n_expert}]")
            found.append((p, ds, t, shape, off))
        f = blob_format(found[0][2], found[2][2], found[1][2], n_embd, n_ff)
        per = per_role(f)
        for r, (p, ds, t, shape, off) in enumerate(found):
            if payload_bytes(t, shape) != per[r] * n_expert:
                raise PackError(f"block {b}'s {ROLES[r]} tensor is not {per[r]} B per expert")
            pk["gguf_off"][3 * l + r] = ds + off
            pk["gguf_file"][3 * l + r] = os.path.basename(p)
        f.update(block=b, offset=at)
        pk["layers"].append(f)
        at += f["bytes"] * n_expert
    pk.update(total=at, max_blob=max(L["bytes"] for L in pk["layers"]))
    return pk


def assemble(pk, native):
    """The arena as uint8: blob (l, e) at layers[l].offset + e * bytes holds [gate | up | down] of expert e."""
    out = np.zeros(pk["total"], dtype=np.uint8)
    E = pk["n_expert"]
    for l, L in enumerate(pk["layers"]):
        per, at = per_role(L), at_role(L)
        for r in range(3):
            with open(file_of(pk, native, l, r), "rb") as f:
                f.seek(pk["gguf_off"][3 * l + r])
                src = np.frombuffer(f.read(per[r] * E), dtype=np.uint8)
            if src.size != per[r] * E:
                raise PackError("short read")
            for e in range(E):
                o = L["offset"] + e * L["bytes"] + at[r]
                out[o:o + per[r]] = src[e * per[r]:(e + 1) * per[r]]
    return out
