"""Regenerate tests/golden/*.npz.  Run in the build container (it needs the reference tree for oracle/_ref):

    python tests/golden/make_golden.py

  reference_vectors.npz - outputs of the reference's OWN host code, compiled from include/strata/artifact/dequant.hpp
      and include/strata/kernels/canon_math.hpp where they lie (oracle/_ref, built by oracle/Makefile): dequantized
      Q8_0 / Q4_K / Q6_K / IQ4_XS blocks, fp16 -> fp32 for all 65536 halves, canon exp / rcp / silu_mul.
  seeded_inputs.npz     - the reference parity tests' seeded inputs (tests/golden/seeded_inputs.cpp).
Inputs are data and outputs are data: no reference source is copied into the repository.
"""
import pathlib
import subprocess
import sys
import tempfile

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT / "oracle"))
import xs_oracle as xo  # noqa: E402


def blocks(rng, t, nb):
    """Random blocks of type t with finite, realistic fp16 scales (and a few edge values)."""
    bs = xo.BLOCK_BYTES[t]
    b = rng.integers(0, 256, size=(nb, bs), dtype=np.uint8)
    d = (rng.standard_normal(nb) * 0.01).astype(np.float16)
    d[:4] = np.array([0.0, -0.0, 6.0e-8, 65504.0], np.float16)       # zero, signed zero, subnormal, max
    dm = np.abs(rng.standard_normal(nb) * 0.01).astype(np.float16)
    if t == xo.Q6_K:
        b[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    else:
        b[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    if t == xo.Q4_K:
        b[:, 2:4] = dm.view(np.uint8).reshape(nb, 2)
    return b


def main():
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    R = xo.ref()
    if R is None:
        sys.exit("oracle/_ref/libxsref.so is not built (the reference tree is absent)")
    rng = np.random.default_rng(20261201)
    out = {}
    for t in (xo.Q8_0, xo.Q4_K, xo.Q6_K, xo.IQ4_XS):
        nb = 96
        b = blocks(rng, t, nb)
        y = np.zeros(nb * xo.BLOCK_VALUES[t], np.float32)
        assert R.xsref_dequant(t, xo._a(b), nb, xo._a(y)) == 0
        out[f"blocks_{t}"] = b
        out[f"dequant_{t}"] = y
    out["fp16_to_fp32"] = np.array([R.xsref_fp16_to_fp32(h) for h in range(65536)], np.float32)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32) * 20,
                        np.array([-90, -80, -79.9, -0.0, 0.0, 1e-30, 80, 88.7, 100], np.float32)])
    y = np.empty_like(x)
    R.xsref_canon_exp(xo._a(x), x.size, xo._a(y))
    out["canon_exp_x"], out["canon_exp_y"] = x, y
    r = np.abs(rng.standard_normal(4096).astype(np.float32)) * np.exp(rng.uniform(-20, 20, 4096)).astype(np.float32)
    r = r.astype(np.float32) + np.float32(1e-6)
    y = np.empty_like(r)
    R.xsref_canon_rcp(xo._a(r), r.size, xo._a(y))
    out["canon_rcp_x"], out["canon_rcp_y"] = r, y
    g = (rng.standard_normal(4096) * 6).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    h = np.empty_like(g)
    R.xsref_canon_silu_mul(xo._a(g), xo._a(u), g.size, xo._a(h))
    out["silu_g"], out["silu_u"], out["silu_h"] = g, u, h
    # canon q8_scale / q8_inv / q8_value over whole blocks (one scale a block): 256- and 32-value blocks of normal
    # data at magnitudes from 1e-3 to 1e5, plus the edges - an all-zero block, amax below the 1e-30 inverse cut
    # (1e-29 and 1e-28 / 127), amax past 65504 * 127 = 8.3e6 (the scale held at 65504 and the values at +-127),
    # signed zeros, values at exact .5 steps of the scale
    q8_x, q8_d, q8_id, q8_q, q8_n = [], [], [], [], []
    def q8_block(v):
        v = np.ascontiguousarray(v, np.float32)
        d = np.zeros(1, np.float32)
        i = np.zeros(1, np.float32)
        q = np.zeros(v.size, np.int8)
        R.xsref_canon_q8(xo._a(v), v.size, xo._a(d), xo._a(i), xo._a(q))
        q8_x.append(v)
        q8_d.append(d[0])
        q8_id.append(i[0])
        q8_q.append(q)
        q8_n.append(v.size)
    for n in (256, 32):
        for mag in (1e-3, 0.02, 1.0, 30.0, 1e5):
            for _ in range(24):
                q8_block(rng.standard_normal(n) * mag)
        q8_block(np.zeros(n))
        q8_block(np.full(n, -0.0))
        q8_block(rng.standard_normal(n) * 1e-29)
        q8_block(np.linspace(-1.27e-28, 1.27e-28, n))
        big = rng.standard_normal(n) * 1e3
        big[3] = 9.0e6
        q8_block(big)
        big2 = rng.standard_normal(n) * 3e6
        big2[0] = -2.0e7
        q8_block(big2)
        steps = (np.arange(n) - n // 2 + 0.5) * (127.0 / (n // 2 + 0.5))   # values near the .5 rounding edges
        q8_block(steps)
    out["q8_n"] = np.array(q8_n, np.int32)
    out["q8_x"] = np.concatenate(q8_x)
    out["q8_d"] = np.array(q8_d, np.float32)
    out["q8_id"] = np.array(q8_id, np.float32)
    out["q8_q"] = np.concatenate(q8_q)
    # bf16_from_f32 (bf16_bits.hpp): random magnitudes, exact ties on both parities, the carry into the exponent, the
    # largest finite values (rounding to inf), NaNs whose rounding add would carry, infinities, zeros, subnormals
    rb = np.random.default_rng(20261202)
    bits = np.concatenate([
        (rb.standard_normal(4096) * np.exp(rb.uniform(-40, 40, 4096))).astype(np.float32).view(np.uint32),
        np.array([0x3F808000, 0x3F818000, 0xBF808000, 0xBF818000, 0x3F7FFFFF, 0x3F7F8000, 0x7F7FFFFF, 0x7F7F8000,
                  0xFF7FFFFF, 0x7F7F7FFF, 0x7FFFFFFF, 0x7F800001, 0xFFC00001, 0x7FC00000, 0xFF800001, 0x7F800000,
                  0xFF800000, 0x00000000, 0x80000000, 0x00008000, 0x00018000, 0x00000001, 0x807FFFFF], np.uint32),
        rb.integers(0, 2**32, 1024, dtype=np.uint64).astype(np.uint32)])
    bx = bits.view(np.float32)
    by = np.zeros(bx.size, np.uint16)
    R.xsref_bf16_from_f32(xo._a(bx), bx.size, xo._a(by))
    out["bf16_x"], out["bf16_y"] = bx, by
    np.savez_compressed(HERE / "reference_vectors.npz", **out)

    with tempfile.TemporaryDirectory() as tmp:
        exe = pathlib.Path(tmp) / "seeded"
        subprocess.run(["g++", "-O2", "-std=c++17", "-o", str(exe), str(HERE / "seeded_inputs.cpp")], check=True)
        subprocess.run([str(exe), tmp], check=True)
        seeded = dict(router_cases=np.fromfile(pathlib.Path(tmp) / "router_cases.f32", np.float32).reshape(-1, 512),
                      plan_ids=np.fromfile(pathlib.Path(tmp) / "plan_ids.i32", np.int32),
                      router256=np.fromfile(pathlib.Path(tmp) / "router256.f32", np.float32).reshape(3, 256))
    np.savez_compressed(HERE / "seeded_inputs.npz", **seeded)
    print("wrote", HERE / "reference_vectors.npz", HERE / "seeded_inputs.npz")


if __name__ == "__main__":
    main()
