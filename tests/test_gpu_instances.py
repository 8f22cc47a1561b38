"""Kernel instances the bench times, each against the CPU oracle bit for bit on the same seeded inputs:

* config 1's one-token instance (moe_decode_t1_kernel, Q8_0, hidden 1024, F 512, 8 experts, top-2) - the bench's
  cpu_baseline line at T=1 runs it;
* the one-token kernel's router widths at config 2's expert shape (Q4_K / Q6_K, hidden 2048, F 768, top-8): PER = 1
  (64 experts), PER = 2 (128, config 2 itself, tested in test_gpu_layer.py) and PER = 4 (256);
* the one-token kernel's instance for config 2's shape quantized all Q4_K;
* config 3's spec-verify batch exactly as bench.py builds it (4 tokens, Zipf(1.2) popularity from numpy's
  default_rng(3), Gumbel-top-k logits, the layer sized for 4 tokens), every copy of its rotation."""
import numpy as np
import pytest
import torch

from test_gpu_layer import decode_case

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_config1_one_token_instance(xm, xo):
    """Config 1's layer at one token: the T=1 kernel's Q8_0 instance, seeds as the smoke test's."""
    H, E, k, F = 1024, 8, 2, 512
    arena, L = xm.build_arena(E, H, F, xm.Q8_0, xm.Q8_0, seed=0, gen_device="cpu")
    for seed in range(3):
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(1, H, generator=g).to(DEV)
        wr = (torch.randn(E, H, generator=g) * 0.02).to(DEV)
        print(f"[case] config1 T=1 seed={seed}", flush=True)
        logits = xm.router_logits_f32(x, wr)
        rel, moe_rel = decode_case(xm, xo, arena, L, E, k, 1, logits, seed)
        assert rel <= 1e-3 and moe_rel <= 1e-3, (rel, moe_rel)


@pytest.mark.parametrize("E", [64, 256])
def test_one_token_router_widths(xm, xo, E):
    """The one-token kernel at config 2's expert shape with 64 experts (one logit a lane) and 256 (four a lane)."""
    arena, L = xm.build_arena(E, 2048, 768, xm.Q4_K, xm.Q6_K, seed=20 + E)
    for seed in range(2):
        g = torch.Generator(device=DEV).manual_seed(300 + E + seed)
        logits = torch.randn(1, E, device=DEV, generator=g)
        print(f"[case] t1 E={E} seed={seed}", flush=True)
        rel, moe_rel = decode_case(xm, xo, arena, L, E, 8, 1, logits, seed)
        assert rel <= 1e-3 and moe_rel <= 1e-3, (rel, moe_rel)


def test_config3_verify_as_benched(xm, xo):
    """bench.py's config-3 verify inputs: pop = -1.2 log(rank) over a permutation from default_rng(3), logits =
    pop + Gumbel noise for each of the rotation's copies, a layer sized for 4 tokens (the same kernel instance and
    plan the bench times); one arena, every copy's logits."""
    E, k, T, copies = 128, 8, 4, 8
    arena, L = xm.build_arena(E, 2048, 768, xm.Q4_K, xm.Q6_K, seed=0)
    rng = np.random.default_rng(3)
    pop = -1.2 * np.log(np.arange(1, E + 1))[rng.permutation(E)]
    zv = torch.from_numpy((pop[None, None, :] + rng.gumbel(size=(copies, T, E))).astype(np.float32)).to(DEV)
    for c in range(copies):
        print(f"[case] config3 verify copy={c}", flush=True)
        rel, moe_rel = decode_case(xm, xo, arena, L, E, k, T, zv[c].contiguous(), 40 + c)
        assert rel <= 1e-3 and moe_rel <= 1e-3, (c, rel, moe_rel)


def test_one_token_all_q4k_instance(xm, xo):
    """The one-token kernel's instance for config 2's shape quantized all Q4_K (hidden 2048, F 768, 128 experts,
    top-8): gate/up as config 2's, the down rows Q4_K (Unit<Q4_K>'s 32-value units on the raw rows, no decode)."""
    arena, L = xm.build_arena(128, 2048, 768, xm.Q4_K, xm.Q4_K, seed=31)
    for seed in range(2):
        g = torch.Generator(device=DEV).manual_seed(700 + seed)
        logits = torch.randn(1, 128, device=DEV, generator=g)
        print(f"[case] t1 all-Q4_K seed={seed}", flush=True)
        rel, moe_rel = decode_case(xm, xo, arena, L, 128, 8, 1, logits, 710 + seed)
        assert rel <= 1e-3 and moe_rel <= 1e-3, (rel, moe_rel)
