"""The tier protocol on the GPU (include/xs_tiers.h): a decode layer whose routed experts are split over three tiers,
as the reference's verify window runs it (src/core/moe_window.cpp:196-250), must give the parts of the all-HBM path
bit for bit.

  - HBM tier: groups whose blobs are in the device arena (plan ptr / start / counts[0]);
  - PCIe tier: groups whose blobs are in pinned host memory (ptr2 / start2 / counts[2]), either staged into HBM by
    xs_fetch_blobs + xs_rebase_ptrs (the copy-kernel mode) or read by the grouped kernel over PCIe directly;
  - CPU tier: rows the host computed (here the CPU oracle, whose rows are the kernels' bit for bit), in mapped host
    memory, taken by xs_copy_rows_from_mapped (+0.0 at the GPU's rows), then xs_moe_hit_add adds the GPU's rows.
The plan (GpuPlanSink words) is written by the host into mapped memory and copied in by xs_copy_i32_from_mapped after
xs_wait_flag_ge.  The flag wait is also checked on its own: already set, set by the host while the kernel polls, and
never set (the bound, forced small from the host, ends it and sets the status word)."""
import time

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
Q8_0 = 8
H, F, E, K, T = 1024, 512, 8, 2, 6


def pinned(shape, dtype):
    return torch.zeros(shape, dtype=dtype, pin_memory=True)


def test_wait_flag_already_set(xm):
    flag = pinned(4, torch.int32)
    flag[0] = 7
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    xm.wait_flag_ge(flag, 7, limit_us=2_000_000, status=status)
    torch.cuda.synchronize()
    assert int(status[0]) == 0


def test_wait_flag_set_by_host_while_polling(xm):
    flag = pinned(4, torch.int32)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    done = torch.zeros(1, dtype=torch.int32, device=DEV)
    s = torch.cuda.Stream()            # not the NULL stream: a NULL-stream call would wait for the kernel itself
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(s):
        xm.wait_flag_ge(flag, 3, limit_us=2_000_000, status=status)
        done.fill_(1)                  # runs after the wait on the same stream
    time.sleep(0.05)                   # (no host read of device state here: it would wait for the polling kernel)
    flag[0] = 3                        # the host's write to pinned memory, seen by the polling kernel
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    print(f"\n[tiers] host-set flag seen after {dt * 1e3:.1f} ms (host slept 50 ms)")
    assert int(status[0]) == 0 and int(done[0]) == 1
    assert dt < 1.5, "the wait ended only at its bound"


def test_wait_flag_bound_ends_the_wait(xm):
    flag = pinned(4, torch.int32)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    t0 = time.perf_counter()
    xm.wait_flag_ge(flag, 1, limit_us=20_000, status=status)
    torch.cuda.synchronize()
    assert int(status[0]) == 1
    assert time.perf_counter() - t0 < 1.0


def test_copies_and_hit_add(xm):
    rng = np.random.default_rng(3)
    n = 1003                                            # not a multiple of 4: the tail copies one by one
    src = pinned(n + 5, torch.int32)
    src[:] = torch.from_numpy(rng.integers(-2**31, 2**31 - 1, n + 5).astype(np.int32))
    dst = torch.full((n + 8,), -1, dtype=torch.int32, device=DEV)
    xm.copy_i32_from_mapped(dst, src, n)
    xm.copy_i32_from_mapped(dst[4:].data_ptr() + 4, src.data_ptr() + 8, 5)   # unaligned ends: the scalar form
    torch.cuda.synchronize()
    want = src[:n].clone()
    want[5:10] = src[2:7]
    assert torch.equal(dst[:n].cpu(), want) and bool((dst[n:].cpu() == -1).all())

    rows, width = 12, 1024
    m = pinned((rows, width), torch.float32)
    m[:] = torch.from_numpy(rng.standard_normal((rows, width)).astype(np.float32))
    hits = torch.tensor([7, 2, 11, 2], dtype=torch.int32, device=DEV)
    count = torch.tensor([3], dtype=torch.int32, device=DEV)            # the 4th listed row is not a hit
    parts = torch.full((rows, width), 9.0, device=DEV)
    xm.copy_rows_from_mapped(parts, m, rows, width, hits, count)
    hit_out = torch.from_numpy(rng.standard_normal((rows, width)).astype(np.float32)).to(DEV)
    xm.moe_hit_add(parts, hit_out, hits, count, 4, width)
    torch.cuda.synchronize()
    got = parts.cpu()
    for r in range(rows):
        if r in (7, 2, 11):
            # +0.0 + hit: the hit's value (a -0.0 hit gives +0.0)
            assert torch.equal(got[r], hit_out[r].cpu() + 0.0), r
        else:
            assert torch.equal(got[r], m[r]), r

    blob = 4096 + 48
    host = pinned((5, blob), torch.uint8)
    host[:] = torch.from_numpy(rng.integers(0, 256, (5, blob)).astype(np.uint8))
    order = [3, 0, 4]
    src_tab = torch.tensor([host[i].data_ptr() for i in order] + [0] * 5, dtype=torch.int64, device=DEV)
    cnt = torch.tensor([3], dtype=torch.int32, device=DEV)
    staging = torch.full((8 * blob,), 0xAB, dtype=torch.uint8, device=DEV)
    xm.fetch_blobs(src_tab, cnt, staging, blob, 8)
    xm.rebase_ptrs(src_tab, cnt, staging, blob)
    torch.cuda.synchronize()
    st = staging.cpu().view(8, blob)
    for k, i in enumerate(order):
        assert torch.equal(st[k], host[i]), k
    assert bool((st[3:] == 0xAB).all())
    tab = src_tab.cpu().tolist()
    assert tab[:3] == [staging.data_ptr() + k * blob for k in range(3)] and tab[3:] == [0] * 5


def build_plan(xm, ids, tier, arena, host_blobs, capx):
    """The host pool's GpuPlanSink words for one layer: HBM groups first (distinct experts in routing order, their
    entries ascending), then the PCIe groups, whose entries follow in the same dst / tok arrays."""
    o = xm.plan_offsets(capx)
    words = xm.plan_words(capx)
    plan = np.zeros(words, dtype=np.int32)
    flat = ids.reshape(-1)
    groups = {0: [], 1: []}
    for e in dict.fromkeys(flat.tolist()):
        if tier[e] in (0, 1):
            groups[tier[e]].append(e)
    ents, starts = [], {0: [0], 1: []}
    for t in (0, 1):
        if t == 1:
            starts[1].append(len(ents))
        for e in groups[t]:
            ents += [i for i in range(flat.size) if flat[i] == e]
            starts[t].append(len(ents))
    n_gpu = len(ents)
    plan[0:4] = [len(groups[0]), n_gpu, len(groups[1]), 0]
    plan[o["start"]:o["start"] + len(starts[0])] = starts[0]
    plan[o["dst"]:o["dst"] + n_gpu] = ents
    plan[o["tok"]:o["tok"] + n_gpu] = [i // K for i in ents]
    ptr = np.zeros(2 * capx, dtype=np.uint64)
    for g, e in enumerate(groups[0]):
        ptr[g] = arena[e].data_ptr()
    for q, e in enumerate(groups[1]):
        ptr[capx + q] = host_blobs[e].data_ptr()
    plan[o["ptr"]:o["ptr"] + 4 * capx] = ptr.view(np.int32)
    plan[o["start2"]:o["start2"] + len(starts[1])] = starts[1]
    return plan, ents, groups


@pytest.mark.parametrize("pcie_mode", ["staged", "direct"])
def test_three_tier_layer_equals_all_hbm(xm, xo, pcie_mode):
    rng = np.random.default_rng(11)
    arena, L = xm.build_arena(E, H, F, Q8_0, Q8_0, seed=9)
    blob = int(L.bytes)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(DEV)
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).to(DEV)
    ids_d, w_d = xm.router_top10(logits, K)
    ids = ids_d.cpu().numpy().astype(np.int32)
    tier = {e: e % 3 for e in range(E)}                 # 0 HBM, 1 PCIe, 2 CPU
    flat = ids.reshape(-1)
    assert {tier[e] for e in flat.tolist()} == {0, 1, 2}, "the routing must touch all three tiers"
    capx = T * K
    host_blobs = {e: pinned(blob, torch.uint8) for e in range(E)}
    for e in range(E):
        host_blobs[e][:] = arena[e].cpu()
    plan, ents, groups = build_plan(xm, ids, tier, arena, host_blobs, capx)
    xq = xm.quantize_q8_1_rows(x)

    # the CPU tier's rows: the oracle's, at each entry's routed index (token * k + j)
    ol = xo.layout(Q8_0, Q8_0, H, F)
    blobs = arena.cpu().numpy()
    all_start = np.arange(capx + 1, dtype=np.int32)
    all_dst = np.arange(capx, dtype=np.int32)
    all_tok = (all_dst // K).astype(np.int32)
    want = xo.native_expert_grouped(ol, [blobs[e] for e in flat], all_start, all_dst, all_tok, xq.cpu().numpy(), capx)
    m_rows = pinned((capx, H), torch.float32)
    m_rows[:] = 5.0                                     # the GPU's rows must not take these
    for i in range(capx):
        if tier[int(flat[i])] == 2:
            m_rows[i] = torch.from_numpy(want[i])
    m_plan = pinned(plan.size, torch.int32)
    m_plan[:] = torch.from_numpy(plan)
    flag = pinned(4, torch.int32)
    flag[0] = 1                                         # the pool has published this ring
    status = torch.zeros(1, dtype=torch.int32, device=DEV)

    o = xm.plan_offsets(capx)
    pl = torch.zeros(plan.size + 16, dtype=torch.int32, device=DEV)
    a = lambda w: pl.data_ptr() + 4 * w                 # device address of plan word w
    hit_out = torch.zeros(capx, H, device=DEV)
    parts = torch.full((capx, H), -3.0, device=DEV)
    scratch = torch.zeros(xm.native_expert_scratch_bytes(capx, F), dtype=torch.uint8, device=DEV)
    staging = torch.zeros(capx * blob, dtype=torch.uint8, device=DEV)

    xm.wait_flag_ge(flag, 1, limit_us=2_000_000, status=status)
    xm.copy_i32_from_mapped(pl, m_plan, plan.size)
    xm.native_expert_grouped(L, a(o["ptr"]), a(o["start"]), a(0), a(o["dst"]), a(o["tok"]), capx, capx, xq, scratch,
                             hit_out)
    if pcie_mode == "staged":
        xm.fetch_blobs(a(o["ptr"] + 2 * capx), a(2), staging, blob, capx)
        xm.rebase_ptrs(a(o["ptr"] + 2 * capx), a(2), staging, blob)
    xm.native_expert_grouped(L, a(o["ptr"] + 2 * capx), a(o["start2"]), a(2), a(o["dst"]), a(o["tok"]), capx, capx, xq,
                             scratch, hit_out)
    xm.copy_rows_from_mapped(parts, m_rows, capx, H, a(o["dst"]), a(1))
    xm.moe_hit_add(parts, hit_out, a(o["dst"]), a(1), capx, H)
    torch.cuda.synchronize()
    assert int(status[0]) == 0
    got = parts.cpu().numpy()
    assert np.array_equal(got, want), f"max |diff| {np.abs(got - want).max()}"
    if pcie_mode == "staged":
        st = staging.cpu().numpy().reshape(capx, blob)
        for q, e in enumerate(groups[1]):
            assert np.array_equal(st[q], blobs[e])
    # and the combine over these parts is the all-HBM layer's
    out = torch.empty(T, H, device=DEV)
    xm.native_moe_combine_multi(parts, w_d, None, out, H, K, T)
    ref = torch.empty(T, H, device=DEV)
    xm.native_moe_combine_multi(torch.from_numpy(want).to(DEV), w_d, None, ref, H, K, T)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
