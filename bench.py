#!/usr/bin/env python3
"""bench.py - XeStrata's MoE-layer hot path on one MI355X.

Metric: MoE-layer decode us/token and expert-weight HBM GB/s (% of peak); prefill TFLOP/s.
Workload of `value`: config 2 (Qwen3-30B-A3B-shaped layer: hidden 2048, 128 experts, top-8, F 768, Q4_K gate/up,
Q6_K down), decode batch 1; a step = one whole MoE layer (router -> plan -> q8_1 -> grouped experts -> combine ->
residual) for one token, the layer's weights rotated over `--copies` distinct HBM copies (>= 1 GB, past the 256 MB
Infinity Cache).  value = expert-weight GB/s = (distinct experts touched x blob bytes) / time per step.
Each step sequence is captured once in a HIP graph and replayed; inputs are resident in HBM before timing.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import math
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "xestrata-win_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 and fp16 MFMA, published
METRIC = "MoE-layer decode µs/token + expert-weight HBM GB/s (% of peak); prefill TFLOP/s"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


_FLUSH = []


def flush_caches(torch):
    """Read 1 GiB of unrelated memory (4x the 256 MB Infinity Cache) with the library's read-only stream kernel
    (xs_bench_hbm_read): nothing a timed step reads is left in the caches by the untimed runs before it, and - unlike
    a copy - the flush leaves no dirty lines whose write-back would compete with the timed steps' reads (a 1 GiB copy
    here cost the T=1 decode layer 0.5 us a step even at 400 steps)."""
    import xsmoe as xm
    if not _FLUSH:
        _FLUSH.append(torch.ones(1 << 30, dtype=torch.uint8, device="cuda"))
        _FLUSH.append(torch.zeros(4096, dtype=torch.int32, device="cuda"))
    xm._check(xm.lib().xs_bench_hbm_read(_FLUSH[0].data_ptr(), _FLUSH[0].numel(), _FLUSH[1].data_ptr(), 4096,
                                         torch.cuda.current_stream().cuda_stream))


def graph_time(torch, fn, replays, flush=False):
    """Capture fn() once in a HIP graph; replay `replays` times between two events; return ms per replay.  The cache
    flush (1 GiB read, when asked) is enqueued right before the first event with no synchronisation in
    between, so the host prepares the replays while it runs and the events hold the replays' GPU time only, not the
    graph launch's host latency (at 20 steps that latency alone was ~1.5 us a step)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()                                  # eager warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    g.replay()
    torch.cuda.synchronize()
    if flush:
        flush_caches(torch)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / replays, g


def run_graph(torch, calls):
    """Capture the calls once, in order, as one HIP graph; replay it once between two events on the replay stream;
    return the elapsed ms (each call's kernels run exactly once in the timed region)."""
    def fn():
        for c in calls:
            c()
    ms, _ = graph_time(torch, fn, 1, flush=True)
    return ms


def best_of_means(torch, fn, reps, trials=5):
    """The reference's prompt timing rule (src/kernels/iq_mmq_parity.cpp:150-163: the best of 5 means of 10): fn()
    captured once in a HIP graph; `trials` times, `reps` replays between two events; the smallest mean, ms."""
    _, g = graph_time(torch, fn, 1)
    best = float("inf")
    for _ in range(trials):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) / reps)
    return best


def measured_peaks(torch, xm, arena, span):
    """This box's achieved peaks, measured with the library's probes (xs_bench_hbm_read, xs_bench_mfma_f16):
    - hbm_stream_gbs: a read-only stream over 2 GiB, nontemporal 16-byte loads, the best of four grid sizes (means of
      5 launches after one untimed);
    - hbm_one_launch: `span` bytes (one decode layer's experts) read by one launch, the launches rotated over the
      headline's arena in `span`-byte regions (the caches hold none of them) and replayed from one graph, as the
      headline is; the best of four grid sizes;
    - mfma_f16_tflops: v_mfma_f32_32x32x16_f16 back to back, 8 accumulators a wave, 2 waves a SIMD on every CU."""
    dev = "cuda"
    st = torch.cuda.current_stream().cuda_stream
    sink = torch.zeros(1 << 16, dtype=torch.int32, device=dev)
    buf = torch.empty(2 << 30, dtype=torch.uint8, device=dev).fill_(7)
    stream = {}
    for grid in (1024, 2048, 4096, 8192):
        xm.lib().xs_bench_hbm_read(buf.data_ptr(), buf.numel(), sink.data_ptr(), grid, st)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            xm._check(xm.lib().xs_bench_hbm_read(buf.data_ptr(), buf.numel(), sink.data_ptr(), grid, st))
        e1.record()
        torch.cuda.synchronize()
        stream[grid] = buf.numel() / (e0.elapsed_time(e1) / 5 * 1e-3) / 1e9
    del buf
    torch.cuda.empty_cache()
    flat = arena.view(-1)
    n_reg = flat.numel() // span
    one = {}
    for grid in (256, 512, 1024, 2048):
        def fn(grid=grid):
            cs = torch.cuda.current_stream().cuda_stream
            for r in range(n_reg):
                xm._check(xm.lib().xs_bench_hbm_read(flat.data_ptr() + r * span, span, sink.data_ptr(), grid, cs))
        ms = run_graph(torch, [fn])
        one[grid] = ms * 1e3 / n_reg
    g1 = min(one, key=one.get)
    grid_m, iters = 1024, 2000
    fsink = torch.zeros(grid_m * 128, device=dev)
    xm._check(xm.lib().xs_bench_mfma_f16(iters, grid_m, fsink.data_ptr(), st))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        xm._check(xm.lib().xs_bench_mfma_f16(iters, grid_m, fsink.data_ptr(), st))
    e1.record()
    torch.cuda.synchronize()
    tf = grid_m * 2 * iters * 8 * 32768.0 / (e0.elapsed_time(e1) / 5 * 1e-3) / 1e12
    gs = max(stream, key=stream.get)
    out = dict(hbm_stream_gbs=round(stream[gs], 1), hbm_stream_grid=gs, hbm_stream_bytes=2 << 30,
               hbm_one_launch_bytes=span, hbm_one_launch_us=round(one[g1], 3),
               hbm_one_launch_gbs=round(span / (one[g1] * 1e-6) / 1e9, 1), hbm_one_launch_grid=g1,
               mfma_f16_tflops=round(tf, 1),
               method="xs_bench_hbm_read / xs_bench_mfma_f16 (xestrata-win_amd/csrc/peaks.hip)")
    log(f"measured peaks: HBM stream {out['hbm_stream_gbs']} GB/s (grid {gs}); one launch of {span / 1e6:.2f} MB "
        f"{out['hbm_one_launch_us']} us = {out['hbm_one_launch_gbs']} GB/s (grid {g1}); f16 MFMA {tf:.0f} TFLOP/s")
    return out


TRAFFIC_FILE = ROOT / "profiles" / "moe_decode_t1_config2_traffic.md"


def read_traffic():
    """HBM bytes per launch of the fused decode kernel, from the committed rocprofv3 --pmc summary (FETCH_SIZE +
    WRITE_SIZE scaled by a copy kernel of known size), or None when that summary is absent."""
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    except (OSError, ValueError):
        pass
    return None


def pmc_kernel_and_scale(rows, ctr, kernel, copy_kib, n_copies=4, min_dispatches=64):
    """From a rocprofv3 --pmc counter CSV's rows (dicts: Dispatch_Id, Kernel_Name, Counter_Name, Counter_Value; a
    counter may span several rows of one dispatch, which add up): (the kernel's mean `ctr` a dispatch, the scale that
    makes the last n_copies device copies read copy_kib KiB each, the kernel's dispatch count), or None when there are
    fewer than min_dispatches of the kernel, fewer than n_copies copies or copies whose counts differ."""
    sums, names = {}, {}
    for row in rows:
        if row.get("Counter_Name") != ctr:
            continue
        did = int(row["Dispatch_Id"])
        sums[did] = sums.get(did, 0.0) + float(row["Counter_Value"])
        names[did] = row["Kernel_Name"]
    ks = [v for i, v in sums.items() if kernel in names[i]]
    cps = [sums[i] for i in sorted(sums) if "copyBuffer" in names[i]][-n_copies:]
    if len(ks) < min_dispatches or len(cps) < n_copies or min(cps) <= 0 or max(cps) > 1.01 * min(cps):
        return None   # (copies of one size read one count: anything else is not the calibration)
    return sum(ks) / len(ks), copy_kib / (sum(cps) / len(cps)), len(ks)


def live_traffic(timeout_s=180):
    """HBM bytes per launch of the one-token kernel, measured in this run: two rocprofv3 --pmc passes (FETCH_SIZE, then
    WRITE_SIZE, one counter a pass), each over a child `bench.py --pmc-run` - one cycle of the headline's rotation
    (128 launches, every one reading its 8 experts from HBM), then 4 device copies of 256 MiB.  Each counter is scaled
    by what it reads for those copies (a copy reads and writes its size).  Returns (bytes, detail) or (None, reason):
    no rocprofv3, this process itself under a profiler, or a pass that failed or timed out (timeout -s KILL)."""
    import csv
    import glob
    import shutil
    import subprocess
    import tempfile
    rp = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(rp):
        return None, "rocprofv3 not found"
    if any(k.startswith(("ROCPROF", "ROCP_")) for k in os.environ):
        return None, "this run is itself under a profiler"
    copy_kib = (256 << 20) / 1024.0
    per = {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="xs_pmc_")
        try:
            cmd = ["timeout", "-s", "KILL", str(timeout_s), rp, "--pmc", ctr, "--output-format", "csv", "-d", d,
                   "-o", "run", "--", sys.executable, str(ROOT / "bench.py"), "--pmc-run"]
            r = subprocess.run(cmd, capture_output=True, text=True, cwd=str(ROOT))
            files = glob.glob(os.path.join(d, "**", "run_counter_collection.csv"), recursive=True)
            if not files:
                return None, f"{ctr} pass: no counter file (exit {r.returncode})"
            with open(files[0]) as fh:
                got = pmc_kernel_and_scale(csv.DictReader(fh), ctr, "moe_decode_t1_kernel", copy_kib)
            if got is None:
                return None, f"{ctr} pass: too few kernel or copy dispatches in its counters (exit {r.returncode})"
            per[ctr] = got
        finally:
            shutil.rmtree(d, ignore_errors=True)
    (f, fs, n), (w, ws, _) = per["FETCH_SIZE"], per["WRITE_SIZE"]
    traffic = int(round((f * fs + w * ws) * 1024))
    return traffic, (f"measured in this run: rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, over `bench.py --pmc-run` "
                     f"({n} launches of the kernel), {f:.1f} x {fs:.3f} + {w:.1f} x {ws:.3f} KiB a launch, the "
                     f"scales from 4 device copies of 256 MiB")


def pmc_run(torch, xm, copies):
    """The workload of a rocprofv3 --pmc pass: the headline's rotation, one cycle of config-2 decode layers at T=1
    (8 copies x 16 disjoint expert sets = 128 launches, each reading its 8 experts from HBM) and, for calibration,
    4 device-to-device copies of 256 MiB."""
    E, H, F, k = 128, 2048, 768, 8
    arena, L = xm.build_arena(E, H, F, xm.Q4_K, xm.Q6_K, seed=0, copies=copies)
    gen = torch.Generator(device="cuda").manual_seed(1)
    n_sets = E // k
    logits = set_logits(torch, n_sets, 1, E, k, "cuda", gen)
    x = torch.randn(1, H, device="cuda", generator=gen).to(torch.bfloat16).float()
    res = torch.randn(1, H, device="cuda", generator=gen)
    out = torch.empty(1, H, device="cuda")
    layer = xm.MoeLayer(L, arena, E, k, 1)
    for i in range(copies * n_sets):
        c, s = i % copies, (i // copies) % n_sets
        layer(x, logits[s], res, out, arena=arena[c * E])
    status = layer.status()   # (read before the calibration copies: its own small copy must not be among their last 4)
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"pmc run: {copies * n_sets} decode layers ({k * L.bytes / 1e6:.2f} MB of expert weights each), "
        f"4 copies of {256 << 20} bytes; status {status}")


def pmc_prefill(torch, xm):
    """The workload of a rocprofv3 --pmc pass on the prompt path: 4 config-3 prefill layers (2048 tokens, Zipf(1.2)
    routing), the grouped GEMMs' counters read per dispatch."""
    import numpy as np
    E, H, F, k, Tp = 128, 2048, 768, 8, 2048
    arena, L = xm.build_arena(E, H, F, xm.Q4_K, xm.Q6_K, seed=0, copies=1)
    rng = np.random.default_rng(3)
    pop = -1.2 * np.log(np.arange(1, E + 1))[rng.permutation(E)]
    zl = torch.from_numpy((pop[None, :] + rng.gumbel(size=(Tp, E))).astype(np.float32)).cuda()
    gen = torch.Generator(device="cuda").manual_seed(1)
    xp = torch.randn(Tp, H, device="cuda", generator=gen).to(torch.bfloat16).float()
    rp = torch.randn(Tp, H, device="cuda", generator=gen)
    op = torch.empty(Tp, H, device="cuda")
    layer = xm.MoeLayer(L, arena, E, k, Tp, prefill=True)
    for _ in range(4):
        layer(xp, zl, rp, op)
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(2):   # calibration of FETCH_SIZE / WRITE_SIZE: copies of a known size
        dst.copy_(src)
    torch.cuda.synchronize()
    log("pmc prefill run: 4 config-3 prefill layers, 2 copies of 256 MiB")


def pmc_verify(torch, xm):
    """The workload of a rocprofv3 pass on config 3's spec-verify decode: 4 tokens, Zipf(1.2) popularity (the bench's
    own logits: default_rng(3)), one rotation over 8 HBM copies of the config-2-shaped layer (8 launches of the fused
    kernel, ~21.5 distinct experts each)."""
    import numpy as np
    E, H, F, k, copies = 128, 2048, 768, 8, 8
    arena, L = xm.build_arena(E, H, F, xm.Q4_K, xm.Q6_K, seed=0, copies=copies)
    rng = np.random.default_rng(3)
    pop = -1.2 * np.log(np.arange(1, E + 1))[rng.permutation(E)]
    zv = torch.from_numpy((pop[None, None, :] + rng.gumbel(size=(copies, 4, E))).astype(np.float32)).cuda()
    gen = torch.Generator(device="cuda").manual_seed(1)
    xv = torch.randn(4, H, device="cuda", generator=gen).to(torch.bfloat16).float()
    rv = torch.randn(4, H, device="cuda", generator=gen)
    ov = torch.empty(4, H, device="cuda")
    layer = xm.MoeLayer(L, arena, E, k, 4)
    for c in range(copies):
        layer(xv, zv[c], rv, ov, arena=arena[c * E])
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(2):   # calibration of FETCH_SIZE / WRITE_SIZE: copies of a known size
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"pmc verify run: {copies} config-3 verify layers (T=4, Zipf); status {layer.status()}")


def pmc_c5dec(torch, xm):
    """The workload of a rocprofv3 pass on config 5's one-token decode: the bench's own rotation (32 routed sets, 8
    copies of the shared expert; the group-limited sigmoid router inside the routed launch), one call a step, then 2
    calibration copies of 256 MiB."""
    E, H, F, k = 256, 7168, 2048, 8
    gen = torch.Generator(device="cuda").manual_seed(1)
    arena, L = xm.build_arena(E, H, F, xm.Q4_K, xm.Q4_K, seed=5)
    sarena, SL = xm.build_arena(1, H, 2048, xm.Q8_0, xm.Q8_0, seed=55, copies=8)
    bias = torch.randn(E, device="cuda", generator=gen) * 0.1
    router = xm.grouped_sigmoid_router(bias, 8, 4, 2.5)
    n_sets = E // k
    lg = torch.randn(n_sets, 1, E, device="cuda", generator=gen) - 4.0
    for st in range(n_sets):
        idx = [gi * 32 + 2 * (st // 2) + j for gi in ((0, 1, 2, 3) if st % 2 == 0 else (4, 5, 6, 7)) for j in (0, 1)]
        lg[st, :, idx] += 12.0
    x = torch.randn(1, H, device="cuda", generator=gen).to(torch.bfloat16).float()
    res = torch.randn(1, H, device="cuda", generator=gen)
    o = torch.empty(1, H, device="cuda")
    layer = xm.MoeLayer(L, arena, E, k, 1, shared=(SL, sarena[0], None), router=router)
    for st in range(n_sets):
        layer(x, lg[st], res, o, shared_blob=sarena[st % 8])
    status = layer.status()
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(2):   # calibration of FETCH_SIZE / WRITE_SIZE: copies of a known size
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"pmc config-5 decode run: {n_sets} one-token layers (8 routed Q4_K experts + the Q8_0 shared expert each); "
        f"status {status}")


def pmc_tput(torch, xm):
    """The workload of a rocprofv3 --pmc pass on the throughput decode: one rotation of config-2 layers at T=16 (8 HBM
    copies, disjoint expert sets) and of config-4 layers at T=8 (2 HBM copies of the IQ4_XS layer, disjoint sets)."""
    gen = torch.Generator(device="cuda").manual_seed(1)
    for name, (E, H, F, gt, dt, T, copies, seed) in (("config 2 T=16", (128, 2048, 768, xm.Q4_K, xm.Q6_K, 16, 8, 0)),
                                                     ("config 4 T=8", (128, 4096, 1536, xm.IQ4_XS, xm.IQ4_XS, 8, 2, 4))):
        k = 8
        arena, L = xm.build_arena(E, H, F, gt, dt, seed=seed, copies=copies)
        n_sets = max(1, E // (T * k))
        lg = set_logits(torch, n_sets, T, E, k, "cuda", gen)
        x = torch.randn(T, H, device="cuda", generator=gen).to(torch.bfloat16).float()
        res = torch.randn(T, H, device="cuda", generator=gen)
        out = torch.empty(T, H, device="cuda")
        layer = xm.MoeLayer(L, arena, E, k, T)
        for c in range(copies):
            for st in range(n_sets):
                layer(x, lg[st], res, out, arena=arena[c * E])
        torch.cuda.synchronize()
        log(f"pmc tput run: {name}, {copies * n_sets} layers; status {layer.status()}")
        del arena
        torch.cuda.empty_cache()


def set_logits(torch, n_sets, T, E, k, dev, gen):
    """n_sets logit sets [n_sets, T, E]: i.i.d. N(0,1) plus +8 on set s's T*k experts (s*T*k .. mod E), so that the
    steps of a rotation touch disjoint experts and no step finds its blobs still in the caches."""
    lg = torch.randn(n_sets, T, E, device=dev, generator=gen)
    for s in range(n_sets):
        lg[s, :, (torch.arange(T * k, device=dev) + s * T * k) % E] += 8.0
    return lg


def time_steps(torch, calls, steps, warmup):
    """calls: one zero-argument callable a step, captured as one graph round and replayed; ms per step."""
    def one_round():
        for c in calls:
            c()
    graph_time(torch, one_round, max(1, math.ceil(warmup / len(calls))))
    ms, _ = graph_time(torch, one_round, max(1, math.ceil(steps / len(calls))))
    return ms / len(calls)


def distinct_experts(torch, lg, k):
    return float(sum(len(torch.unique(torch.topk(lg[s], k, dim=1).indices)) for s in range(lg.shape[0])) / lg.shape[0])


def other_configs(torch, xm, dev, gen, steps):
    """Decode of configs 4 and 5 (reported beside the value, not the value): the layer per step, weights rotated so
    that every step reads its experts from HBM."""
    import numpy as np
    out = {}
    # config 4: the Qwen3-235B-A22B-shaped stack, IQ4_XS experts (hidden 4096, 128 experts, top-8, F 1536): 94 layers
    # resident in HBM (120.6 GB), one token (or 8) through all 94 in one graph - per-stack time.  Each layer is
    # quantized from its own seeded random weights (seeds 4000 + layer), so every layer's experts are distinct bytes
    # read from HBM
    E, H, F, k, NL = 128, 4096, 1536, 8, 94
    L = xm.native_expert_layout(xm.IQ4_XS, xm.IQ4_XS, H, F)
    t0 = time.time()
    stack = torch.empty(NL * E, L.bytes, dtype=torch.uint8, device=dev)
    for li in range(NL):   # every layer its own seeded random weights, quantized to IQ4_XS
        xm.fill_layer(stack[li * E:(li + 1) * E], L, seed=4000 + li)
    torch.cuda.synchronize()
    log(f"config 4: {NL}-layer stack resident, {stack.numel() / 1e9:.1f} GB, {NL} distinct seeds, built in "
        f"{time.time() - t0:.1f} s")
    for T in (1, 8):
        lg = torch.randn(NL, T, E, device=dev, generator=gen)   # each layer its own routing
        x = torch.randn(T, H, device=dev, generator=gen).to(torch.bfloat16).float()
        res = torch.randn(T, H, device=dev, generator=gen)
        o = torch.empty(T, H, device=dev)
        layer = xm.MoeLayer(L, stack, E, k, T)

        def one_token():
            for li in range(NL):
                layer(x, lg[li], res, o, arena=stack[li * E])
        graph_time(torch, one_token, 1)
        ms, _ = graph_time(torch, one_token, 3)
        b = sum(len(torch.unique(torch.topk(lg[li], k, dim=1).indices)) for li in range(NL)) * L.bytes
        out[f"config4_T{T}"] = dict(us_per_stack=round(ms * 1e3, 1), us_per_token=round(ms * 1e3 / T, 1),
                                    us_per_layer=round(ms * 1e3 / NL, 2), tokens_per_s=round(T / (ms * 1e-3), 1),
                                    expert_gbs=round(b / (ms * 1e-3) / 1e9, 1),
                                    frac_hbm_peak=round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                    expert_gb_per_step=round(b / 1e9, 2), layers=NL,
                                    stack_gb=round(stack.numel() / 1e9, 1), status=layer.status())
        log(f"config 4 decode T={T}, {NL}-layer stack: {ms * 1e3:.1f} us/stack ({ms * 1e3 / T:.1f} us/token, "
            f"{ms * 1e3 / NL:.2f} us/layer), {out[f'config4_T{T}']['expert_gbs']} GB/s")
    del stack
    torch.cuda.empty_cache()
    # config 5: DeepSeek-V3-shaped (hidden 7168, 256 routed Q4_K experts, top-8, F 2048, one shared Q8_0 expert),
    # routed by its own group-limited sigmoid router (bias, 8 groups, top-4, routed scale 2.5), the shared expert's
    # row added by the combine: one call a layer (xs_moe_layer_decode_ex / xs_moe_layer_prefill_ex)
    E, H, F, k = 256, 7168, 2048, 8
    arena, L = xm.build_arena(E, H, F, xm.Q4_K, xm.Q4_K, seed=5)
    s_copies = 8
    sarena, SL = xm.build_arena(1, H, 2048, xm.Q8_0, xm.Q8_0, seed=55, copies=s_copies)
    bias = torch.randn(E, device=dev, generator=gen) * 0.1
    router = xm.grouped_sigmoid_router(bias, 8, 4, 2.5)
    n_sets = E // k
    # logits whose group-limited top-8 are disjoint from set to set and cover all 256 experts once: set s lifts two
    # experts in each of four groups (groups 0-3 for even s, 4-7 for odd; pair s // 2 of the group's 16), the rest
    # sit 4 below N(0,1), so the four lifted groups win and their lifted pairs are the top-8 (checked below)
    lg = torch.randn(n_sets, 1, E, device=dev, generator=gen) - 4.0
    boosted = []
    for st in range(n_sets):
        idx = [gi * 32 + 2 * (st // 2) + j for gi in ((0, 1, 2, 3) if st % 2 == 0 else (4, 5, 6, 7)) for j in (0, 1)]
        lg[st, :, idx] += 12.0
        boosted.append(sorted(idx))
    for st in range(n_sets):
        got = sorted(xm.router_grouped_sigmoid(lg[st], bias, 8, 4, k, 2.5)[0].view(-1).tolist())
        assert got == boosted[st], (st, got, boosted[st])
    x = torch.randn(1, H, device=dev, generator=gen).to(torch.bfloat16).float()
    res = torch.randn(1, H, device=dev, generator=gen)
    o = torch.empty(1, H, device=dev)
    layer = xm.MoeLayer(L, arena, E, k, 1, shared=(SL, sarena[0], None), router=router)
    # step st: routed set st, shared copy st % 8 (a routed expert comes back after 32 steps, 6.3 GB later; a shared
    # copy after 8, 1.96 GB later: both past the 256 MB Infinity Cache)
    ms = time_steps(torch, [(lambda st=st: layer(x, lg[st], res, o, shared_blob=sarena[st % s_copies]))
                            for st in range(n_sets)], steps, n_sets)
    ms_r = time_steps(torch, [lambda: xm.router_grouped_sigmoid(lg[0], bias, 8, 4, k, 2.5)] * 32, steps, 32)
    distinct = float(np.mean([len(torch.unique(xm.router_grouped_sigmoid(lg[st], bias, 8, 4, k, 2.5)[0]))
                              for st in range(n_sets)]))
    b = distinct * L.bytes + SL.bytes
    out["config5_T1"] = dict(us_per_layer=round(ms * 1e3, 2), expert_gbs=round(b / (ms * 1e-3) / 1e9, 1),
                             shared_copies=s_copies, sets=n_sets,
                             frac_hbm_peak=round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), expert_mb=round(b / 1e6, 1),
                             routing="the group-limited sigmoid router (bias, 8 groups, top-4, k 8, scale 2.5) inside "
                                     "the one-call layer (its own launch, included); the shared expert's row added",
                             router_alone_us=round(ms_r * 1e3, 2))
    log(f"config 5 decode T=1 (sigmoid router + shared expert, one call): {ms * 1e3:.2f} us/layer, "
        f"{out['config5_T1']['expert_gbs']} GB/s; the router alone {ms_r * 1e3:.2f} us")
    # config 5 prefill, 1024 tokens: the whole prompt layer in one call - router, permutation, routed experts, the
    # shared expert over every token, the combine with the shared row, the residual
    Tq = 1024
    lq = torch.randn(Tq, E, device=dev, generator=gen)
    xq = torch.randn(Tq, H, device=dev, generator=gen).to(torch.bfloat16).float()
    rq = torch.randn(Tq, H, device=dev, generator=gen)
    oq = torch.empty(Tq, H, device=dev)
    qlayer = xm.MoeLayer(L, arena, E, k, Tq, prefill=True, shared=(SL, sarena[0], None), router=router)
    ms_q = time_steps(torch, [lambda: qlayer(xq, lq, rq, oq)] * 2, 4, 2)
    fr, fs = 6.0 * Tq * k * H * F, 6.0 * Tq * H * 2048
    tq = (fr + fs) / (ms_q * 1e-3) / 1e12
    ids_q, _ = xm.router_grouped_sigmoid(lq, bias, 8, 4, k, 2.5)
    bq = len(torch.unique(ids_q)) * L.bytes + SL.bytes
    out["config5_prefill_T1024"] = dict(us_per_layer=round(ms_q * 1e3, 1), tflops=round(tq, 2),
                                        frac_mfma_peak=round(tq / BF16_PEAK_TFLOPS, 4),
                                        gflops_per_layer=round((fr + fs) / 1e9, 1),
                                        expert_gb=round(bq / 1e9, 3),
                                        expert_gbs=round(bq / (ms_q * 1e-3) / 1e9, 1),
                                        frac_hbm_peak=round(bq / (ms_q * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                        bound="hbm (every expert streamed once at ~32 rows an expert)",
                                        routing="the group-limited sigmoid router; the shared row added by the "
                                                "combine; one call")
    log(f"config 5 prefill T={Tq} (one call): {ms_q * 1e3:.1f} us, {tq:.1f} TFLOP/s")
    del arena, sarena
    torch.cuda.empty_cache()
    return out


def cpu_info():
    """The host's CPU as /proc/cpuinfo names it: the full model string, logical CPUs, physical cores (distinct
    (physical id, core id) pairs), sockets, and the CPUs this process may run on."""
    model, logical, cores, sockets, phys = "unknown", 0, set(), set(), None
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "processor":
                logical += 1
            elif key == "model name" and model == "unknown":
                model = val
            elif key == "physical id":
                phys = val
                sockets.add(val)
            elif key == "core id":
                cores.add((phys, val))
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except OSError:
        allowed = None
    return dict(model=model, logical_cpus=logical, physical_cores=len(cores) or None, sockets=len(sockets) or None,
                cpus_allowed=allowed)


def cpu_baseline(torch, xm, np, arena, L, E, H, F, k, dev, gen, max_threads=16):
    """The reference's CPU/host decode path (oracle/cpu_path.cpp: ggml's Q8_K / Q8_0 activations, the multi-token
    AVX2 rows, g / (1 + exp(-g)) u, the rank-order combine) on this box's host cores: one pinned thread a physical
    core, at most 16 (the box's CPU share), timed as the best of 5 means of 10 calls with the expert sets rotated so
    the weights come from DRAM.  Config 2 at one token (the headline's workload) and config 1 (its own 4 tokens, and
    1); each with the largest difference to the GPU's output of the same call, relative to the GPU's largest
    magnitude of the MoE part."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import xs_oracle as xo
    threads = xo.cpu().xscpu_init(max_threads)

    def rel(cpu_out, gpu_out, res):
        moe = gpu_out - res
        return float(np.max(np.abs(cpu_out - gpu_out)) / np.max(np.abs(moe)))

    # config 2, T = 1: one host copy of the layer (128 experts, 392 MB), the 16 disjoint 8-expert sets of the GPU
    # rotation, so 16 calls read every expert once
    host = arena[:E].reshape(-1).cpu().numpy()
    ol = xo.layout(xm.Q4_K, xm.Q6_K, H, F)
    n_sets = E // k
    lg = set_logits(torch, n_sets, 1, E, k, dev, gen)
    x = torch.randn(1, H, device=dev, generator=gen).to(torch.bfloat16).float()
    res = torch.randn(1, H, device=dev, generator=gen)
    us2 = xo.cpu_time(ol, host, L.bytes, E, k, x.cpu().numpy(), lg.cpu().numpy(), res.cpu().numpy())
    out = torch.empty(1, H, device=dev)
    xm.MoeLayer(L, arena, E, k, 1)(x, lg[0], res, out)
    c_out = xo.cpu_layer_decode(ol, host, L.bytes, E, k, x.cpu().numpy(), lg[0].cpu().numpy(), res.cpu().numpy())
    r2 = rel(c_out, out.cpu().numpy(), res.cpu().numpy())
    gbs2 = k * L.bytes / (us2 * 1e-6) / 1e9
    log(f"cpu baseline config 2 T=1: {us2:.1f} us/token, {gbs2:.2f} GB/s on {threads} threads; rel to GPU {r2:.2e}")
    # config 1: hidden 1024, 8 Q8_0 experts, top-2, F 512, fp32 router N(0, 0.02), N(0,1) activations, seed 0; 32
    # copies of the 13 MB layer in host memory, as 256 experts of which a call's logits enable one copy's 8
    E1, H1, F1, k1, copies = 8, 1024, 512, 2, 32
    arena1, L1 = xm.build_arena(E1, H1, F1, xm.Q8_0, xm.Q8_0, seed=0)
    ol1 = xo.layout(xm.Q8_0, xm.Q8_0, H1, F1)
    host1 = np.tile(arena1[:E1].reshape(-1).cpu().numpy(), copies)
    g0 = torch.Generator().manual_seed(0)
    wr = torch.randn(E1, H1, generator=g0) * 0.02
    c1 = {}
    for T in (4, 1):
        x1 = torch.randn(T, H1, generator=g0)
        res1 = torch.randn(T, H1, generator=g0)
        lg1 = xm.router_logits_f32(x1.to(dev), wr.to(dev))                   # the decode GEMV's order
        sets = np.full((copies, T, E1 * copies), -1e30, np.float32)
        for c in range(copies):
            sets[c, :, c * E1:(c + 1) * E1] = lg1.cpu().numpy()
        us1 = xo.cpu_time(ol1, host1, L1.bytes, E1 * copies, k1, x1.numpy(), sets, res1.numpy())
        o1 = torch.empty(T, H1, device=dev)
        xm.MoeLayer(L1, arena1, E1, k1, T)(x1.to(dev), lg1, res1.to(dev), o1)
        co1 = xo.cpu_layer_decode(ol1, host1, L1.bytes, E1, k1, x1.numpy(), lg1.cpu().numpy(), res1.numpy())
        r1 = rel(co1, o1.cpu().numpy(), res1.numpy())
        ids = torch.topk(lg1, k1, dim=1).indices
        b1 = len(torch.unique(ids)) * L1.bytes
        c1[f"T{T}"] = dict(us_per_layer=round(us1, 2), us_per_token=round(us1 / T, 2),
                           expert_gbs=round(b1 / (us1 * 1e-6) / 1e9, 2), rel_to_gpu=float(f"{r1:.3e}"))
        log(f"cpu baseline config 1 T={T}: {us1:.1f} us/layer, {c1[f'T{T}']['expert_gbs']} GB/s; rel to GPU "
            f"{r1:.2e}")
    del arena1
    return dict(value=round(1e6 / us2, 1), unit="tokens/s", cores=threads, kind="port",
                sample="config 2, one token a call: the best of 5 means of 10 calls (after 2), the calls rotating "
                       "over the 16 disjoint 8-expert sets of one 392 MB host copy (every 16 calls read all 128 "
                       "experts from DRAM); config 1 likewise over 32 host copies of its 13 MB layer",
                us_per_token=round(us2, 1), expert_gbs=round(gbs2, 2), rel_to_gpu=float(f"{r2:.3e}"),
                cpu=cpu_info(), threads="one a physical core, pinned, at most 16 (the box's CPU share)",
                path="oracle/cpu_path.cpp: Q8_K activations, AVX2 multi-token Q4_K/Q6_K rows, SwiGLU "
                     "g/(1+exp(-g))*u, h re-quantized to Q8_K, rank-order combine (src/kernels/cpu/"
                     "native_expert.cpp, iq_avx2_rows.inl); the float accumulation order is this file's",
                config1=c1)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--copies", type=int, default=8, help="distinct HBM copies of the layer's weights to rotate over")
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-others", action="store_true", help="skip configs 3 (verify), 4 and 5")
    ap.add_argument("--no-live-pmc", action="store_true",
                    help="take roofline.traffic from the committed rocprofv3 summary instead of two --pmc passes")
    ap.add_argument("--pmc-run", action="store_true", help="only the short workload of a rocprofv3 --pmc pass")
    ap.add_argument("--pmc-prefill", action="store_true", help="only 4 prefill layers, for a rocprofv3 --pmc pass")
    ap.add_argument("--pmc-verify", action="store_true",
                    help="only a rotation of config 3's verify layers (T=4, Zipf), for a rocprofv3 --pmc pass")
    ap.add_argument("--prefill-split", type=int, default=1, choices=(0, 1, 2),
                    help="the prompt layer's tall-tile split (xs_moe_set_prefill_tall): 1 on (the default), 0 off, 2 "
                         "its two chains one after the other (each kernel then times alone)")
    ap.add_argument("--pmc-c5dec", action="store_true", help="only config 5's one-token rotation, for a rocprofv3 pass")
    ap.add_argument("--pmc-tput", action="store_true",
                    help="only config-2 T=16 and config-4 T=8 decode rotations, for a rocprofv3 --pmc pass")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build's MoE path runs on a single MI355X (no multi-GPU path); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import xsmoe as xm

    dev = "cuda:0"
    torch.cuda.set_device(0)
    xm.lib().xs_moe_set_prefill_tall(args.prefill_split)
    if args.pmc_run:
        pmc_run(torch, xm, args.copies)
        return
    if args.pmc_prefill:
        pmc_prefill(torch, xm)
        return
    if args.pmc_tput:
        pmc_tput(torch, xm)
        return
    if args.pmc_c5dec:
        pmc_c5dec(torch, xm)
        return
    if args.pmc_verify:
        pmc_verify(torch, xm)
        return
    E, H, F, k = 128, 2048, 768, 8
    copies = args.copies
    log(f"building {copies} copies of the config-2 layer ({E} experts, Q4_K/Q6_K)")
    arena, L = xm.build_arena(E, H, F, xm.Q4_K, xm.Q6_K, seed=0, copies=copies)
    blob = L.bytes
    layer_bytes = E * blob
    log(f"arena {copies * layer_bytes / 1e9:.2f} GB, blob {blob} B")
    gen = torch.Generator(device=dev).manual_seed(1)

    inputs = {}

    def decode_run(T, steps, warmup):
        """Time exactly `steps` decode layer steps of T tokens after `warmup` untimed ones; returns (ms/step,
        bytes/step).  Steps rotate over (copy, logit set) pairs, copy first, so consecutive steps read other copies
        and, at T = 1, other experts: one token's 8 experts are the 8 boosted ones of its set (16 disjoint sets cover
        all 128 experts), so a cycle of 8 copies x 16 sets reads all 3.13 GB once and no step finds its blobs in the
        256 MB Infinity Cache.  T > 1: i.i.d. N(0,1) logits per set (uniform routing), 8 sets.  The warm-up takes the
        pairs before the timed ones in the same cycle.  The inputs stay in `inputs[T]` (logits, x)."""
        if T == 1:
            n_sets = E // k
            logits = set_logits(torch, n_sets, T, E, k, dev, gen)
        else:
            n_sets = copies
            logits = torch.randn(n_sets, T, E, device=dev, generator=gen)
        x = torch.randn(T, H, device=dev, generator=gen).to(torch.bfloat16).float()
        res = torch.randn(T, H, device=dev, generator=gen)
        out = torch.empty(T, H, device=dev)
        layer = xm.MoeLayer(L, arena, E, k, T)
        inputs[T] = (logits, x)
        cycle = [(i % copies, (i // copies) % n_sets) for i in range(copies * n_sets)]

        def calls(first, n):
            return [(lambda c=c, s=s: layer(x, logits[s], res, out, arena=arena[c * E]))
                    for c, s in (cycle[(first + i) % len(cycle)] for i in range(n))]

        timed = calls(warmup, steps)
        if warmup:
            run_graph(torch, calls(0, warmup))
        ms = run_graph(torch, timed) / steps
        pairs = [cycle[(warmup + i) % len(cycle)] for i in range(steps)]
        distinct = [len(torch.unique(torch.topk(logits[s], k, dim=1).indices)) for _, s in pairs]
        return ms, float(np.mean(distinct)) * blob

    # ---------------------------------------------------------------- decode, batch 1 (the value)
    ms1, bytes1 = decode_run(1, args.steps, args.warmup)
    gbs1 = bytes1 / (ms1 * 1e-3) / 1e9
    log(f"decode T=1: {ms1 * 1e3:.2f} us/layer, {gbs1:.0f} GB/s expert weights")

    # ---------------------------------------------------------------- the dominant kernel: the fused decode layer
    # At T = 1 the layer is one launch (moe_decode_t1_kernel), so the per-step time above is that kernel's average
    # launch duration: events on the stream the graph replays on bracket the replays.  Algorithmic bytes per launch =
    # the distinct experts' blob bytes.
    roof_bytes = bytes1
    roof_us = ms1 * 1e3
    roof_gbs = roof_bytes / (roof_us * 1e-6) / 1e9
    traffic, traffic_source = (None, "not measured (--no-live-pmc)") if args.no_live_pmc else live_traffic()
    if traffic is None:
        log(f"live HBM traffic: {traffic_source}; the committed summary's figure instead")
        traffic = read_traffic()
        traffic_source = (f"{TRAFFIC_FILE.relative_to(ROOT)}: rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE of the same "
                          "rotation (bench.py --pmc-run), scaled by a copy kernel of known size; read from the "
                          f"committed summary, not measured in this run ({traffic_source})") if traffic else None
    log(f"fused decode kernel: {roof_us:.2f} us/launch, {roof_gbs:.0f} GB/s of {roof_bytes / 1e6:.2f} MB"
        + (f", HBM traffic {traffic / 1e6:.2f} MB/launch ({traffic_source.split(':')[0]})" if traffic else ""))

    # ---------------------------------------------------------------- this box's achieved peaks
    peaks = measured_peaks(torch, xm, arena, int(round(roof_bytes)) // 16 * 16)

    # ---------------------------------------------------------------- decode batches 4 and 16, verify 4
    extra = {}
    for T in (4, 16):
        ms, b = decode_run(T, max(copies, args.steps // 4), copies)
        extra[f"T{T}"] = dict(us_per_layer=round(ms * 1e3, 2), us_per_token=round(ms * 1e3 / T, 3),
                              tokens_per_s=round(T / (ms * 1e-3), 1), expert_gbs=round(b / (ms * 1e-3) / 1e9, 1),
                              frac_hbm_peak=round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                              distinct_experts=round(b / blob, 2))
        log(f"decode T={T}: {ms * 1e3:.2f} us/layer, {extra[f'T{T}']['expert_gbs']} GB/s")

    # ---------------------------------------------------------------- prefill 2048 tokens, Zipf(1.2) routing
    Tp = 2048
    rng = np.random.default_rng(3)
    pop = -1.2 * np.log(np.arange(1, E + 1))[rng.permutation(E)]
    if not args.no_others:   # config 3's spec-verify batch: 4 tokens, Zipf(1.2) routing, one step per copy
        zv = torch.from_numpy((pop[None, None, :] + rng.gumbel(size=(copies, 4, E))).astype(np.float32)).to(dev)
        xv = torch.randn(4, H, device=dev, generator=gen).to(torch.bfloat16).float()
        rv = torch.randn(4, H, device=dev, generator=gen)
        ov = torch.empty(4, H, device=dev)
        vlayer = xm.MoeLayer(L, arena, E, k, 4)
        ms_v = time_steps(torch, [(lambda c=c: vlayer(xv, zv[c], rv, ov, arena=arena[c * E])) for c in range(copies)],
                          max(copies, args.steps // 4), copies)
        bv = distinct_experts(torch, zv, k) * blob
        extra["config3_verify_T4_zipf"] = dict(us_per_layer=round(ms_v * 1e3, 2),
                                                expert_gbs=round(bv / (ms_v * 1e-3) / 1e9, 1),
                                                frac_hbm_peak=round(bv / (ms_v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                                distinct_experts=round(bv / blob, 2))
        log(f"config 3 verify T=4 (Zipf): {ms_v * 1e3:.2f} us/layer, {extra['config3_verify_T4_zipf']['expert_gbs']} "
            f"GB/s")
    zl = torch.from_numpy((pop[None, :] + rng.gumbel(size=(Tp, E))).astype(np.float32)).to(dev)
    xp = torch.randn(Tp, H, device=dev, generator=gen).to(torch.bfloat16).float()
    rp = torch.randn(Tp, H, device=dev, generator=gen)
    op = torch.empty(2, Tp, H, device=dev)
    player = xm.MoeLayer(L, arena, E, k, Tp, prefill=True)
    pc = min(2, copies)

    def prefill_round():
        for c in range(pc):
            player(xp, zl, rp, op[c], arena=arena[c * E])

    ms_p = best_of_means(torch, prefill_round, max(1, args.prefill_steps // pc)) / pc
    flops = 6.0 * Tp * k * H * F
    tf = flops / (ms_p * 1e-3) / 1e12
    log(f"prefill T={Tp}: {ms_p * 1e3:.1f} us/layer, {tf:.1f} TFLOP/s")
    prefill = dict(tokens=Tp, us_per_layer=round(ms_p * 1e3, 1), tflops=round(tf, 2),
                   frac_mfma_peak=round(tf / BF16_PEAK_TFLOPS, 4),
                   frac_measured_mfma=round(tf / peaks["mfma_f16_tflops"], 4), mfma="f16 operands, fp32 accumulate (dense peak "
                   "2.5 PFLOP/s, as bf16)", tokens_per_s=round(Tp / (ms_p * 1e-3), 0),
                   flops_per_layer=flops, routing="Zipf alpha=1.2 (Gumbel-top-k)",
                   split={0: "off: every row on the 128/64-row GEMMs",
                          1: "whole 256-row tiles on the tall-tile GEMMs, the rest beside them on a side stream",
                          2: "tall-tile and remainder chains one after the other"}[args.prefill_split],
                   timing=f"best of 5 means of {max(1, args.prefill_steps // pc)} graph replays of {pc} layers "
                          "(two HBM copies of the weights)")

    others = {} if args.no_others else other_configs(torch, xm, dev, gen, max(64, args.steps // 4))

    # ---------------------------------------------------------------- the CPU baseline (the reference's CPU path)
    cpu = None if args.no_cpu else cpu_baseline(torch, xm, np, arena, L, E, H, F, k, dev, gen)

    line = {
        "metric": METRIC,
        "value": round(gbs1, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms1, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: N(0,0.02) fp32 weights quantized by this library's quantizer, bf16 N(0,1) activations, "
                "uniform routing (i.i.d. N(0,1) logits)",
        "config": {"workload": "config 2 decode batch 1: Qwen3-30B-A3B-shaped MoE layer (hidden 2048, 128 experts, "
                               "top-8, F 768, Q4_K gate/up, Q6_K down), weights rotated over "
                               f"{copies} HBM copies ({copies * layer_bytes / 1e9:.2f} GB)",
                   "global_batch": 1, "seq_len": 1, "parallelism": "none (1 GPU)"},
        "us_per_token": round(ms1 * 1e3, 3),
        "tokens_per_s": round(1.0 / (ms1 * 1e-3), 1),
        "frac_hbm_peak": round(gbs1 / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(roof_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(roof_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "frac_measured_stream": round(roof_gbs / peaks["hbm_stream_gbs"], 4),
                     "frac_measured_one_launch": round(roof_gbs / peaks["hbm_one_launch_gbs"], 4),
                     "traffic_source": traffic_source,
                     "kernel": "moe_decode_t1_kernel<Q4_K, Q6_K, 2, 2048, 768, 8> (xs_moe_layer_decode at one token, "
                               "one launch a layer)",
                     "algorithmic_bytes_per_launch": round(roof_bytes), "avg_launch_us": round(roof_us, 3)},
        "measured_peaks": peaks,
        "decode_batches": extra,
        "prefill": prefill,
        "other_configs": others,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
