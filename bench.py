#!/usr/bin/env python3
"""Decode-attention benchmark of the compressed-KV path on one MI355X.

Workload (default c2a, the headline shape): Llama-3.1-8B attention, 32 query / 8 KV heads,
head dim 128, batch 8 x 8,192 context, page 16, synthetic K/V of the configuration-0 recipe
(RoPE'd keys with per-channel scales, 0.04% zeros, 0.3% raw rows). One step = one decode
attention call (split kernel + merge) over the compressed cache, inputs resident in HBM.
The Infinity Cache (256 MB) is defeated by rotating over several cache copies.

Prints one JSON line: value = microseconds per call (lower is better), the roofline of the
dominant kernel (the split kernel: algorithmic bytes / its average duration, HIP events on
the launch stream), the bf16-uncompressed twin for comparison, the encoder's throughput,
and the CPU baseline (the reference codec restated in PyTorch decoding both caches, then
fp32 attention, on every host core this process may use; median of full calls).
The default line also carries the metric's second half, `e2e`: c4 greedy decode tok/s of
both caches (random-init Llama-3.1-8B, 4096-token prompts, 256 tokens, each cache at the
largest batch its KV budget holds), from `--workload e2e --e2e-rows own` run first as a
child process (about 2.5 minutes; --no-e2e leaves it out).
--workload cpu times that baseline at every benchmark shape without the GPU.

    python bench.py [--steps 400] [--warmup 200] [--workload c2a]
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode-attn µs & % HBM peak at 32q/8kv, 8×8K ctx; e2e greedy decode tok/s"
HBM_PEAK_GBPS = 8000.0

WORKLOADS = {   # name: (B, T, TS, Hq, Hkv, description)
    "c2a": (8, 8192, 8192, 32, 8, "Llama-3.1-8B decode attention 32q/8kv, B8 x 8192 ctx"),
    "c2a_ragged": (8, 8185, 8192, 32, 8, "Llama-3.1-8B decode attention 32q/8kv, B8 x 8185 ctx (partial page)"),
    "c2b": (1, 131072, 131072, 32, 8, "Llama-3.1-8B decode attention 32q/8kv, B1 x 131072 ctx"),
    "c1": (1, 32768, 32768, 28, 4, "Qwen2.5-7B decode attention 28q/4kv, B1 x 32768 ctx"),
    # a serving batch: long splits (one per sequence at head dims 64 / 256)
    "long": (128, 4352, 4352, 32, 8, "decode attention 32q/8kv, B128 x 4352 ctx (serving batch)"),
}


def profiled_traffic(workload):
    """HBM bytes per split-kernel launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary of this workload (scaled by the copy-kernel calibration), or None."""
    path = os.path.join(ROOT, "profiles", f"attn_split_{workload}_traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return None, None
    if d.get("workload") != workload:
        return None, None
    return int(d["traffic_bytes"]), os.path.relpath(path, ROOT)


def cpu_model():
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def algorithmic_bytes(caches, B, T, Hq, Hkv, lens=None, window=0, D=128):
    """Bytes a decode-attention call must move: per K/V cache and valid token row
    D (sm) + D/2 (code); per touched page and head D (base) + 8 (rowmask, rowoff);
    2 D per raw row referenced; plus q and the output (head dim D: 192 + 136 per page +
    256 per raw row at 128). lens: per-sequence lengths; window: only each sequence's last
    `window` tokens count."""
    import torch
    lens = [T] * B if lens is None else [int(x) for x in lens]
    total = 0
    for c in caches:
        for b, L in enumerate(lens):
            lo = max(L - window, 0) if window else 0
            p0, npg = lo // 16, -(-L // 16)
            rm = c.rowmask[b, p0:npg].to(torch.int64)                       # [pages, Hkv]
            bit = torch.arange(16, device=rm.device)
            tok = torch.arange(p0, npg, device=rm.device)[:, None] * 16 + bit   # [pages, 16]
            raw = (rm[:, :, None] >> bit) & 1                                 # [pages, Hkv, 16]
            raw_rows = int((raw * ((tok < L) & (tok >= lo))[:, None, :]).sum().item())
            total += (L - lo) * Hkv * (3 * D // 2) + (npg - p0) * Hkv * (D + 8) + raw_rows * 2 * D
    return total + 2 * B * Hq * D * 2


MALL_BYTES = 256 << 20


def rotation_copies(read_bytes, most=16):
    """Cache copies to rotate over: at least 4, and enough that the compressed bytes the calls
    read add up to twice the 256 MiB Infinity Cache, so that no call finds its cache there
    (c1 reads 53 MB per call: 4 copies would fit), but at most `most` (a short window reads
    a few MB per call, which no practical rotation keeps out of the cache)."""
    return min(most, max(4, -(-2 * MALL_BYTES // int(read_bytes))))


def gpu_lead():
    """Keep the GPU busy for about a millisecond ahead of a timed region: the calls that
    follow are queued while it spins, so the first event does not start an interval in which
    the GPU waits for the host to launch the first call (with 20 timed calls, that wait
    would add a few tenths of a microsecond to each)."""
    import torch
    torch.cuda._sleep(2_000_000)


def nearby_plans(ns, sl, T):
    """Split plans around (ns, sl) for T tokens: 0.5, 0.75, 1, 1.5 and 2 times the split
    count, split lengths rounded up to whole 16-token pages (the planner's own choices for
    other workgroup targets, for any head dim)."""
    out = []
    for m in (0.5, 0.75, 1.0, 1.5, 2.0):
        n = max(1, round(ns * m))
        s = -(-(-(-T // n)) // 16) * 16
        p = (-(-T // s), s)
        if p not in out:
            out.append(p)
    return out


def time_loop(fn, n, warmup, copies):
    """Average ms per call of fn(i) over n calls, rotating over `copies` inputs, timed with
    HIP events on the current stream (the stream every call launches on)."""
    import torch
    for i in range(warmup):
        fn(i % copies)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    gpu_lead()
    e0.record(s)
    for i in range(n):
        fn(i % copies)
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n


def settle(fns, copies, seconds=0.5):
    """Run the calls untimed, in turn, until `seconds` of wall time have passed, so that the
    GPU is at its steady clocks before the timed loops whatever --warmup is (a short warmup
    leaves it below them: +1-3 us per call). Returns the number of calls made."""
    import torch
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(50):
            for f in fns:
                f(n % copies)
            n += 1
        torch.cuda.synchronize()
    return n * len(fns)


def time_calls(fn, n, warmup, copies):
    """Per-call times (ms): an event before each call and after the last, all on the launch
    stream; returns (median, p10, p90)."""
    import torch
    for i in range(warmup):
        fn(i % copies)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    gpu_lead()
    for i in range(n):
        ev[i].record(s)
        fn(i % copies)
    ev[n].record(s)
    torch.cuda.synchronize()
    t = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(n))
    return t[n // 2], t[n // 10], t[(9 * n) // 10]


def _hip():
    """The HIP runtime torch has loaded (for raw event calls)."""
    import ctypes
    import torch
    lib = ctypes.CDLL(os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so"))
    lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
    return lib


def time_split_kernel(launch, n, warmup, copies):
    """Average and median ms of the split kernel itself: each of n calls of launch(i) (rotating
    over `copies` inputs, back to back; a full call, or the split kernel alone) has the pair of
    HIP events of exkv_time_next_split recorded at its split kernel's own start and end on the
    launch stream (hipExtLaunchKernelGGL)."""
    import ctypes
    import torch
    from exactkv_amd import _lib
    lib, hip = _lib.load(), _hip()
    for i in range(warmup):
        launch(i % copies)
    torch.cuda.synchronize()
    ev = []
    for _ in range(2 * n):
        e = ctypes.c_void_p()
        assert hip.hipEventCreate(ctypes.byref(e)) == 0
        ev.append(e)
    for i in range(n):
        lib.exkv_time_next_split(ev[2 * i], ev[2 * i + 1])
        launch(i % copies)
    torch.cuda.synchronize()
    t = []
    for i in range(n):
        ms = ctypes.c_float()
        assert hip.hipEventElapsedTime(ctypes.byref(ms), ev[2 * i], ev[2 * i + 1]) == 0
        t.append(ms.value)
    for e in ev:
        hip.hipEventDestroy(e)
    t.sort()
    return sum(t) / n, t[n // 2]


def time_graph(fn, n, warmup, copies, per_graph=32):
    """Average ms per call of fn(i) with the calls captured in a HIP graph (per_graph calls
    rotating over `copies` inputs) and the graph replayed until n calls ran: the launch
    path of a captured decode step, with no Python work between kernels. 32 calls per
    graph are the attention calls of one 32-layer decode step (the engine captures a whole
    step); each graph launch itself costs ~25 us on top of its calls, which graphs of 1-4
    calls would charge to every call (c2a: +1.2-2 us per call). Workspaces are
    allocated by eager calls on the capture stream beforehand; the graph is replayed
    untimed (at least 8 times, about 10 ms at c2a) before the timed replays; timed with
    HIP events on the stream the graph is launched on."""
    import torch
    cs = torch.cuda.Stream()
    with torch.cuda.stream(cs):
        for i in range(max(warmup, copies)):
            fn(i % copies)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        for i in range(per_graph):
            fn(i % copies)
    torch.cuda.synchronize()
    reps = max(1, -(-n // per_graph))
    with torch.cuda.stream(cs):
        # untimed replays first, as the eager loops have their warmup: the first replays of a
        # new graph can run a few us per call slower for a few ms (measured at c2a: replays
        # 3-6 of 16 at 42.7-44.2 against 39.7-40.6 us per call later)
        for _ in range(max(8, -(-warmup // per_graph))):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        gpu_lead()
        e0.record(cs)
        for _ in range(reps):
            g.replay()
        e1.record(cs)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * per_graph)


def graph_cost_split(fn, warmup, copies, small=32, large=128, reps=8):
    """Graph replay time t(n) of graphs of n calls = F + n * c: the marginal cost c of a call
    inside a graph and the fixed cost F of launching one graph, from graphs of `small` and
    `large` calls (each replayed `reps` times back to back, HIP events on the launch stream).
    graph_replay_us (graphs of 32 calls) is c + F / 32."""
    t_small = time_graph(fn, small * reps, warmup, copies, per_graph=small)
    t_large = time_graph(fn, large * reps, warmup, copies, per_graph=large)
    c = (large * t_large - small * t_small) / (large - small)
    return {"per_call_us": round(c * 1e3, 2), "per_graph_launch_us": round((t_small - c) * small * 1e3, 1),
            "calls_per_graph": [small, large]}


def cpu_threads():
    """Host threads for the CPU baseline: every core this process may run on."""
    return len(os.sched_getaffinity(0))


def host_cache(c, nseq=None):
    """A compressed cache's six tensors and shape as CPU tensors (the first nseq sequences)."""
    import torch
    d = {k: (getattr(c, k)[:nseq] if nseq else getattr(c, k)).cpu() for k in ("sm", "code", "base", "rowmask", "rowoff")}
    d["raw"] = c.raw.cpu()
    d["shape"] = (nseq or c.B, c.TS, c.H, c.D)
    return d


def median_seconds(fn, runs):
    """Median and minimum wall time of `runs` calls of fn (time.perf_counter)."""
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2], ts[0]


def cpu_baseline(kc, vc, q, B, T, runs, lens=None):
    """The reference codec restated in PyTorch (oracle.torch_codec, byte-identical to
    codec.py) decoding both caches, then fp32 GQA attention, on every host core this process
    may use; the median of `runs` full calls, in microseconds."""
    import torch
    from oracle import torch_codec
    n = cpu_threads()
    torch.set_num_threads(n)
    hk, hv, hq = host_cache(kc), host_cache(vc), q.cpu()
    med, best = median_seconds(lambda: torch_codec.decode_attention(hq, hk, hv, T, lens=lens), runs)
    return dict(value=round(med * 1e6, 1), unit="us", cores=n, kind="port",
                sample=f"median of {runs} full calls on the same caches ({B} x {T} tokens): torch restatement "
                       f"of the reference codec decoding K and V, then fp32 GQA attention",
                min_us=round(best * 1e6, 1), cpu=cpu_model(), torch_threads=torch.get_num_threads())


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default: 400 for the attention shapes, 50 for the other workloads)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed warmup steps (default: 200 for the attention shapes, 10 otherwise); a short "
                         "warmup leaves the GPU below its steady clocks, which shows as +1-3 us per call")
    ap.add_argument("--workload", default="c2a",
                    choices=sorted(WORKLOADS) + ["c3", "e2e", "c2a_paged", "wire", "prefill", "e2e_paged", "cpu"])
    ap.add_argument("--e2e-prompt", type=int, default=4096)
    ap.add_argument("--e2e-gen", type=int, default=256)
    ap.add_argument("--e2e-batch", type=int, default=0, help="cap the e2e batch (0: as many as fit)")
    ap.add_argument("--e2e-model", default="llama3.1-8b", choices=sorted(E2E_MODELS),
                    help="the e2e model's shape (random init): c4's Llama-3.1-8B, or Llama-3.2-1B (head dim 64)")
    ap.add_argument("--e2e-work-gib", type=float, default=6.0,
                    help="memory kept free beyond the caches for activations, logits and pool growth")
    ap.add_argument("--e2e-rows", default="all", choices=("all", "own"),
                    help="e2e runs: 'own' = each cache at its own largest batch; 'all' adds the compressed cache "
                         "at the bf16 batch (same work: step-time ratio and token identity)")
    ap.add_argument("--no-e2e", action="store_true",
                    help="default line without its e2e leg (c4 decode tok/s of both caches, run first as a child "
                         "process: about 2.5 minutes)")
    ap.add_argument("--e2e-timeout", type=float, default=420.0,
                    help="seconds the default line's e2e child may take before it is stopped and reported as such")
    ap.add_argument("--copies", type=int, default=None,
                    help="cache copies rotated to defeat the 256 MB MALL (default: at least 4, and enough that "
                         "the compressed copies of the attention shapes hold twice the MALL)")
    ap.add_argument("--cpu-runs", type=int, default=5, help="CPU baseline: median of this many runs")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--target-blocks", type=int, default=None)
    ap.add_argument("--window", type=int, default=0,
                    help="sliding-window attention over each sequence's last WINDOW tokens (0: all)")
    ap.add_argument("--head-dim", type=int, default=128, choices=(64, 128, 256),
                    help="head dim of the attention shapes (64 and 256 run the generic-head-dim kernels; "
                         "the workload's heads and context stay)")
    ap.add_argument("--profile", action="store_true",
                    help="counter-collection run: a 256 MiB copy kernel (for scaling FETCH_SIZE / WRITE_SIZE), "
                         "then a few launches of each attention kernel (with --workload c3: of the encoder "
                         "over the prefill's keys); no timing")
    a = ap.parse_args()
    attn = a.workload in WORKLOADS or a.workload in ("c3", "c2a_paged")
    if a.steps is None:
        a.steps = 400 if attn else 50
    if a.warmup is None:
        a.warmup = 200 if attn else 10
    if a.workload in ("e2e", "c3", "c2a_paged", "wire", "prefill", "e2e_paged", "cpu"):
        if a.copies is None:
            a.copies = 4
        if a.gpus != 1:
            print("bench.py measures one GPU", file=sys.stderr)
            sys.exit(2)
        return {"e2e": e2e, "c3": c3_stress, "c2a_paged": paged_c2a, "wire": wire_bench,
                "prefill": prefill_bench, "e2e_paged": e2e_paged, "cpu": cpu_sweep}[a.workload](a)
    if a.profile:
        a.copies = 1
    if a.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {a.gpus} is not supported in this build "
              "(the decode path shards by KV head or sequence with no exchange)", file=sys.stderr)
        sys.exit(2)

    B, T, TS, Hq, Hkv, desc = WORKLOADS[a.workload]
    D = a.head_dim
    default_line = a.workload == "c2a" and D == 128 and not a.window and not a.profile and not a.target_blocks

    import torch
    import exactkv_amd as exactkv
    from exactkv_amd import kernels, synthetic

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if a.copies is None:                               # sized on the tokens a call reads (a window's only)
        a.copies = rotation_copies(2 * B * (min(T, a.window + 15) if a.window else T) * Hkv * D * 200.5 / 128)
    if D != 128:
        desc = f"{desc}, head dim {D}"
    # the c4 protocol's sequences-fit on this GPU, before the workload's data takes memory
    fit = e2e_fit() if default_line else None
    print(f"[bench] {a.workload}: {desc}; generating data", file=sys.stderr, flush=True)
    k = synthetic.make_kv(B, TS, Hkv, D=D, kind="k", seed=100, device=dev)
    v = synthetic.make_kv(B, TS, Hkv, D=D, kind="v", seed=101, device=dev)
    q = synthetic.make_q(B, Hq, D=D, seed=102, device=dev)
    kcs, vcs, kbs, vbs = [], [], [], []
    for i in range(a.copies):
        kc, vc = exactkv.CompressedKV(B, TS, Hkv, D), exactkv.CompressedKV(B, TS, Hkv, D)
        for b in range(B):
            kc.prefill_slot(b, k[b:b + 1, :T])
            vc.prefill_slot(b, v[b:b + 1, :T])
        kcs.append(kc)
        vcs.append(vc)
        kbs.append(k.clone())
        vbs.append(v.clone())
    del k, v
    torch.cuda.synchronize()
    print("[bench] caches encoded", file=sys.stderr, flush=True)
    W = a.window
    reach = min(T, W + 15) if W else T                 # the splits start at the window's first page
    if a.target_blocks or D == 128:
        ns, sl = kernels.plan_splits(B, Hkv, Hq, reach, **({"target_blocks": a.target_blocks} if a.target_blocks else {}))
    else:
        ns, sl = kernels.plan_splits_hd(B, Hkv, Hq, reach, D)
    out = torch.empty_like(q)
    if a.profile:
        profile_run(kernels, q, kcs[0], vcs[0], kbs[0], vbs[0], T, ns, sl, out)
        return
    o_c = kernels.attention_compressed(q, kcs[0], vcs[0], T, nsplit=ns, split_len=sl, window=W)
    o_r = kernels.attention_reference(q, kbs[0], vbs[0], T, nsplit=ns, split_len=sl, window=W)
    identical = torch.equal(o_c.view(torch.int16), o_r.view(torch.int16))

    def full_c(i):
        kernels.attention_compressed(q, kcs[i], vcs[i], T, nsplit=ns, split_len=sl, out=out, window=W)

    def full_b(i):
        kernels.attention_reference(q, kbs[i], vbs[i], T, nsplit=ns, split_len=sl, out=out, window=W)

    settled = settle([full_c, full_b], a.copies)
    ms_c = time_loop(full_c, a.steps, a.warmup, a.copies)
    ms_b = time_loop(full_b, a.steps, a.warmup, a.copies)
    # the twin at plans around this one: bit-identity needs both kernels on one plan, but
    # the twin alone is faster on some others (fewer, longer splits), so its best is reported
    twin_plans = {}
    for ns2, sl2 in nearby_plans(ns, sl, reach):
        def full_b2(i, ns2=ns2, sl2=sl2):
            kernels.attention_reference(q, kbs[i], vbs[i], T, nsplit=ns2, split_len=sl2, out=out, window=W)
        twin_plans[f"{ns2}x{sl2}"] = time_loop(full_b2, a.steps, a.warmup, a.copies)
    twin_best = min(twin_plans, key=twin_plans.get)
    # the split kernels launched back to back (as the rocprofv3 kernel trace of this run times
    # them); inside full calls the events also catch the launch's setup behind the previous
    # call's merge, so that figure is an upper bound (kernel_us_in_calls)
    ms_split, ms_split_med = time_split_kernel(lambda i: split_only(kernels, q, kcs[i], vcs[i], T, ns, sl, True,
                                                                    window=W), max(a.steps, 50), a.warmup, a.copies)
    ms_split_b, _ = time_split_kernel(lambda i: split_only(kernels, q, kbs[i], vbs[i], T, ns, sl, False, window=W),
                                      max(a.steps, 50), a.warmup, a.copies)
    ms_split_calls, _ = time_split_kernel(full_c, max(a.steps, 50), a.warmup, a.copies)
    ms_c_graph = time_graph(full_c, max(a.steps, 200), a.warmup, a.copies)
    graph_split = graph_cost_split(full_c, a.warmup, a.copies)
    med, p10, p90 = time_calls(full_c, max(a.steps, 50), a.warmup, a.copies)
    print("[bench] attention timed", file=sys.stderr, flush=True)

    alg = algorithmic_bytes([kcs[0], vcs[0]], B, T, Hq, Hkv, window=W, D=D)
    alg_b = 2 * B * min(T, W or T) * Hkv * 2 * D + 2 * B * Hq * D * 2
    gbps = alg / (ms_split * 1e-3) / 1e9
    enc = encoder_gbps(exactkv, kernels, kbs[:2], T, a.steps, a.warmup)
    print("[bench] encoder timed", file=sys.stderr, flush=True)

    traffic, traffic_src = profiled_traffic(a.workload) if not W and D == 128 else (None, None)
    res = {
        "metric": METRIC, "value": round(ms_c * 1e3, 2), "unit": "us", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms_c, 5), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{a.workload}: {desc}", "B": B, "T": T, "TS": TS, "Hq": Hq, "Hkv": Hkv,
                   "head_dim": D, "page": 16, "nsplit": ns, "split_len": sl, "cache_copies": a.copies,
                   "parallelism": "single GPU", **({"window": W} if W else {})},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": traffic, "traffic_source": traffic_src,
                     "kernel": "attn_split_kernel<compressed>" if D == 128 else f"attn_dgen_kernel<{D}, compressed>",
                     "algorithmic_bytes": alg,
                     "kernel_us": round(ms_split * 1e3, 2), "kernel_us_median": round(ms_split_med * 1e3, 2),
                     "kernel_timing": "HIP events recorded at each split kernel's own start and end "
                                      "(hipExtLaunchKernelGGL) on its launch stream, back-to-back launches",
                     "kernel_us_in_calls": round(ms_split_calls * 1e3, 2)},
        "timing": "HIP events around back-to-back calls on one stream",
        "settle_calls": settled,
        "graph_replay_us": round(ms_c_graph * 1e3, 2),
        "graph_replay_calls": max(a.steps, 200),
        "graph_replay_split": graph_split,
        "per_call_us": {"median": round(med * 1e3, 2), "p10": round(p10 * 1e3, 2), "p90": round(p90 * 1e3, 2),
                        "calls": max(a.steps, 50)},
        "bf16_twin_us": round(ms_b * 1e3, 2),
        "bf16_split_us": round(ms_split_b * 1e3, 2),
        "bf16_split_GBps": round(alg_b / (ms_split_b * 1e-3) / 1e9, 1),
        "speedup_vs_bf16": round(ms_b / ms_c, 3),
        "speedup_vs_bf16_note": "both kernels on this plan (bit-identity needs one plan)",
        "bf16_twin_plans_us": {k: round(v * 1e3, 2) for k, v in twin_plans.items()},
        "bf16_twin_best_plan": twin_best,
        "bf16_twin_best_us": round(twin_plans[twin_best] * 1e3, 2),
        "speedup_vs_bf16_best_plan": round(twin_plans[twin_best] / ms_c, 3),
        "bit_identical_to_bf16": bool(identical),
        "bits_per_value": round((kcs[0].nbytes() + vcs[0].nbytes()) * 8 / (2 * B * TS * Hkv * D), 3),
        "encoder_GBps": enc,
        "gpu": torch.cuda.get_device_name(0),
    }
    if not a.no_cpu_baseline and not W and D == 128:   # the baseline is the full-context attention at the metric's shape
        res["cpu_baseline"] = cpu_baseline(kcs[0], vcs[0], q, B, T, a.cpu_runs)
        print("[bench] cpu baseline timed", file=sys.stderr, flush=True)
    if fit is not None:
        res["e2e_fit"] = fit
    if default_line and not a.no_e2e:
        # the metric's second half, c4 decode tok/s of both caches, last (two minutes of full
        # load before the attention timing would leave the GPU warmer than the other lines)
        del kcs, vcs, kbs, vbs, q, out, o_c, o_r
        kernels.release_workspaces()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        res["e2e"] = e2e_child(a)
    print(json.dumps(res), flush=True)


def paged_c2a(a):
    """c2a over paged caches: the 8 x 8192 tokens as 4096 pages scattered at random over a
    pool of 4160 pages (one 66,560-token sequence per array), block table [8, 512]."""
    import numpy as np
    import torch
    import exactkv_amd as exactkv
    from exactkv_amd import kernels, synthetic

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, T, Hq, Hkv, POOL = 8, 8192, 32, 8, 4160
    npg = T // 16
    print("[paged] generating data", file=sys.stderr, flush=True)
    q = synthetic.make_q(B, Hq, seed=102, device=dev)
    kcs, vcs, kbs, vbs, bts = [], [], [], [], []
    for i in range(a.copies):
        k = synthetic.make_kv(1, POOL * 16, Hkv, kind="k", seed=300 + i, device=dev)
        v = synthetic.make_kv(1, POOL * 16, Hkv, kind="v", seed=400 + i, device=dev)
        kc, vc = exactkv.CompressedKV(1, POOL * 16, Hkv, 128), exactkv.CompressedKV(1, POOL * 16, Hkv, 128)
        kc.prefill_slot(0, k)
        vc.prefill_slot(0, v)
        perm = np.random.Generator(np.random.PCG64(500 + i)).permutation(POOL)[:B * npg]
        bts.append(torch.tensor(perm.reshape(B, npg), dtype=torch.int32, device=dev))
        kcs.append(kc)
        vcs.append(vc)
        kbs.append(k)
        vbs.append(v)
    torch.cuda.synchronize()
    print("[paged] pools encoded", file=sys.stderr, flush=True)
    ns, sl = kernels.plan_splits(B, Hkv, Hq, T)
    out = torch.empty_like(q)
    o_c = kernels.attention_compressed(q, kcs[0], vcs[0], T, nsplit=ns, split_len=sl, block_table=bts[0])
    o_r = kernels.attention_reference(q, kbs[0], vbs[0], T, nsplit=ns, split_len=sl, block_table=bts[0])
    identical = torch.equal(o_c.view(torch.int16), o_r.view(torch.int16))
    ms_c = time_loop(lambda i: kernels.attention_compressed(q, kcs[i], vcs[i], T, nsplit=ns, split_len=sl,
                                                            out=out, block_table=bts[i]), a.steps, a.warmup, a.copies)
    ms_b = time_loop(lambda i: kernels.attention_reference(q, kbs[i], vbs[i], T, nsplit=ns, split_len=sl, out=out,
                                                           block_table=bts[i]), a.steps, a.warmup, a.copies)
    ms_split, _ = time_split_kernel(lambda i: split_only(kernels, q, kcs[i], vcs[i], T, ns, sl, True,
                                                         block_table=bts[i]), max(a.steps, 50), a.warmup, a.copies)
    # algorithmic bytes: those of the gathered pages (the table's pages of the pool)
    alg = 0
    for c in (kcs[0], vcs[0]):
        rm = c.rowmask[0][bts[0].long().flatten()].to(torch.int64)           # [B * npg, Hkv]
        raw_rows = int(sum(((rm >> bit) & 1).sum().item() for bit in range(16)))
        alg += B * T * Hkv * 192 + B * npg * Hkv * 136 + raw_rows * 256
    alg += 2 * B * Hq * 128 * 2
    gbps = alg / (ms_split * 1e-3) / 1e9
    res = {
        "metric": "c2a decode-attn us over paged caches (block tables)", "value": round(ms_c * 1e3, 2), "unit": "us",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_c, 5), "higher_is_better": False,
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "c2a_paged: Llama-3.1-8B decode attention 32q/8kv, B8 x 8192 ctx, pages scattered "
                               "over a 4160-page pool", "B": B, "T": T, "Hq": Hq, "Hkv": Hkv, "pool_pages": POOL,
                   "nsplit": ns, "split_len": sl, "cache_copies": a.copies},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "attn_split_kernel<compressed> (paged)", "algorithmic_bytes": alg,
                     "kernel_us": round(ms_split * 1e3, 2)},
        "bf16_twin_us": round(ms_b * 1e3, 2), "speedup_vs_bf16": round(ms_b / ms_c, 3),
        "bit_identical_to_bf16": bool(identical), "gpu": torch.cuda.get_device_name(0),
    }
    print(json.dumps(res), flush=True)


def wire_bench(a):
    """Wire form at c2a's shape: pack the 8 sequences of a K and a V cache (B8 x 8192, 8 KV
    heads) into preallocated blobs (one pack call per cache per step), and unpack them into a
    second pair of caches (one unpack call per cache per step). HIP events around the
    launches; cache copies rotated. Algorithmic bytes per step: every blob byte read once and written once."""
    import numpy as np
    import torch
    import exactkv_amd as exactkv
    from exactkv_amd import _lib, kernels, synthetic, wire

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, T, H = 8, 8192, 8
    print("[wire] generating data", file=sys.stderr, flush=True)
    copies, raw_src = [], None
    for i in range(a.copies):
        pair = []
        for kind, seed in (("k", 600 + i), ("v", 700 + i)):
            x = synthetic.make_kv(B, T, H, kind=kind, seed=seed, device=dev)
            c = exactkv.CompressedKV(B, T, H, 128)
            for b in range(B):
                c.prefill_slot(b, x[b:b + 1])
            pair.append(c)
            if i == 0 and kind == "k":
                raw_src = x
        copies.append(pair)
    blobs = [[wire.pack(c, b) for b in range(B)] for c in copies[0]]
    sizes = [[int(bl.numel()) for bl in row] for row in blobs]
    total = sum(map(sum, sizes))
    dst = [exactkv.CompressedKV(B, T, H, 128, reserve=0.02) for _ in range(2)]
    for c, row in zip(dst, blobs):
        for b in range(B):
            wire.unpack(row[b], c, b)
    identical = all(torch.equal(kernels.decode_to_bf16(d.buffers(), T).view(torch.int16),
                                kernels.decode_to_bf16(s.buffers(), T).view(torch.int16))
                    for d, s in zip(dst, copies[0]))
    # one pack call per cache (8 sequences, two launches); one unpack call per cache
    pargs = [[wire._batch_args(c, list(range(B)), [wire._sequence(c, b) for b in range(B)], row, dev)
              for c, row in zip(pair, blobs)] for pair in copies]
    st = _lib.stream()

    def pack_all(i):
        for c, (d, width, max_t, wss) in zip(copies[i], pargs[i]):
            _lib.call("exkv_wire_pack", c.sm.data_ptr(), c.code.data_ptr(), c.base.data_ptr(), c.rowmask.data_ptr(),
                      c.rowoff.data_ptr(), c.raw.data_ptr(), c.raw.shape[0], B * (T // 16), B, d["pages"].data_ptr(),
                      width, d["tokens"].data_ptr(), d["tails"].data_ptr(), d["blobs"].data_ptr(),
                      d["sizes"].data_ptr(), max_t, H, 128, d["ws"].data_ptr(), wss, st)

    dargs = [wire._batch_args(c, list(range(B)), [wire._sequence(c, b) for b in range(B)], row, dev)
             for c, row in zip(dst, blobs)]

    def unpack_all(i):
        for c, (d, width, max_t, wss) in zip(dst, dargs):
            c.cnt.zero_()
            _lib.call("exkv_wire_unpack", c.sm.data_ptr(), c.code.data_ptr(), c.base.data_ptr(), c.rowmask.data_ptr(),
                      c.rowoff.data_ptr(), c.raw.data_ptr(), c.raw.shape[0], c.cap, c.cnt.data_ptr(),
                      c._before.data_ptr(), B * (T // 16), B, d["pages"].data_ptr(), width, d["tokens"].data_ptr(),
                      d["open"].data_ptr(), d["tails"].data_ptr(), d["blobs"].data_ptr(), d["sizes"].data_ptr(),
                      max_t, H, 128, d["ws"].data_ptr(), wss, st)

    ms_pack = time_loop(pack_all, a.steps, a.warmup, a.copies)
    ms_unpack = time_loop(unpack_all, a.steps, a.warmup, 1)
    gb_pack = 2 * total / (ms_pack * 1e-3) / 1e9
    gb_unpack = 2 * total / (ms_unpack * 1e-3) / 1e9
    bf16_bytes = 2 * B * T * H * 128 * 2
    cpu = None
    if not a.no_cpu_baseline:
        from oracle import wire as owire
        x0 = raw_src[0].cpu().view(torch.int16).numpy().view(np.uint16)
        t0 = time.perf_counter()
        n = 0
        while True:                                    # one sequence's K at a time, >= 3 s
            owire.pack(x0)
            n += 1
            if time.perf_counter() - t0 >= 3.0:
                break
        per_seq = (time.perf_counter() - t0) / n
        cpu = {"value": round(2 * sizes[0][0] / per_seq / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"oracle wire.pack (numpy encode + layout) of one 8192 x 8-head key sequence, {n} passes"}
    res = {
        "metric": "wire pack GB/s (blob bytes read + written) at c2a shape", "value": round(gb_pack, 1),
        "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_pack, 5),
        "higher_is_better": True, "vs_baseline": None, "dtype": "u8", "data": "synthetic",
        "config": {"workload": "wire: pack / unpack 8 sequences x (K, V) of B8 x 8192 x 8 heads", "B": B, "T": T,
                   "H": H, "blob_bytes": total, "bf16_bytes": bf16_bytes, "cache_copies": a.copies},
        "roofline": {"bound": "hbm", "achieved": round(gb_pack, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gb_pack / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "wire_scan_kernel + wire_copy_kernel (2 calls x 8 sequences)", "algorithmic_bytes": 2 * total},
        "unpack_GBps": round(gb_unpack, 1), "unpack_ms": round(ms_unpack, 5),
        "blob_vs_bf16": round(total / bf16_bytes, 4), "roundtrip_identical": bool(identical),
        "cpu_baseline": cpu, "gpu": torch.cuda.get_device_name(0),
    }
    print(json.dumps(res), flush=True)


def calibration_copy(dev):
    """The copy kernel that counter runs scale FETCH_SIZE / WRITE_SIZE by: torch.mul over
    64 Mi fp32 (256 MiB read + 256 MiB written). Returns the bytes read (= written)."""
    import torch
    n = 64 << 20
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    return n * 4


def profile_run(kernels, q, kc, vc, kb, vb, T, ns, sl, out):
    """Launch sequence for hardware-counter runs: the calibration copy, then 5 launches each
    of the compressed split kernel, the bf16 split kernel and the full compressed call."""
    import torch
    nbytes = calibration_copy(q.device)
    for _ in range(5):
        split_only(kernels, q, kc, vc, T, ns, sl, True)
    for _ in range(5):
        split_only(kernels, q, kb, vb, T, ns, sl, False)
    for _ in range(5):
        kernels.attention_compressed(q, kc, vc, T, nsplit=ns, split_len=sl, out=out)
    torch.cuda.synchronize()
    print(json.dumps({"profile_run": True, "copy_bytes_read": nbytes, "copy_bytes_written": nbytes,
                      "nsplit": ns, "split_len": sl}), flush=True)


def encoder_profile_run(exactkv, kernels, x):
    """Launch sequence for hardware-counter runs of the encoder: the calibration copy, then
    5 encodes of every page of x (one exkv_encode_pages call each, counter reset between)."""
    import torch
    nbytes = calibration_copy(x.device)
    B, TS, H, D = x.shape
    st = (x.stride(0), 16 * x.stride(1), x.stride(1), x.stride(2))
    c = exactkv.CompressedKV(B, TS, H, D, reserve=0.05)
    for _ in range(5):
        c.cnt.zero_()
        kernels.encode_pages(x, st, c._buf(), 0, 0, B, TS // 16)
    torch.cuda.synchronize()
    rows = B * TS * H
    print(json.dumps({"profile_run": True, "copy_bytes_read": nbytes, "copy_bytes_written": nbytes,
                      "encode_units": B * (TS // 16) * H, "source_bytes": rows * 256,
                      "raw_rows": int(c.cnt.item()),
                      "algorithmic_bytes": rows * 256 + rows * 192 + rows // 16 * 136 + int(c.cnt.item()) * 256}),
          flush=True)


def c3_stress(a):
    """Config 3 (Qwen3-8B shape): 32q/8kv, B32 x 4096, per-sequence lengths U[3500, 4096]
    (seeded), outlier-row rate 0.6%, raw pool started small (reserve 1e-4) so prefill
    grows it several times; the encoder timed on the 4096-token prefill of every sequence."""
    import numpy as np
    import torch
    import exactkv_amd as exactkv
    from exactkv_amd import kernels, synthetic

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, TS, Hq, Hkv = 32, 4096, 32, 8
    lens = np.random.Generator(np.random.PCG64(300)).integers(3500, TS + 1, B)
    print("[c3] generating data", file=sys.stderr, flush=True)
    k = synthetic.make_kv(B, TS, Hkv, kind="k", seed=100, device=dev, raw_row_rate=6e-3)
    v = synthetic.make_kv(B, TS, Hkv, kind="v", seed=101, device=dev, raw_row_rate=6e-3)
    q = synthetic.make_q(B, Hq, seed=102, device=dev)
    if a.profile:                                      # counter run of the encoder over the keys
        encoder_profile_run(exactkv, kernels, k)
        return
    enc = encoder_gbps(exactkv, kernels, [k, v], TS, a.steps, a.warmup)
    print("[c3] encoder timed", file=sys.stderr, flush=True)
    kcs, vcs, kbs, vbs, grows = [], [], [], [], []
    for i in range(a.copies):
        kc, vc = exactkv.CompressedKV(B, TS, Hkv, 128, reserve=1e-4), exactkv.CompressedKV(B, TS, Hkv, 128, reserve=1e-4)
        for b in range(B):
            kc.prefill_slot(b, k[b:b + 1])
            vc.prefill_slot(b, v[b:b + 1])
        grows.append(kc.grows + vc.grows)
        kcs.append(kc)
        vcs.append(vc)
        kbs.append(k.clone())
        vbs.append(v.clone())
    del k, v
    torch.cuda.synchronize()
    print("[c3] caches encoded", file=sys.stderr, flush=True)
    ld = torch.tensor(lens, dtype=torch.int32, device=dev)
    ns, sl = kernels.plan_splits(B, Hkv, Hq, TS)
    out = torch.empty_like(q)
    o_c = kernels.attention_compressed(q, kcs[0], vcs[0], TS, lens=ld, nsplit=ns, split_len=sl)
    o_r = kernels.attention_reference(q, kbs[0], vbs[0], TS, lens=ld, nsplit=ns, split_len=sl)
    identical = torch.equal(o_c.view(torch.int16), o_r.view(torch.int16))
    ms_c = time_loop(lambda i: kernels.attention_compressed(q, kcs[i], vcs[i], TS, lens=ld, nsplit=ns, split_len=sl,
                                                            out=out), a.steps, a.warmup, a.copies)
    ms_b = time_loop(lambda i: kernels.attention_reference(q, kbs[i], vbs[i], TS, lens=ld, nsplit=ns, split_len=sl,
                                                           out=out), a.steps, a.warmup, a.copies)
    ms_split, _ = time_split_kernel(lambda i: split_only(kernels, q, kcs[i], vcs[i], TS, ns, sl, True, ld),
                                    max(a.steps, 50), a.warmup, a.copies)
    alg = algorithmic_bytes([kcs[0], vcs[0]], B, TS, Hq, Hkv, lens)
    gbps = alg / (ms_split * 1e-3) / 1e9
    # the page decoder (compressed -> bf16, the path decode_to_bf16 / decode_reference use):
    # every byte of a key cache read once, the bf16 tensor written once
    ms_dec = time_loop(lambda i: kernels.decode_to_bf16(kcs[i], TS), a.steps, a.warmup, a.copies)
    c0 = kcs[0]
    dec_bytes = (sum(getattr(c0, f).nbytes for f in ("sm", "code", "base", "rowmask", "rowoff"))
                 + int(c0.cnt.item()) * 256 + B * TS * Hkv * 128 * 2)
    res = {
        "metric": "c3 decode-attn us with per-sequence lengths; encoder GB/s", "value": round(ms_c * 1e3, 2),
        "unit": "us", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_c, 5),
        "higher_is_better": False, "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "c3: Qwen3-8B shape 32q/8kv, B32 x 4096, lengths U[3500,4096], 0.6% outlier rows",
                   "B": B, "TS": TS, "Hq": Hq, "Hkv": Hkv, "lens_min": int(lens.min()), "lens_max": int(lens.max()),
                   "nsplit": ns, "split_len": sl, "cache_copies": a.copies},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "attn_split_kernel<compressed>", "algorithmic_bytes": alg,
                     "kernel_us": round(ms_split * 1e3, 2)},
        "bf16_twin_us": round(ms_b * 1e3, 2), "speedup_vs_bf16": round(ms_b / ms_c, 3),
        "bit_identical_to_bf16": bool(identical), "pool_grows_in_prefill": grows[0],
        "raw_rows": int(kcs[0].cnt.item()) + int(vcs[0].cnt.item()), "encoder_GBps": enc,
        "decoder_GBps": round(dec_bytes / (ms_dec * 1e-3) / 1e9, 1),
        "gpu": torch.cuda.get_device_name(0),
    }
    print(json.dumps(res), flush=True)


def cpu_sweep(a):
    """The CPU baseline at every benchmark shape, on the host cores only (no GPU work): the
    reference codec restated in PyTorch (oracle.torch_codec, byte-identical to codec.py) and
    fp32 GQA attention, with torch using every core this process may run on. Each figure is
    the median of --cpu-runs timed runs (time.perf_counter):
      encode GB/s   config 0's keys (1 x 4096 x 4 heads) and the c3 prefill (32 x 4096 x 8
                    heads, keys, 0.6% outlier rows): (bf16 read + compressed written) / time;
      decode GB/s   the c3 prefill's keys back to bf16: (compressed read + bf16 written) / time;
      attention ms  c1, c2a, c2b and c3 (per-sequence lengths): decode K and V, then attention,
                    on the same seeded data as the GPU benchmark of that shape."""
    import numpy as np
    import torch
    from exactkv_amd import synthetic
    from oracle import torch_codec

    n = cpu_threads()
    torch.set_num_threads(n)
    runs = a.cpu_runs

    def comp_bytes(c):
        return sum(c[f].numel() * c[f].element_size() for f in ("sm", "code", "base", "rowmask", "rowoff", "raw"))

    def log(msg):
        print(f"[cpu] {msg}", file=sys.stderr, flush=True)

    enc, dec, attn = {}, {}, {}
    for name, (B, T, H, kw) in {"c0": (1, 4096, 4, {}), "c3": (32, 4096, 8, {"raw_row_rate": 6e-3})}.items():
        x = synthetic.make_kv(B, T, H, kind="k", seed=100, **kw)
        c = torch_codec.encode(x)
        t, _ = median_seconds(lambda: torch_codec.encode(x), runs)
        enc[name] = {"GBps": round((x.numel() * 2 + comp_bytes(c)) / t / 1e9, 3), "s": round(t, 4),
                     "shape": [B, T, H, 128]}
        log(f"encode {name}: {enc[name]}")
        if name == "c3":
            t, _ = median_seconds(lambda: torch_codec.decode(c), runs)
            dec[name] = {"GBps": round((x.numel() * 2 + comp_bytes(c)) / t / 1e9, 3), "s": round(t, 4),
                         "shape": [B, T, H, 128]}
            log(f"decode {name}: {dec[name]}")
        del x, c
    shapes = {"c1": (1, 32768, 28, 4, 3e-3, None), "c2a": (8, 8192, 32, 8, 3e-3, None),
              "c2b": (1, 131072, 32, 8, 3e-3, None), "c3": (32, 4096, 32, 8, 6e-3, 300)}
    for name, (B, T, Hq, Hkv, rate, lseed) in shapes.items():
        k = synthetic.make_kv(B, T, Hkv, kind="k", seed=100, raw_row_rate=rate)
        v = synthetic.make_kv(B, T, Hkv, kind="v", seed=101, raw_row_rate=rate)
        q = synthetic.make_q(B, Hq, seed=102)
        lens = None if lseed is None else np.random.Generator(np.random.PCG64(lseed)).integers(3500, T + 1, B)
        kc, vc = torch_codec.encode(k), torch_codec.encode(v)
        del k, v
        t, best = median_seconds(lambda: torch_codec.decode_attention(q, kc, vc, T, lens=lens), runs)
        attn[name] = {"ms": round(t * 1e3, 2), "min_ms": round(best * 1e3, 2), "B": B, "T": T, "Hq": Hq, "Hkv": Hkv,
                      **({"lens": "U[3500, 4096] (PCG64 seed 300)"} if lens is not None else {})}
        log(f"attention {name}: {attn[name]}")
        del kc, vc
    res = {
        "metric": "CPU baseline: torch restatement of the reference codec + fp32 attention on the host cores",
        "value": attn["c2a"]["ms"], "unit": "ms", "n_gpus": 0, "steps": runs, "warmup": 0,
        "ms_per_step": attn["c2a"]["ms"], "higher_is_better": False, "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "cpu: encode c0 / c3 prefill, decode c3 prefill, decode+attention c1 / c2a / c2b / c3",
                   "runs": runs},
        "encode": enc, "decode": dec, "attention": attn,
        "cores": n, "torch_threads": torch.get_num_threads(), "cpu": cpu_model(),
        "timing": f"time.perf_counter, median of {runs} runs each",
    }
    print(json.dumps(res), flush=True)


E2E_CONFIG = dict(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
                  num_attention_heads=32, num_key_value_heads=8, max_position_embeddings=131072, rope_theta=5e5,
                  rms_norm_eps=1e-5, initializer_range=0.02, tie_word_embeddings=False)
# Llama-3.2-1B's shape: head dim 64 (2048 / 32), 8 KV heads, 16 layers, tied embeddings
E2E_CONFIG_1B = dict(vocab_size=128256, hidden_size=2048, intermediate_size=8192, num_hidden_layers=16,
                     num_attention_heads=32, num_key_value_heads=8, max_position_embeddings=131072, rope_theta=5e5,
                     rms_norm_eps=1e-5, initializer_range=0.02, tie_word_embeddings=True)
E2E_MODELS = {"llama3.1-8b": ("Llama-3.1-8B", E2E_CONFIG), "llama3.2-1b": ("Llama-3.2-1B (head dim 64)", E2E_CONFIG_1B)}


def e2e_child(a):
    """The default line's e2e leg: `bench.py --workload e2e --e2e-rows own` (c4: each cache at
    its own largest batch, 4096-token prompts, 256 greedy tokens) as a child process with a
    time limit, started once this process has freed its tensors (it keeps only its HIP
    context, so the child's KV budget is a few hundred MB below a fresh process's). Its
    progress goes to stderr; its JSON line is summarised here."""
    import subprocess
    cmd = [sys.executable, os.path.abspath(__file__), "--workload", "e2e", "--e2e-rows", "own",
           "--e2e-prompt", str(a.e2e_prompt), "--e2e-gen", str(a.e2e_gen)]
    print(f"[bench] e2e leg: {' '.join(cmd[1:])}", file=sys.stderr, flush=True)
    t0 = time.time()
    try:
        r = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=a.e2e_timeout)
    except subprocess.TimeoutExpired:
        return {"error": f"stopped after {a.e2e_timeout:.0f} s", "command": " ".join(cmd[1:])}
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    if r.returncode != 0 or not lines:
        return {"error": f"exit status {r.returncode}", "command": " ".join(cmd[1:])}
    d = json.loads(lines[-1])
    rows = {row["backend"]: row for row in d["rows"]}
    b, c = rows["bf16"], rows["exactkv"]
    print("[bench] e2e leg done", file=sys.stderr, flush=True)
    return {"workload": d["config"]["workload"], "metric": "decode tok/s = B * (gen - 1) / decode wall time",
            "tok_s": {"bf16": b["decode_tokens_per_s"], "exactkv": c["decode_tokens_per_s"]},
            "ratio": d["throughput_ratio"], "batch": {"bf16": b["batch"], "exactkv": c["batch"]},
            "sequences_fit": d["config"]["sequences_fit"],
            "ms_per_step": {"bf16": b["ms_per_step"], "exactkv": c["ms_per_step"]},
            "prefill_s": {"bf16": b["prefill_s"], "exactkv": c["prefill_s"]},
            "prompt": d["config"]["prompt"], "gen": d["config"]["gen"], "wall_s": round(time.time() - t0, 1),
            "command": " ".join(cmd[1:])}


def e2e_fit(model_key="llama3.1-8b", prompt=4096, gen=256):
    """The sequences-fit half of the c4 protocol (reference bench/e2e.py:54-63), measured
    without running the model: a placeholder of the model's weight bytes (the parameter
    shapes of its config, built on the meta device) is allocated, the KV budget is the free
    device memory after it minus 1.6 GiB, and the KV per sequence is kv_bytes(B=2) -
    kv_bytes(B=1) of every layer's K and V cache at T_max = prompt + gen, as the engine
    builds them. Decode tok/s needs the prefill of every sequence: `--workload e2e`."""
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM
    import exactkv_amd as exactkv

    mname, cfg = E2E_MODELS[model_key]
    with torch.device("meta"):
        m = LlamaForCausalLM(LlamaConfig(**cfg))
    wbytes = sum(p.numel() for p in m.parameters()) * 2          # bf16; tied weights counted once
    del m
    dev = torch.device("cuda", 0)
    torch.cuda.empty_cache()
    w = torch.empty(wbytes, dtype=torch.uint8, device=dev)
    budget = torch.cuda.mem_get_info()[0] - 1.6 * 2**30
    L, Hkv = cfg["num_hidden_layers"], cfg["num_key_value_heads"]
    D = cfg["hidden_size"] // cfg["num_attention_heads"]
    TS = -(-(prompt + gen) // 16) * 16

    def kv_bytes(cls, B):
        c = cls(B, TS, Hkv, D, device=dev)
        n = c.nbytes()
        del c
        return 2 * L * n                                           # every layer's K and V cache

    per_seq = {be: kv_bytes(cls, 2) - kv_bytes(cls, 1)
               for be, cls in (("bf16", exactkv.BF16KV), ("exactkv", exactkv.CompressedKV))}
    del w
    torch.cuda.empty_cache()
    fit = {be: int(budget // n) for be, n in per_seq.items()}
    return {"model": f"{mname} (weights as a placeholder allocation)", "t_max": prompt + gen,
            "weights_gib": round(wbytes / 2**30, 2), "kv_budget_gib": round(budget / 2**30, 2),
            "kv_mib_per_seq": {be: round(n / 2**20, 1) for be, n in per_seq.items()},
            "sequences_fit": fit, "ratio": round(fit["exactkv"] / fit["bf16"], 3),
            "tok_s": "bench.py --workload e2e (the prefill of every sequence; minutes)"}


def prefill_bench(a):
    """Prefill into the compressed cache on a random-init Llama-3.1-8B (c4's model): 8
    prompts of e2e-prompt (4096) tokens, one at a time, with the write-through prefill
    (each layer's K/V encoded straight from the attention module) and with the two-pass
    prefill (the model's DynamicCache holds all 32 layers' K/V, then each layer is encoded).
    Reports tokens/s and the peak memory above the weights and caches for each."""
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM
    import exactkv_amd as exactkv

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    PL, NS = a.e2e_prompt, 8
    print("[prefill] building random-init Llama-3.1-8B", file=sys.stderr, flush=True)
    torch.manual_seed(0)
    with torch.device(dev):
        model = LlamaForCausalLM(LlamaConfig(**E2E_CONFIG)).to(torch.bfloat16).eval()
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, E2E_CONFIG["vocab_size"], (NS, PL), generator=g).to(dev)
    eng = exactkv.Engine(model, NS, PL + 16, backend="exactkv", graph=False)
    res = {}
    for fused in (True, False, True):                  # warm both paths; the last run counts
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        t0 = time.perf_counter()
        toks = eng.prefill(ids, fused=fused)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        res[fused] = (dt, torch.cuda.max_memory_allocated() - base, toks.clone())
        print(f"[prefill] fused={fused}: {NS * PL / dt:.0f} tok/s", file=sys.stderr, flush=True)
    same = torch.equal(res[True][2], res[False][2])
    tps = NS * PL / res[True][0]
    out = {
        "metric": "prefill tokens/s into the compressed cache (write-through), Llama-3.1-8B",
        "value": round(tps, 1), "unit": "tok/s", "n_gpus": 1, "steps": NS, "warmup": NS,
        "ms_per_step": round(res[True][0] / NS * 1e3, 3), "higher_is_better": True, "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "prefill: Llama-3.1-8B random init, 8 prompts x 4096 tokens, one at a time",
                   "prompt": PL, "sequences": NS},
        "two_pass_tok_s": round(NS * PL / res[False][0], 1),
        "peak_extra_gib": {"write_through": round(res[True][1] / 2**30, 3), "two_pass": round(res[False][1] / 2**30, 3)},
        "same_next_tokens": bool(same), "gpu": torch.cuda.get_device_name(0),
    }
    print(json.dumps(out), flush=True)


def e2e_paged(a):
    """Greedy decoding of prompts of mixed lengths (U[1024, 4096], seeded) over a page pool
    (PagedEngine) on the c4 model: the pool takes the KV budget of the e2e protocol and
    admits sequences by the pages they need, where a contiguous cache reserves the longest
    prompt + generation for every sequence. Reports how many sequences each layout fits and
    the paged engine's decode tok/s (eager steps) at its batch."""
    import numpy as np
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM
    import exactkv_amd as exactkv

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    G, LMAX = 64, 4096
    print("[e2e_paged] building random-init Llama-3.1-8B", file=sys.stderr, flush=True)
    torch.manual_seed(0)
    with torch.device(dev):
        model = LlamaForCausalLM(LlamaConfig(**E2E_CONFIG)).to(torch.bfloat16).eval()
    torch.cuda.empty_cache()
    budget = torch.cuda.mem_get_info()[0] - 1.6 * 2**30 - a.e2e_work_gib * 2**30
    cfg = E2E_CONFIG
    L, H = cfg["num_hidden_layers"], cfg["num_key_value_heads"]
    page_bytes = 2 * L * (16 * H * 192 + H * 136)                     # K and V of all layers, one page
    per_seq_contig = exactkv.Engine(model, 2, LMAX + G).kv_bytes() - exactkv.Engine(model, 1, LMAX + G).kv_bytes()
    torch.cuda.empty_cache()
    rng = np.random.Generator(np.random.PCG64(7))
    lens = rng.integers(1024, LMAX + 1, size=4096)
    need = -(-(lens + G) // 16)
    num_pages = int(budget * 0.97 // page_bytes)                     # ~3% for the raw pools and tails
    n_fit = int(np.searchsorted(np.cumsum(need), num_pages, side="right"))
    B = min(n_fit, 2048)
    fit_contig = int(budget // per_seq_contig)
    print(f"[e2e_paged] pool {num_pages} pages: {B} sequences (contiguous would fit {fit_contig})",
          file=sys.stderr, flush=True)
    eng = exactkv.PagedEngine(model, B, LMAX + G, backend="exactkv", num_pages=num_pages)
    g = torch.Generator().manual_seed(1)
    t0 = time.perf_counter()
    toks = []
    for i in range(B):
        ids = torch.randint(0, cfg["vocab_size"], (int(lens[i]),), generator=g).to(dev)
        toks.append(eng.add(ids)[1])
        if i % 64 == 63:
            print(f"[e2e_paged] prefilled {i + 1}", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    t = torch.stack(toks)
    for s in range(G - 1):
        t = eng.step(t).argmax(-1)
        if s % 16 == 15:
            print(f"[e2e_paged] step {s + 1}", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    tps = B * (G - 1) / (t2 - t1)
    res = {
        "metric": "paged e2e greedy decode tok/s, prompts U[1024, 4096] (Llama-3.1-8B random init)",
        "value": round(tps, 1), "unit": "tok/s", "n_gpus": 1, "higher_is_better": True, "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (random weights N(0,0.02), random token ids)",
        "config": {"workload": "e2e_paged: mixed prompt lengths over one page pool", "gen": G,
                   "prompt_lengths": "U[1024, 4096] seed 7", "pool_pages": num_pages,
                   "kv_budget_gib": round(budget / 2**30, 2)},
        "sequences": B, "contiguous_sequences_fit": fit_contig, "fit_ratio": round(B / max(fit_contig, 1), 3),
        "mean_prompt": round(float(lens[:B].mean()), 1), "ms_per_step": round((t2 - t1) / (G - 1) * 1e3, 2),
        "prefill_s": round(t1 - t0, 1), "pool_grows": eng.grows, "free_pages_after": eng.table.free_pages(),
        "gpu": torch.cuda.get_device_name(0),
    }
    print(json.dumps(res), flush=True)


def e2e(a):
    """Config 4: batched greedy decoding with the engine on a random-init Llama-3.1-8B
    (weights N(0, 0.02) bf16; --e2e-model llama3.2-1b: Llama-3.2-1B's shape, head dim 64),
    prompts of uniform random token ids, the reference's protocol (bench/e2e.py:43-101): KV
    budget = free memory after the weights minus 1.6 GiB, KV per sequence = kv_bytes(B=2) -
    kv_bytes(B=1), each backend at the largest batch that fits, then the compressed cache
    also at the bf16 batch (same work)."""
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM
    import exactkv_amd as exactkv

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    PL, G = a.e2e_prompt, a.e2e_gen
    TM = PL + G
    mname, mcfg = E2E_MODELS[a.e2e_model]
    print(f"[e2e] building random-init {mname}", file=sys.stderr, flush=True)
    torch.manual_seed(0)
    with torch.device(dev):
        model = LlamaForCausalLM(LlamaConfig(**mcfg)).to(torch.bfloat16).eval()
    torch.cuda.empty_cache()
    wbytes = sum(p.numel() * p.element_size() for p in model.parameters())
    budget = torch.cuda.mem_get_info()[0] - 1.6 * 2**30

    def per_seq(be):
        e1, e2 = exactkv.Engine(model, 1, TM, backend=be), exactkv.Engine(model, 2, TM, backend=be)
        d = e2.kv_bytes() - e1.kv_bytes()
        del e1, e2
        torch.cuda.empty_cache()
        return d
    ps = {be: per_seq(be) for be in ("bf16", "exactkv")}
    fit = {be: int(budget // ps[be]) for be in ps}
    # working memory beyond the caches (prefill activations, logits, pool growth)
    work = a.e2e_work_gib * 2**30
    run_b = {be: max(1, min(fit[be], int((budget - work) // ps[be]))) for be in ps}
    if a.e2e_batch:
        run_b = {be: min(a.e2e_batch, run_b[be]) for be in ps}
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, mcfg["vocab_size"], (max(run_b.values()), PL), generator=g).to(dev)

    def run(be, B):
        eng = exactkv.Engine(model, B, TM, backend=be)
        torch.cuda.synchronize()
        t0 = time.time()
        nxt = []
        for b0 in range(0, B, 64):
            nxt.append(eng.prefill(ids[b0:min(B, b0 + 64)], b0=b0))
            print(f"[e2e] {be} B={B}: prefilled {min(B, b0 + 64)}", file=sys.stderr, flush=True)
        t = torch.cat(nxt)
        torch.cuda.synchronize()
        t1 = time.time()
        toks = [t]
        for s in range(G - 1):
            t = eng.step(t).argmax(-1)
            toks.append(t)
            if s % 64 == 63:
                print(f"[e2e] {be} B={B}: step {s + 1}", file=sys.stderr, flush=True)
        torch.cuda.synchronize()
        t2 = time.time()
        r = dict(backend=be, batch=B, kv_mib_per_seq=round(ps[be] / 2**20, 1),
                 ms_per_step=round((t2 - t1) / (G - 1) * 1e3, 2),
                 decode_tokens_per_s=round(B * (G - 1) / (t2 - t1), 1), prefill_s=round(t1 - t0, 1),
                 pool_grows=eng.grows)
        print(json.dumps(r), file=sys.stderr, flush=True)
        out = torch.stack(toks, 1).cpu()
        del eng
        torch.cuda.empty_cache()
        return r, out

    r_b, tok_b = run("bf16", run_b["bf16"])
    r_c, tok_c = run("exactkv", run_b["exactkv"])
    r_s, tok_s = run("exactkv", r_b["batch"]) if a.e2e_rows == "all" else (None, None)
    res = {
        "metric": f"e2e greedy decode tok/s ({mname} random init, {PL}-token prompts, {G} new tokens)",
        "value": r_c["decode_tokens_per_s"], "unit": "tok/s", "n_gpus": 1, "higher_is_better": True,
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (random weights N(0,0.02), random token ids)",
        "config": {"workload": f"{'c4: ' if a.e2e_model == 'llama3.1-8b' else ''}{mname} e2e greedy decode",
                   "prompt": PL, "gen": G, "head_dim": mcfg["hidden_size"] // mcfg["num_attention_heads"],
                   "weights_gib": round(wbytes / 2**30, 2), "kv_budget_gib": round(budget / 2**30, 2),
                   "sequences_fit": fit, "batch_run": run_b},
        "rows": [r for r in (r_b, r_c, r_s) if r is not None],
        "throughput_ratio": round(r_c["decode_tokens_per_s"] / r_b["decode_tokens_per_s"], 3),
        "gpu": torch.cuda.get_device_name(0),
    }
    if r_s is not None:
        res["step_time_ratio_same_batch"] = round(r_b["ms_per_step"] / r_s["ms_per_step"], 3)
        res["tokens_equal_same_batch"] = bool(torch.equal(tok_b, tok_s))
    print(json.dumps(res), flush=True)


def split_only(kernels, q, kc, vc, T, ns, sl, compressed, lens=None, block_table=None, window=0):
    """Launch only the split kernel (the dominant kernel) into the shared workspace."""
    from exactkv_amd import _lib
    B, Hq, D = q.shape
    wo, wm, wl = kernels._workspace(q.device, B * Hq, ns, D)
    scale = D ** -0.5 * kernels.LOG2E
    lp, lstride = (lens.data_ptr(), lens.stride(0)) if lens is not None else (None, 0)
    if block_table is not None:                        # compressed pool of pages
        ka, TSp, Hkv, Bp = kernels._cache_args(kc)
        va, _, _, _ = kernels._cache_args(vc)
        _lib.call("exkv_attn_split_compressed_paged", q.data_ptr(), *ka, *va, wo.data_ptr(), wm.data_ptr(),
                  wl.data_ptr(), block_table.data_ptr(), block_table.shape[1], Bp * TSp // 16, B, Hq, Hkv, D, T,
                  block_table.shape[1] * 16, lp, lstride, ns, sl, window, scale, _lib.stream())
        return
    if compressed:
        ka, TS, Hkv, _ = kernels._cache_args(kc)
        va, _, _, _ = kernels._cache_args(vc)
        _lib.call("exkv_attn_split_compressed", q.data_ptr(), *ka, *va, wo.data_ptr(), wm.data_ptr(),
                  wl.data_ptr(), B, Hq, Hkv, D, T, TS, lp, lstride, ns, sl, window, scale, _lib.stream())
    else:
        TS, Hkv = kc.shape[1], kc.shape[2]
        _lib.call("exkv_attn_split_bf16", q.data_ptr(), kc.data_ptr(), vc.data_ptr(), wo.data_ptr(), wm.data_ptr(),
                  wl.data_ptr(), B, Hq, Hkv, D, T, TS, lp, lstride, ns, sl, window, scale, _lib.stream())


def encoder_gbps(exactkv, kernels, xs, T, steps, warmup):
    """Page-encoder throughput over a prefill of the workload's keys: (bf16 read + compressed
    write) bytes / time, alternating between len(xs) sources and as many caches so that the
    working set (> 256 MB at c2a and c3) is not held by the 256 MB Infinity Cache. Each cache's
    pool has room for every timed encode, so the raw-row counter is never reset inside the
    timed region and every raw row is written."""
    import torch
    B, TS, H, D = xs[0].shape
    npg = T // 16
    st = (xs[0].stride(0), 16 * xs[0].stride(1), xs[0].stride(1), xs[0].stride(2))
    n = max(5, steps // 5)
    raw = []
    for x in xs:                                       # raw rows one encode of each source writes
        probe = exactkv.CompressedKV(B, TS, H, D, reserve=0.05)
        kernels.encode_pages(x, st, probe._buf(), 0, 0, B, npg)
        raw.append(int(probe.cnt.item()))
        del probe
    reps = n + warmup
    caches = [exactkv.CompressedKV(B, TS, H, D, reserve=(reps * max(r, 1) * 2.0) / (B * TS * H)) for r in raw]

    def enc(i):
        kernels.encode_pages(xs[i], st, caches[i]._buf(), 0, 0, B, npg)
    ms = time_loop(enc, n, warmup, len(xs))
    torch.cuda.synchronize()
    assert all(int(c.cnt.item()) <= c.cap for c in caches)
    rows = B * npg * 16 * H
    byts = rows * 2 * D + rows * (3 * D // 2) + B * npg * H * (D + 8) + sum(raw) / len(raw) * 2 * D
    return round(byts / (ms * 1e-3) / 1e9, 1)


if __name__ == "__main__":
    main()
