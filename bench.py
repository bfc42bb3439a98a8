"""Benchmark of the Qwen3-30B-A3B MoE block on one MI355X.

Workload (default): the MoE block at decode shape, T=1 token, bf16, all 128
experts resident, H=2048, I=768, top-8.  48 distinct layers of random-init
weights (58 GB) are resident and the timed steps rotate through them, so the
76 MB touched per block call cannot be served from the 256 MB Infinity Cache.
A step is one MoE block call (router -> dispatch -> experts -> combine with
the residual add) on the next layer's weights; the 48-call rotation is
captured once in a HIP graph and replayed.

Prints ONE JSON line.  ``value`` is MoE-block tokens/s (T tokens per step).
``roofline`` is for the decode block (one ``qmoe_moe_decode_block`` call:
router logits, fused expert items, reduce), timed with HIP events on the
stream the graph replays on, against its algorithmic bytes
U * 9,437,184 + 524,288 (U = distinct experts touched, measured).
``roofline.traffic`` is the HBM-side bytes per call measured live with two
``rocprofv3 --pmc`` child runs of this script in ``--traffic-probe`` mode
(FETCH_SIZE, then WRITE_SIZE, summed over the call's kernels), each scaled by
what the same counter reads for a plain elementwise kernel of known size.
``cpu_baseline`` is the fp32 CPU oracle (the reference's decode schedule) on a
bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nki-moe-7013_amd"))
sys.path.insert(0, ROOT)

METRIC = "Qwen3-30B-A3B-shape decode tokens/s & MoE-block GB/s (% of HBM peak)"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2517.0  # 256 CU x 2.4 GHz x 4096 flop/clk (dense)
H, E, I, K_TOP = 2048, 128, 768, 8
EXPERT_BYTES = 3 * H * I * 2  # 9,437,184
ROUTER_BYTES = E * H * 2


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=960, help="timed MoE block calls (exactly this many)")
    ap.add_argument("--warmup", type=int, default=96)
    ap.add_argument("--tokens", type=int, default=1, help="T tokens per MoE block call")
    ap.add_argument("--layers", type=int, default=48, help="distinct weight sets rotated through")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--extra", action="store_true",
                    help="time T=8/64 decode and the attention layer (the default; kept for old command lines)")
    ap.add_argument("--no-extra", action="store_true", help="skip the T=8/64 decode and attention-layer timings")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 PMC traffic runs")
    ap.add_argument("--traffic-probe", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--no-prefill", action="store_true", help="skip the T=4096 prefill MoE block")
    ap.add_argument("--no-model", action="store_true",
                    help="skip the full 48-layer model (TTFT at 640 tokens, 256 greedy steps; "
                         "run in a child process)")
    ap.add_argument("--only-prefill", action="store_true",
                    help="only the T=4096 prefill MoE block (Zipf-skewed routing); prints its dict")
    ap.add_argument("--only-model", action="store_true",
                    help="time only the full model, in this process, and print its numbers as JSON")
    ap.add_argument("--only-attention", action="store_true",
                    help="only the B=8 attention layer (prefill 1024, decode at ctx 1280 and 8192); prints its dict")
    return ap.parse_args()


def git_sha():
    """The commit measured: git when the tree has .git, else the commit the
    library was built from (recorded by the build next to libqmoe.so, with a
    +dirty suffix when the build tree had uncommitted changes)."""
    try:
        return subprocess.check_output(["git", "rev-parse", "--short", "HEAD"], cwd=ROOT,
                                       stderr=subprocess.DEVNULL).decode().strip()
    except Exception:
        pass
    try:
        with open(os.path.join(ROOT, "nki-moe-7013_amd", "qmoe", "build_info.json")) as f:
            info = json.load(f)
        return (info["git"] + ("+dirty" if info.get("dirty") else "")) if info.get("git") else None
    except (OSError, ValueError, KeyError):
        return None


def _gemv_max_tokens():
    from qmoe.moe import GEMV_MAX_TOKENS

    return GEMV_MAX_TOKENS


def make_layers(n_layers, dev, seed=0):
    import torch

    g = torch.Generator(device=dev).manual_seed(seed)
    layers = []
    for _ in range(n_layers):
        w_router = torch.empty(E, H, device=dev, dtype=torch.bfloat16).normal_(0.0, 0.02, generator=g)
        w13 = torch.empty(E, 2 * I, H, device=dev, dtype=torch.bfloat16).normal_(0.0, 0.02, generator=g)
        w2 = torch.empty(E, I // 8, H, 8, device=dev, dtype=torch.bfloat16).normal_(0.0, 0.02, generator=g)
        layers.append((w_router, w13, w2))
    return layers


def time_graph(fn, steps_per_replay, steps, warmup, spread=None, part=None):
    """Capture fn() (which performs steps_per_replay steps) in a HIP graph and
    time exactly ``steps`` steps: steps // steps_per_replay replays, then, when
    ``part(r)`` is given (a function doing the first r steps), one replay of
    a second graph capturing part(steps % steps_per_replay).  Without
    ``part`` the step count is rounded up to whole replays.  ``warmup`` steps
    run untimed first (whole replays).  Returns (seconds by the host clock,
    seconds by HIP events on the replay stream, steps_done).

    With ``spread = n``, n further replays (after the timed region, not part
    of it) are each bracketed by their own HIP events, and the per-step
    microseconds of every replay are stored in ``spread_us`` (a list passed by
    the caller) for the median / p10 / p90."""
    import torch

    def capture(f):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            f()  # eager warm-up: allocations, lazy init
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            f()
        return gr

    graph = capture(fn)
    rem = steps % steps_per_replay if part is not None else 0
    tail = capture(lambda: part(rem)) if rem else None
    reps_w = max(1, math.ceil(warmup / steps_per_replay))
    reps = steps // steps_per_replay if part is not None else max(1, math.ceil(steps / steps_per_replay))
    for _ in range(reps_w):
        graph.replay()
    if tail is not None:
        tail.replay()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(reps):
        graph.replay()
    if tail is not None:
        tail.replay()
    ev1.record()
    torch.cuda.synchronize()
    secs = time.perf_counter() - t0
    if spread is not None:
        n = spread.pop() if spread else 0
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        for a, b in evs:
            a.record()
            graph.replay()
            b.record()
        torch.cuda.synchronize()
        spread.extend(a.elapsed_time(b) * 1e3 / steps_per_replay for a, b in evs)
    return secs, ev0.elapsed_time(ev1) * 1e-3, reps * steps_per_replay + rem


def percentiles(us):
    """median, p10 and p90 (nearest rank) of a list of per-step microseconds."""
    v = sorted(us)
    at = lambda q: v[min(len(v) - 1, max(0, int(round(q * (len(v) - 1)))))]
    return {"median": round(at(0.5), 3), "p10": round(at(0.1), 3), "p90": round(at(0.9), 3), "samples": len(v)}


def event_time_experts(run_one, n):
    """Average and median GPU duration of run_one(i), each call bracketed by
    HIP events on the current stream, in steady state: n untimed calls first
    (clocks and memory state settle under the same load), then n timed ones
    enqueued back to back (each call takes hundreds of microseconds, so the
    host stays ahead and the GPU never idles between them)."""
    import torch

    for i in range(n):
        run_one(i)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for i in range(n):
        starts[i].record()
        run_one(i)
        ends[i].record()
    torch.cuda.synchronize()
    ms = [a.elapsed_time(b) for a, b in zip(starts, ends)]
    ms.sort()
    return sum(ms) / len(ms), ms[len(ms) // 2]


def bench_decode(layers, T, steps, warmup, dev):
    import torch

    from qmoe import ops
    from qmoe.moe import MoEBlock

    L = len(layers)
    g = torch.Generator(device=dev).manual_seed(1234 + T)
    xs = [torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16) for _ in range(L)]
    res = [torch.randn(T, H, generator=g, device=dev) for _ in range(L)]
    outs = [torch.empty(T, H, device=dev) for _ in range(L)]
    blocks = [MoEBlock(*w, K_TOP) for w in layers]

    def first_layers(n):
        for l in range(n):
            blocks[l](xs[l], res[l], out=outs[l])

    spread = [60]  # 60 individually timed replays of the L-call graph
    secs, ev_secs, done = time_graph(lambda: first_layers(L), L, steps, warmup, spread=spread,
                                     part=first_layers)
    U = []
    for l in range(L):
        _, _, ti = ops.router_topk(xs[l], layers[l][0], K_TOP)
        U.append(int(torch.unique(ti).numel()))
    u_mean = sum(U) / len(U)
    expert_bytes = u_mean * EXPERT_BYTES
    block_bytes = expert_bytes + ROUTER_BYTES
    us_per_step = ev_secs / done * 1e6
    return {
        "T": T,
        "us_per_block": us_per_step,
        "us_per_block_host_clock": secs / done * 1e6,
        "tokens_per_s": T * done / ev_secs,
        "U_mean": u_mean,
        "block_bytes": block_bytes,
        "block_GBps": block_bytes / (us_per_step * 1e-6) / 1e9,
        "block_frac": block_bytes / (us_per_step * 1e-6) / 1e9 / HBM_PEAK_GBS,
        "us_per_block_spread": percentiles(spread),
        "secs": secs,
        "steps": done,
    }


def zipf_targets(n_experts, T, k, s=1.1):
    """Rows per expert, by popularity rank r = 1..E, when expert popularity
    follows Zipf(s) under top-k routing: n_r = min(T, C * r^-s) with C set so
    that sum(n_r) = T * k.  An expert takes each token at most once, so the
    head of the distribution saturates at T (water-filling).  Returns a list
    of E floats, rank 1 first."""
    w = [(r + 1) ** -s for r in range(n_experts)]
    lo, hi = 0.0, float(T) * n_experts
    for _ in range(200):
        c = 0.5 * (lo + hi)
        if sum(min(T, c * x) for x in w) > T * k:
            hi = c
        else:
            lo = c
    return [min(float(T), lo * x) for x in w]


def zipf_router_bias(x, w_router, k, s=1.1, rank_seed=5, iters=400, step=0.3):
    """A per-expert router bias under which the routing of the tokens ``x``
    follows Zipf(s) popularity: experts get popularity ranks from a seeded
    permutation and ``top-k(x . w_router^T + bias)`` takes expert e in about
    ``zipf_targets(...)[rank(e) - 1]`` rows.  Fitted by damped log-count
    updates on the tokens' own fp32 logits (selection counts rise
    monotonically with an expert's bias); an expert whose target is every
    token gets the least bias that puts it in each token's top-k.  Returns
    ``(bias f32 [E] on x's device, target rows per expert id)``."""
    import torch

    T, n_e = x.shape[0], w_router.shape[0]
    rank = torch.randperm(n_e, generator=torch.Generator().manual_seed(rank_seed))
    tgt = torch.tensor(zipf_targets(n_e, T, k, s), dtype=torch.float32)[rank].to(x.device)
    logits = x.float() @ w_router.float().t()
    bias = torch.zeros(n_e, dtype=torch.float32, device=x.device)
    sat = tgt >= T - 0.5  # experts every token must choose
    n_sat = int(sat.sum())
    for _ in range(iters):
        if n_sat:
            # the least bias that puts each saturated expert in every token's
            # top-k: above the (k - n_sat + 1)-th largest other biased logit
            other = (logits + bias).masked_fill(sat, float("-inf"))
            v = torch.topk(other, k - n_sat + 1, dim=1).values[:, -1:]
            bias[sat] = (v - logits[:, sat]).max(dim=0).values + 1e-3
        idx = torch.topk(logits + bias, k, dim=1).indices
        cnt = torch.bincount(idx.flatten(), minlength=n_e).float()
        upd = step * (torch.log(tgt + 0.5) - torch.log(cnt + 0.5))
        bias += upd.masked_fill(sat, 0.0)
    return bias, tgt


def routing_histogram(top_i, target, T):
    """Achieved rows per expert against the Zipf target, for the bench line."""
    import torch

    cnt = torch.bincount(top_i.long().flatten(), minlength=target.numel()).float()
    order = torch.argsort(target, descending=True)
    return {
        "zipf_s": 1.1,
        "target_rows_top8": [round(float(v)) for v in target[order][:8]],
        "achieved_rows_top8": [int(v) for v in cnt[order][:8]],
        "target_rows_min": round(float(target.min())),
        "achieved_rows_min": int(cnt.min()),
        "experts_below_32_rows": int((cnt < 32).sum()),
        "touched_experts": int((cnt > 0).sum()),
        "l1_vs_target": float((cnt - target).abs().sum() / (T * K_TOP)),
    }


def bench_prefill(layers, dev, T=4096, reps=20, zipf_s=1.1):
    """MoE block at prefill shape.  With ``zipf_s``: Zipf(s) expert
    popularity, a router bias per layer fitted so that the T tokens' top-8
    routing follows the Zipf row targets (at T = 4096 the most popular expert
    takes every token); without it the plain router (near-uniform load)."""
    import torch

    from qmoe import ops
    from qmoe.moe import MoEBlock, tile_m_for

    g = torch.Generator(device=dev).manual_seed(77 + T)
    L = min(4, len(layers))
    xs = [torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16) for _ in range(L)]
    fits = [zipf_router_bias(xs[l], layers[l][0], K_TOP, zipf_s) if zipf_s else (None, None)
            for l in range(L)]
    biases = [f[0] for f in fits]
    blocks = [MoEBlock(*layers[l], K_TOP, router_bias=biases[l]) for l in range(L)]

    def run():
        for l in range(L):
            blocks[l](xs[l])

    spread = [50]
    secs, ev_secs, done = time_graph(run, L, reps * L, 5 * L, spread=spread)
    counts, routes, hist = [], [], None
    for l in range(L):
        _, tw, ti = ops.router_topk(xs[l], layers[l][0], K_TOP, biases[l])
        counts.append(torch.bincount(ti.long().flatten(), minlength=E))
        routes.append(ops.moe_permute(ti, E, tile_m_for(T, K_TOP)))
        if l == 0 and zipf_s:
            hist = routing_histogram(ti, fits[0][1], T)
    cnt = torch.stack(counts).float().mean(0)

    def run_experts(i):
        l = i % L
        ops.moe_experts_grouped(xs[l], layers[l][1], layers[l][2], routes[l])

    mean_ms, med_ms = event_time_experts(run_experts, 4 * L)
    flops = T * K_TOP * 2 * 3 * H * I
    dense = None
    if zipf_s:
        # The same grouped GEMMs with every token on experts 0..7 (each expert
        # T rows: only full 256 x 256 tiles, weights shared by T/256 tiles):
        # the expert kernels' rate when MFMA work is all there is.
        top = torch.arange(K_TOP, dtype=torch.int32, device=dev).repeat(T, 1)
        droute = ops.moe_permute(top, E, tile_m_for(T, K_TOP))
        dmean, _ = event_time_experts(
            lambda i: ops.moe_experts_grouped(xs[i % L], layers[i % L][1], layers[i % L][2], droute), 4 * L)
        dense = {"experts_us_mean": dmean * 1e3, "experts_TFLOPs": flops / (dmean * 1e-3) / 1e12}
    us = ev_secs / done * 1e6
    # touched experts' weights once, the router, x in and the output, as bf16
    touched = float((torch.stack(counts) > 0).sum(1).float().mean())
    block_bytes = touched * EXPERT_BYTES + ROUTER_BYTES + 2 * T * H * 2
    return {
        "T": T,
        "us_per_block": us,
        "us_per_block_spread": percentiles(spread),
        "tokens_per_s": T / (us * 1e-6),
        "touched_experts": touched,
        "block_bytes": block_bytes,
        "block_hbm_frac": block_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
        "experts_us_mean": mean_ms * 1e3,
        "experts_TFLOPs": flops / (mean_ms * 1e-3) / 1e12,
        "experts_mfma_frac": flops / (mean_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
        "top_expert_share": float(cnt.max() / cnt.sum()),
        "routing_vs_zipf": hist,
        "experts_dense_routing_8_experts": dense,
        "_cpu_case": (xs[0], biases[0]),  # layer 0's tokens and bias, for the CPU leg
    }


def measure_peaks(dev):
    """Measured ceilings next to the published ones: the bf16 MFMA rate of a
    pure v_mfma_f32_32x32x16_bf16 loop (probe library) on random and on
    constant operands (the chip is power-limited: random data lowers the
    clock), and a plain device-to-device copy of 1 GiB (STREAM-like)."""
    import ctypes

    import torch

    path = os.path.join(ROOT, "nki-moe-7013_amd", "qmoe", "libqmoe_probe.so")
    lib = ctypes.CDLL(path)
    lib.qmoe_probe_mfma.restype = ctypes.c_int
    lib.qmoe_probe_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.qmoe_probe_mfma_flops.restype = ctypes.c_double
    lib.qmoe_probe_mfma_flops.argtypes = [ctypes.c_int, ctypes.c_int]
    n_cu = torch.cuda.get_device_properties(dev).multi_processor_count
    blocks, iters = 2 * n_cu, 2048
    g = torch.Generator(device=dev).manual_seed(11)
    rnd = torch.randn(blocks * 8 * 256 * 8, generator=g, device=dev).to(torch.bfloat16)
    const = torch.ones_like(rnd)
    out = torch.empty(blocks * 256, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    res = {}
    for name, src in (("random", rnd), ("constant", const)):
        def launch():
            rc = lib.qmoe_probe_mfma(ctypes.c_void_p(src.data_ptr()), blocks, iters,
                                     ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(stream))
            if rc:
                raise RuntimeError(f"qmoe_probe_mfma failed ({rc})")
        launch()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            launch()
        e1.record()
        torch.cuda.synchronize()
        secs = e0.elapsed_time(e1) * 1e-3 / 5
        res[f"mfma_bf16_{name}_TFLOPs"] = round(lib.qmoe_probe_mfma_flops(blocks, iters) / secs / 1e12, 1)
    del rnd, const, out
    a = torch.empty(1 << 29, dtype=torch.bfloat16, device=dev)  # 1 GiB
    b = torch.empty_like(a)
    a.fill_(1.0)
    b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    res["hbm_copy_GBps"] = round(2 * a.numel() * 2 * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9, 1)
    del a, b
    # The vendor GEMM library (torch.matmul -> hipBLASLt) on dense bf16: the
    # prefill experts' whole work at T = 4096 as one GEMM per projection (all
    # T*k = 32768 (token, expert) rows against one weight: gate_up 32768 x 1536
    # x 2048, down 32768 x 2048 x 768; no gather, no skew, no per-expert
    # tiles), one expert's share at full load (4096 rows: too few tiles to
    # fill 256 CUs), and 8192^3: what a tuned library reaches on this chip, as
    # a ceiling beside the published peak.  Measurement only; the product
    # never calls it.
    lib_res = {}
    for M, N, K in ((32768, 1536, 2048), (32768, 2048, 768), (4096, 1536, 2048), (4096, 2048, 768),
                    (8192, 8192, 8192)):
        A = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        B = torch.randn(K, N, generator=g, device=dev).to(torch.bfloat16)
        C = torch.matmul(A, B)
        reps = 20 if M * N * K < (1 << 34) else 5
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            torch.matmul(A, B, out=C)
        e1.record()
        torch.cuda.synchronize()
        secs = e0.elapsed_time(e1) * 1e-3 / reps
        lib_res[f"{M}x{N}x{K}"] = round(2.0 * M * N * K / secs / 1e12, 1)
        del A, B, C
    res["hipblaslt_bf16_TFLOPs"] = lib_res
    res.update(measure_hw_probes(dev, lib))
    return res


def measure_hw_probes(dev, lib):
    """The probe library's hardware ceilings (probes/hw.hip): the cost of a
    kernel boundary inside a HIP graph, the HBM read rate at 256 and 1024
    workgroups on a 76 MB working set (the decode block's), rotated over 1 GiB
    so the 256 MB Infinity Cache cannot serve it, and the L2 -> CU read rate
    into VGPRs and through the LDS DMA."""
    import ctypes

    import torch

    P, I64, INT = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.qmoe_probe_empty.argtypes, lib.qmoe_probe_empty.restype = [INT, P], INT
    lib.qmoe_probe_stream.argtypes, lib.qmoe_probe_stream.restype = [P, I64, INT, P, P], INT
    lib.qmoe_probe_l2.argtypes, lib.qmoe_probe_l2.restype = [P, INT, INT, INT, P, P], INT

    def ok(rc):
        if rc:
            raise RuntimeError(f"probe launch failed ({rc})")

    def graph_us(fn, n, reps=5):
        """Per-launch microseconds of n launches of fn() captured in one graph."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(n):
                fn()
        gr.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            gr.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * n)

    out = torch.empty(4096, dtype=torch.int32, device=dev)
    cur = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    res = {}
    small = torch.ones(1 << 22, dtype=torch.uint8, device=dev)  # 4 MB
    res["graph_launch_us"] = {
        "empty_1wg": round(graph_us(lambda: ok(lib.qmoe_probe_empty(1, cur())), 200), 3),
        "read_4MB_1024wg": round(graph_us(lambda: ok(lib.qmoe_probe_stream(
            ctypes.c_void_p(small.data_ptr()), small.numel(), 1024, ctypes.c_void_p(out.data_ptr()), cur())), 200), 3),
    }
    del small
    window = 18560 * 4096  # 76,021,760 bytes: the decode block's touched weights at T = 1
    big = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
    n_win = big.numel() // window
    res["hbm_read_76MB_GBps"] = {}
    for blocks in (256, 1024):
        def rotate():
            for w in range(n_win):
                ok(lib.qmoe_probe_stream(ctypes.c_void_p(big.data_ptr() + w * window), window, blocks,
                                         ctypes.c_void_p(out.data_ptr()), cur()))
        rotate()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(3):
            rotate()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (3 * n_win)
        res["hbm_read_76MB_GBps"][f"{blocks}wg"] = round(window / (us * 1e-6) / 1e9, 1)
        res["hbm_read_76MB_GBps"][f"{blocks}wg_us"] = round(us, 2)
    del big
    l2 = torch.ones(512 * 1024, dtype=torch.uint8, device=dev)
    n_cu = torch.cuda.get_device_properties(dev).multi_processor_count
    res["l2_read_TBps"] = {}
    for name, dma in (("vgpr", 0), ("lds_dma", 1)):
        blocks, iters = n_cu, 2048
        launch = lambda: ok(lib.qmoe_probe_l2(ctypes.c_void_p(l2.data_ptr()), blocks, iters, dma,
                                              ctypes.c_void_p(out.data_ptr()), cur()))
        launch()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            launch()
        e1.record()
        torch.cuda.synchronize()
        secs = e0.elapsed_time(e1) * 1e-3 / 5
        res["l2_read_TBps"][name] = round(blocks * 4 * iters * 8192 / secs / 1e12, 2)
    return res


def bench_attention(dev, B=8, S=1024, ctx_points=(1280, 8192), reps=10):
    """One GQA attention layer (QKV+qk-norm+RoPE, flash attention, o_proj +
    residual): prefill B x S, then single-token decode steps at the given
    context lengths (cache capacity 8192 + 1)."""
    import torch

    from qmoe.attention import Attention, KVCache, rope_tables

    Hq, Hkv, D, Hd = 32, 4, 128, 2048
    g = torch.Generator(device=dev).manual_seed(4)
    rnd = lambda *sh: torch.empty(*sh, dtype=torch.bfloat16, device=dev).normal_(0.0, 0.02, generator=g)
    one = torch.ones(D, dtype=torch.bfloat16, device=dev)
    att = Attention(rnd((Hq + 2 * Hkv) * D, Hd), one, one, rnd(Hd, Hq * D), Hq, Hkv, D, 1e-6)
    cap = max(ctx_points) + 1
    cache = KVCache(B, Hkv, cap, D, dev)
    cos, sin = rope_tables(D, cap, 1.0e6, dev)
    x = torch.randn(B * S, Hd, generator=g, device=dev).to(torch.bfloat16)
    res = torch.zeros(B * S, Hd, device=dev)
    pos = torch.arange(S, device=dev, dtype=torch.int32).repeat(B)

    def pre():
        att.forward(x, res, pos, B, S, cache, cos, sin, 0)

    secs, ev_secs, done = time_graph(pre, 1, reps, 2)
    # QKV + o_proj GEMMs and causal attention (S^2/2 scores, QK^T and PV)
    flops = 2 * B * S * Hd * (Hq + 2 * Hkv) * D + 2 * B * S * Hq * D * Hd + 2 * 2 * B * Hq * S * S // 2 * D
    t_pre = ev_secs / done
    out = {"prefill_us": t_pre * 1e6, "prefill_TFLOPs": flops / t_pre / 1e12,
           "prefill_mfma_frac": flops / t_pre / 1e12 / BF16_PEAK_TFLOPS, "prefill_flop": flops,
           "prefill_tokens_per_s": B * S / t_pre,
           "_weights": (att.wqkv, att.q_norm, att.k_norm, att.wo)}
    xd = torch.randn(B, Hd, generator=g, device=dev).to(torch.bfloat16)
    rd = torch.zeros(B, Hd, device=dev)
    for L in ctx_points:
        pd = torch.full((B,), L - 1, device=dev, dtype=torch.int32)

        byts = ((Hq + 2 * Hkv) * D * Hd + Hd * Hq * D) * 2 + B * Hkv * L * D * 2 * 2
        bucket = min(cap, 1 << max(8, (L - 1).bit_length()))  # the model's decode-graph bucket
        for tag, mc in (("", bucket), ("_full_launch", None)):
            def dec():
                att.forward(xd, rd, pd, B, 1, cache, cos, sin, 0, max_ctx=mc)

            secs, ev_secs, done = time_graph(dec, 1, 200, 20)
            us = ev_secs / done * 1e6
            out[f"decode_ctx{L}{tag}_us"] = us
            out[f"decode_ctx{L}{tag}_GBps"] = byts / (us * 1e-6) / 1e9
            out[f"decode_ctx{L}{tag}_hbm_frac"] = byts / (us * 1e-6) / 1e9 / HBM_PEAK_GBS
            out[f"decode_ctx{L}{tag}_tokens_per_s"] = B / (us * 1e-6)
        out[f"decode_ctx{L}_bytes"] = byts
    return out


def bench_model(dev, prompt_len=640, new_tokens=256, n_layers=48):
    """Full Qwen3-30B-A3B-shaped model, random-init bf16, batch 1: TTFT of a
    640-token prompt of uniform random ids, then greedy decode tokens/s."""
    import torch

    sys.path.insert(0, os.path.join(ROOT, "nki-moe-7013_amd"))
    import qwen_with_nki as qn

    nc = qn.MoENeuronConfig(batch_size=1, seq_len=prompt_len + new_tokens, max_length=prompt_len + new_tokens)
    cfg = qn.Qwen3MoeInferenceConfig(nc)
    cfg.num_hidden_layers = n_layers
    m = qn.NeuronQwen3MoeForCausalLM(None, cfg)
    t0 = time.perf_counter()
    m.load()
    torch.cuda.synchronize()
    print(f"[bench] model: 48 layers loaded (random init) in {time.perf_counter() - t0:.1f}s",
          file=sys.stderr, flush=True)
    prompt = torch.randint(0, cfg.vocab_size, (1, prompt_len), generator=torch.Generator().manual_seed(0))
    touched = None
    for w in range(2):  # warm-up (lazy allocations, graph capture)
        m.reset()
        first = m.prefill(prompt).argmax(-1)
        if touched is None:  # distinct experts each layer's prompt tokens route to (the prefill is deterministic)
            touched = [int(torch.unique(l.mlp.last_routing[2]).numel()) for l in m.model.layers]
        m.greedy_decode(first, 4)
        torch.cuda.synchronize()
        print(f"[bench] model: warm-up {w} done", file=sys.stderr, flush=True)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    m.reset()
    ev[0].record()
    first = m.prefill(prompt).argmax(-1)
    ev[1].record()
    toks = m.greedy_decode(first, new_tokens)
    ev[2].record()
    torch.cuda.synchronize()
    ttft_ms = ev[0].elapsed_time(ev[1])
    dec_ms = ev[1].elapsed_time(ev[2])
    # prompt-lookup speculation (spec_len 5) on the same prompt: the same tokens,
    # several verified per step when the n-gram candidates agree
    spec_out, _ = m.spec_generate(prompt, 8, spec_len=5)  # warm-up: captures the verify graph
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    spec_out, spec_stats = m.spec_generate(prompt, new_tokens + 1, spec_len=5)
    torch.cuda.synchronize()
    spec_ms = (time.perf_counter() - t0) * 1e3 - ttft_ms
    # leading tokens identical to plain greedy: the verification pass (5-token
    # shapes) and the one-token step round differently, so the two paths may
    # part at a near-tied step (top-2 logits within ~1e-3 on this random model)
    same = (spec_out[0, prompt_len + 1:].cpu() == toks[0].cpu()).int()
    spec_prefix = int(same.cumprod(0).sum())
    # TTFT reads the attention, router, norm and lm_head weights (2.46 GB of
    # bf16) and the weights of every expert the prompt routes to in each layer
    # (9,437,184 B each; all 128 experts of all 48 layers would make 60.44 GB),
    # and does 3.66 TFLOP (2 x 30.2 B non-embedding params x 640 tokens, and
    # the causal attention)
    ttft_all_bytes, ttft_flop = 60.44e9, 3.66e12
    ttft_bytes = ttft_all_bytes - (n_layers * E - sum(touched)) * EXPERT_BYTES
    return {
        "ttft_ms": ttft_ms,
        "ttft_hbm_frac": ttft_bytes / (ttft_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "ttft_bytes_GB": ttft_bytes / 1e9,
        "ttft_touched_experts_per_layer": {"mean": sum(touched) / len(touched), "min": min(touched),
                                           "max": max(touched)},
        "ttft_hbm_frac_if_all_experts": ttft_all_bytes / (ttft_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "ttft_mfma_frac": ttft_flop / (ttft_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
        "prefill_tokens_per_s": prompt_len / (ttft_ms * 1e-3),
        "decode_tokens_per_s": new_tokens / (dec_ms * 1e-3),
        "decode_ms_per_token": dec_ms / new_tokens,
        "decode_bytes_per_token_GB": 6.083,
        "decode_GBps": 6.083e9 / (dec_ms / new_tokens * 1e-3) / 1e9,
        "distinct_tokens": int(torch.unique(toks).numel()),
        # prompt-lookup speculation on this random-init model: its greedy
        # stream repeats a few tokens, which n-gram lookup predicts almost
        # always, so this is an upper bound on a repetitive sequence
        "spec_decode_tokens_per_s_repetitive_upper_bound": new_tokens / (spec_ms * 1e-3),
        "spec_tokens_per_verify": (spec_stats["accepted"] + spec_stats["verify_steps"]) / max(1, spec_stats["verify_steps"]),
        "spec_steps": spec_stats["steps"],
        "spec_greedy_prefix_match": spec_prefix,
    }


def model_child():
    """The full-model numbers from ``bench.py --only-model`` in a child process
    (its own 61 GB of weights; this process keeps its MoE layers)."""
    cmd = [sys.executable, os.path.abspath(__file__), "--only-model"]
    try:
        r = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=300)
    except subprocess.TimeoutExpired:
        return {"error": "timed out"}
    lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
    if r.returncode != 0 or not lines:
        return {"error": f"exit {r.returncode}", "stderr_tail": r.stderr[-400:]}
    return json.loads(lines[-1])


CAL_ELEMS = 64 << 20  # bf16 elements of the calibration kernel (128 MiB in, 128 MiB out)


def traffic_probe(T):
    """Child mode run under ``rocprofv3 --pmc``: decode-block calls over 8
    rotating layers (9.7 GB of experts, beyond the 256 MB Infinity Cache),
    then the calibration kernel: ``neg`` over CAL_ELEMS bf16 values (reads and
    writes exactly 2 * CAL_ELEMS bytes)."""
    import torch

    from qmoe import _lib
    from qmoe.moe import MoEBlock

    _lib.lib()
    dev = torch.device("cuda:0")
    layers = make_layers(8, dev, seed=3)
    g = torch.Generator(device=dev).manual_seed(99)
    x = torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16)
    res = torch.randn(T, H, generator=g, device=dev)
    blocks = [MoEBlock(*w, K_TOP) for w in layers]
    for _ in range(3):
        for b in blocks:
            b(x, res)
    src = torch.randn(CAL_ELEMS, generator=g, device=dev).to(torch.bfloat16)
    dst = torch.empty_like(src)
    for _ in range(2):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()


def measure_traffic(T):
    """HBM-side bytes per decode-block call from two rocprofv3 PMC runs of
    ``--traffic-probe`` (FETCH_SIZE, WRITE_SIZE; KiB per dispatch), each
    scaled by bytes / counter of the calibration kernel.  Returns a dict or
    None (rocprofv3 missing or failed)."""
    import csv
    import shutil
    import tempfile

    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(prof):
        return None
    res = {}
    with tempfile.TemporaryDirectory(prefix="qmoe_pmc_") as tmp:
        for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
            out = os.path.join(tmp, ctr)
            cmd = [prof, "--pmc", ctr, "-d", out, "-o", "c", "--output-format", "csv", "--",
                   sys.executable, os.path.abspath(__file__), "--traffic-probe", "--tokens", str(T)]
            try:
                subprocess.run(cmd, cwd=ROOT, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                               timeout=180, check=True)
            except Exception as exc:  # noqa: BLE001 - reported, never fatal
                print(f"[bench] traffic: {ctr} run failed: {exc}", file=sys.stderr, flush=True)
                return None
            files = [os.path.join(dp, f) for dp, _, fs in os.walk(out) for f in fs
                     if f.endswith("counter_collection.csv")]
            if not files:
                return None
            calls, cal = {}, []
            for r in csv.DictReader(open(files[0])):
                name, v = r["Kernel_Name"], float(r["Counter_Value"])
                if "neg_kernel" in name and int(r["Grid_Size"]) * 8 >= CAL_ELEMS:
                    cal.append(v)
                elif "qmoe::block_" in name:
                    calls.setdefault(name.split("(")[0], []).append(v)
            if not cal or not calls:
                return None
            factor = 2.0 * CAL_ELEMS / (min(cal) * 1024.0)
            # per call: the median dispatch of each kernel of the block, summed
            per_call = sum(sorted(v)[len(v) // 2] for v in calls.values()) * 1024.0 * factor
            res[ctr] = {"bytes_per_call": per_call, "scale": factor,
                        "kernels": sorted(calls), "dispatches": sum(len(v) for v in calls.values())}
    return res


def cpu_threads():
    """Host threads for the CPU baseline: the cores this process may run on
    (its affinity mask), capped by OMP_NUM_THREADS when that is set (a GPU
    job's share of the host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_model_name():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_median(fn, warmup, runs, budget_s):
    """Median seconds of fn() over up to ``runs`` timed calls after ``warmup``
    untimed ones; stops early once ``budget_s`` of timed work is spent (at
    least one timed call).  Returns (median seconds, calls timed)."""
    for _ in range(warmup):
        fn()
    ts, t_all = [], time.perf_counter()
    while len(ts) < runs and (not ts or time.perf_counter() - t_all < budget_s):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2], len(ts)


def cpu_baseline(layer, attn_gpu, lm_head_gpu, prefill_case, dev, seconds):
    """The fp32 CPU oracle (the reference's torch math restated) timed on the
    host cores, one figure per GPU workload, weights copied from the GPU run:

    * MoE block, decode schedule (qwen_with_nki.py:3456-3478) at T = 1, 8, 64;
    * MoE block, prefill schedule (5728-5789) at T = 128 and at T = 4096 with
      the GPU run's Zipf(1.1) router bias and tokens on the same layer
      (``prefill_case = (x, bias)``: the same routing);
    * the attention layer (10081-10109): B = 8 x 1024 prefill, one B = 8
      decode step at context 1280 and at 8192;
    * the model: one decoder layer (attention + MoE) at the model workload's
      shapes times 48, plus the final norm and lm_head, for decode (T = 1 at
      context 768) and for the 640-token prefill: an extrapolation.

    ``seconds`` bounds the headline T = 1 sample; the others take a median of
    up to 10 calls after warm-up, within a few seconds each."""
    import torch

    import oracle
    from qmoe import weights

    threads = cpu_threads()
    torch.set_num_threads(threads)
    t_start = time.perf_counter()
    w_router, w13, w2 = layer
    router = w_router.float().cpu()
    gate_up = torch.empty(E, H, 2 * I)
    for e0 in range(0, E, 16):  # unpack on the GPU in slices, then upcast on the host
        gate_up[e0 : e0 + 16] = weights.unpack_gate_up(w13[e0 : e0 + 16]).float().cpu()
    down = weights.unpack_down(w2).float().cpu()  # (E, I, H)
    g = torch.Generator().manual_seed(0)
    rnd = lambda *sh: torch.randn(*sh, generator=g)
    out = {}

    # headline: T = 1 decode MoE blocks, fresh tokens, until `seconds` elapse
    for _ in range(3):
        oracle.moe_block_decode(rnd(1, H), router, gate_up, down, K_TOP)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.moe_block_decode(rnd(1, H).to(torch.bfloat16), router, gate_up, down, K_TOP)
        n += 1
    dt = time.perf_counter() - t0
    out["moe_block_decode_T1"] = {"tokens_per_s": n / dt, "sample": f"{n} blocks in {dt:.1f} s"}
    for T in (8, 64):
        x = rnd(T, H)
        sec, k = cpu_median(lambda: oracle.moe_block_decode(x, router, gate_up, down, K_TOP), 2, 10, 4.0)
        out[f"moe_block_decode_T{T}"] = {"tokens_per_s": T / sec, "sample": f"median of {k} blocks"}
    x = rnd(128, H)
    sec, k = cpu_median(lambda: oracle.moe_block_prefill(x, router, gate_up, down, K_TOP), 2, 10, 4.0)
    out["moe_block_prefill_T128"] = {"tokens_per_s": 128 / sec, "sample": f"median of {k} blocks"}
    if prefill_case is not None:  # (tokens, Zipf bias) of the GPU run on this same layer
        xz, bz = prefill_case[0].float().cpu(), prefill_case[1].float().cpu()
        sec, k = cpu_median(lambda: oracle.moe_block_prefill(xz, router, gate_up, down, K_TOP, bz), 1, 5, 6.0)
        out["moe_block_prefill_T4096_zipf"] = {"tokens_per_s": 4096 / sec, "sample": f"median of {k} blocks"}

    # attention layer (B = 8), the GPU run's weights
    Hq, Hkv, D = 32, 4, 128
    wqkv, qn, kn, wo = (t.float().cpu() for t in attn_gpu)
    wq, wk, wv = wqkv.split([Hq * D, Hkv * D, Hkv * D])
    wa = {"q_proj": wq, "k_proj": wk, "v_proj": wv, "o_proj": wo, "q_norm": qn, "k_norm": kn}
    c = dict(n_q=Hq, n_kv=Hkv, head_dim=D, eps=1e-6, theta=1.0e6)
    xa = rnd(8, 1024, H)
    pa = torch.arange(1024).expand(8, 1024)
    sec, k = cpu_median(lambda: oracle.attention_layer(xa, wa, pa, c), 1, 3, 6.0)
    out["attention_B8_prefill1024"] = {"tokens_per_s": 8 * 1024 / sec, "sample": f"median of {k} layers"}
    del xa
    for L in (1280, 8192):
        past = (rnd(8, Hkv, L - 1, D), rnd(8, Hkv, L - 1, D))
        xd, pd = rnd(8, 1, H), torch.full((8, 1), L - 1)
        sec, k = cpu_median(lambda: oracle.attention_layer(xd, wa, pd, c, past), 2, 10, 4.0)
        out[f"attention_B8_decode_ctx{L}"] = {"tokens_per_s": 8 / sec, "sample": f"median of {k} steps"}
        del past

    # the model: one decoder layer x 48 + final norm + lm_head (extrapolated)
    wl = dict(wa, input_layernorm=torch.ones(H), post_attention_layernorm=torch.ones(H), router=router,
              gate_up_proj=gate_up, down_proj=down)
    cl = dict(c, top_k=K_TOP)
    lm = lm_head_gpu.float().cpu()
    norm_w = torch.ones(H)
    head = lambda h: oracle.rmsnorm(h, norm_w, 1e-6) @ lm.t()
    past = (rnd(1, Hkv, 767, D), rnd(1, Hkv, 767, D))
    xd, pd = rnd(1, 1, H), torch.full((1, 1), 767)
    sec_l, k = cpu_median(lambda: oracle.decoder_layer(xd, wl, pd, cl, past), 2, 10, 4.0)
    sec_h, _ = cpu_median(lambda: head(xd[:, 0]), 1, 5, 2.0)
    out["model_decode"] = {"tokens_per_s": 1.0 / (48 * sec_l + sec_h), "extrapolation": True,
                           "sample": f"one decoder layer at T=1, context 768 (median of {k}) x 48 + lm_head"}
    xp, pp = rnd(1, 640, H), torch.arange(640).view(1, 640)
    sec_l, k = cpu_median(lambda: oracle.decoder_layer(xp, wl, pp, cl), 1, 3, 6.0)
    ttft = 48 * sec_l + sec_h
    out["model_prefill_640"] = {"tokens_per_s": 640 / ttft, "ttft_ms": ttft * 1e3, "extrapolation": True,
                                "sample": f"one decoder layer at T=640 (median of {k}) x 48 + lm_head"}
    head_line = out["moe_block_decode_T1"]
    return {
        "value": head_line["tokens_per_s"],
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{head_line['sample']}: single-token MoE blocks (T=1, fp32, one layer's 128 experts, "
                   "decode schedule of qwen_with_nki.py:3456-3478)"),
        "cpu": cpu_model_name(),
        "host_cpu_count": os.cpu_count(),
        "threads": threads,
        "torch": torch.__version__,
        "dtype": "f32",
        "workloads": out,
        "secs": round(time.perf_counter() - t_start, 1),
    }


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: measures one GPU; --gpus {a.gpus} is not supported "
              "(multi-GPU sharding is design-only)", file=sys.stderr)
        sys.exit(2)
    if a.traffic_probe:
        traffic_probe(a.tokens)
        return
    traffic = None
    if not a.no_traffic and not (a.only_model or a.only_prefill or a.only_attention) and a.tokens <= 8:  # before this process touches the GPU
        traffic = measure_traffic(a.tokens)
        print(f"[bench] traffic: {traffic}", file=sys.stderr, flush=True)
    import torch

    from qmoe import _lib

    _lib.lib()
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False
    if a.only_model:
        res = bench_model(dev)
        print(f"[bench] model: {res}", file=sys.stderr, flush=True)
        print(json.dumps({"workload": "Qwen3-30B-A3B-shaped model, 48 layers, random-init bf16, batch 1, "
                                      "640-token prompt, 256 greedy steps", **res}))
        return
    if a.only_attention:
        res = bench_attention(dev)
        res.pop("_weights")
        print(f"[bench] attention: {res}", file=sys.stderr, flush=True)
        print(json.dumps({"workload": "GQA attention layer, B=8, prefill 1024, decode at ctx 1280 and 8192", **res}))
        return
    if a.only_prefill:
        layers = make_layers(min(a.layers, 4), dev)
        res = bench_prefill(layers, dev)
        res.pop("_cpu_case")
        print(f"[bench] prefill: {res}", file=sys.stderr, flush=True)
        print(json.dumps({"workload": "Qwen3-30B-A3B MoE block, prefill T=4096, Zipf(1.1)-skewed routing, "
                                      "4 rotating layers", **res}))
        return
    t_setup = time.perf_counter()
    layers = make_layers(a.layers, dev)
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup
    print(f"[bench] {a.layers} layers of MoE weights resident ({a.layers * E * EXPERT_BYTES / 1e9:.1f} GB), "
          f"setup {setup_s:.1f}s", file=sys.stderr, flush=True)

    dec = bench_decode(layers, a.tokens, a.steps, a.warmup, dev)
    print(f"[bench] decode T={a.tokens}: {dec}", file=sys.stderr, flush=True)
    extra, prefill_case, attn_weights = {}, None, None
    if not a.no_prefill:
        extra["prefill_T4096"] = bench_prefill(layers, dev)
        prefill_case = extra["prefill_T4096"].pop("_cpu_case")
        print(f"[bench] prefill: {extra['prefill_T4096']}", file=sys.stderr, flush=True)
        extra["prefill_T128"] = bench_prefill(layers, dev, T=128, reps=50, zipf_s=None)
        extra["prefill_T128"].pop("_cpu_case")
        print(f"[bench] prefill T=128: {extra['prefill_T128']}", file=sys.stderr, flush=True)
    if not a.no_extra:
        for T in (8, 64):
            extra[f"decode_T{T}"] = bench_decode(layers, T, 480, 48, dev)
            print(f"[bench] decode T={T}: {extra[f'decode_T{T}']}", file=sys.stderr, flush=True)
        extra["attention_B8"] = bench_attention(dev)
        attn_weights = extra["attention_B8"].pop("_weights")
        print(f"[bench] attention: {extra['attention_B8']}", file=sys.stderr, flush=True)
    if not a.no_model:
        extra["model_48L"] = model_child()
        print(f"[bench] model: {extra['model_48L']}", file=sys.stderr, flush=True)

    peaks = measure_peaks(dev)
    print(f"[bench] measured peaks: {peaks}", file=sys.stderr, flush=True)
    for key in ("prefill_T4096", "prefill_T128"):
        if key in extra:
            extra[key]["experts_frac_of_measured_mfma"] = extra[key]["experts_TFLOPs"] / peaks["mfma_bf16_random_TFLOPs"]
    if "prefill_T4096" in extra:
        # hipBLASLt's rate over the same work and flop mix (gate_up : down =
        # 2 : 1) as one dense GEMM per projection: no gather, no skew
        lr = peaks["hipblaslt_bf16_TFLOPs"]
        lib_rate = 3.0 / (2.0 / lr["32768x1536x2048"] + 1.0 / lr["32768x2048x768"])
        extra["prefill_T4096"]["experts_frac_of_hipblaslt_dense"] = round(
            extra["prefill_T4096"]["experts_TFLOPs"] / lib_rate, 4)

    cpu = None
    if not a.no_cpu_baseline:
        if attn_weights is None:  # the attention leg was skipped: same shapes, fresh weights
            gw = torch.Generator(device=dev).manual_seed(4)
            mk = lambda *sh: torch.empty(*sh, dtype=torch.bfloat16, device=dev).normal_(0.0, 0.02, generator=gw)
            one = torch.ones(128, dtype=torch.bfloat16, device=dev)
            attn_weights = (mk(48 * 128, H), one, one, mk(H, 32 * 128))
        lm_head = torch.empty(151936, H, dtype=torch.bfloat16, device=dev).normal_(
            0.0, 0.02, generator=torch.Generator(device=dev).manual_seed(6))
        cpu = cpu_baseline(layers[0], attn_weights, lm_head, prefill_case, dev, a.cpu_seconds)
        del lm_head
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)

    # every throughput with its roofline fraction and, beside it, the CPU
    # oracle's figure for the same workload (cpu_baseline.workloads)
    cw = (cpu or {}).get("workloads", {})
    cpu_of = lambda k: round(cw[k]["tokens_per_s"], 2) if k in cw else None
    tp = {"moe_block_decode_T1": {
        "tokens_per_s": round(dec["tokens_per_s"], 1), "bound": "hbm", "hbm_frac": round(dec["block_frac"], 4),
        "cpu_tokens_per_s": cpu_of("moe_block_decode_T1")}}
    for T in (8, 64):
        d = extra.get(f"decode_T{T}")
        if d:
            tp[f"moe_block_decode_T{T}"] = {"tokens_per_s": round(d["tokens_per_s"], 1), "bound": "hbm",
                                            "hbm_frac": round(d["block_frac"], 4),
                                            "cpu_tokens_per_s": cpu_of(f"moe_block_decode_T{T}")}
    for key, name in (("prefill_T128", "moe_block_prefill_T128"), ("prefill_T4096", "moe_block_prefill_T4096_zipf")):
        d = extra.get(key)
        if d:
            flop = d["T"] * K_TOP * 2 * 3 * H * I
            bound = "mfma" if flop / (BF16_PEAK_TFLOPS * 1e12) > d["block_bytes"] / (HBM_PEAK_GBS * 1e9) else "hbm"
            tp[name] = {"tokens_per_s": round(d["tokens_per_s"], 1), "bound": bound,
                        "experts_mfma_frac": round(d["experts_mfma_frac"], 4),
                        "experts_frac_of_measured_mfma": round(d["experts_frac_of_measured_mfma"], 4),
                        "block_hbm_frac": round(d["block_hbm_frac"], 4), "cpu_tokens_per_s": cpu_of(name)}
            if "experts_frac_of_hipblaslt_dense" in d:
                tp[name]["experts_frac_of_hipblaslt_dense"] = d["experts_frac_of_hipblaslt_dense"]
    at = extra.get("attention_B8")
    if at:
        tp["attention_B8_prefill1024"] = {"tokens_per_s": round(at["prefill_tokens_per_s"], 1), "bound": "mfma",
                                          "mfma_frac": round(at["prefill_mfma_frac"], 4),
                                          "cpu_tokens_per_s": cpu_of("attention_B8_prefill1024")}
        for L in (1280, 8192):
            tp[f"attention_B8_decode_ctx{L}"] = {
                "tokens_per_s": round(at[f"decode_ctx{L}_tokens_per_s"], 1), "bound": "hbm",
                "hbm_frac": round(at[f"decode_ctx{L}_hbm_frac"], 4),
                "cpu_tokens_per_s": cpu_of(f"attention_B8_decode_ctx{L}")}
    md = extra.get("model_48L", {})
    if "decode_tokens_per_s" in md:
        tp["model_decode"] = {"tokens_per_s": round(md["decode_tokens_per_s"], 2), "bound": "hbm",
                              "hbm_frac": round(md["decode_GBps"] / HBM_PEAK_GBS, 4),
                              "cpu_tokens_per_s": cpu_of("model_decode"), "cpu_extrapolated": True}
        tp["model_prefill_640"] = {"tokens_per_s": round(md["prefill_tokens_per_s"], 1), "bound": "hbm",
                                   "ttft_ms": round(md["ttft_ms"], 3), "hbm_frac": round(md["ttft_hbm_frac"], 4),
                                   "mfma_frac": round(md["ttft_mfma_frac"], 4),
                                   "cpu_tokens_per_s": cpu_of("model_prefill_640"), "cpu_extrapolated": True}

    achieved = dec["block_GBps"]
    pre = extra.get("prefill_T4096", {})
    line = {
        "metric": METRIC,
        "value": round(dec["tokens_per_s"], 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": dec["steps"],
        "warmup": a.warmup,
        "ms_per_step": round(dec["us_per_block"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) weights, N(0,1) activations, seeded)",
        "config": {
            "workload": f"Qwen3-30B-A3B MoE block, decode T={a.tokens}, H=2048, 128 experts top-8, "
                        f"I=768, {a.layers} rotating layers resident, HIP-graph replay",
            "tokens_per_step": a.tokens,
            "layers_rotated": a.layers,
            "parallelism": "single GPU",
        },
        "moe_block_GBps": round(dec["block_GBps"], 1),
        "moe_block_hbm_frac": round(dec["block_frac"], 4),
        "moe_block_us_spread": dec["us_per_block_spread"],
        "prefill_moe_block_tokens_per_s": round(pre["tokens_per_s"], 1) if pre else None,
        "prefill_experts_mfma_frac": round(pre["experts_mfma_frac"], 4) if pre else None,
        "prefill_block_hbm_frac": round(pre["block_hbm_frac"], 4) if pre else None,
        "prefill_experts_frac_of_measured_mfma": round(pre["experts_frac_of_measured_mfma"], 4) if pre else None,
        "model_decode_tokens_per_s": round(md["decode_tokens_per_s"], 2) if "decode_tokens_per_s" in md else None,
        "model_decode_hbm_frac": round(md["decode_GBps"] / HBM_PEAK_GBS, 4) if "decode_GBps" in md else None,
        "model_ttft_ms": round(md["ttft_ms"], 3) if "ttft_ms" in md else None,
        "model_prefill_tokens_per_s": round(md["prefill_tokens_per_s"], 1) if "prefill_tokens_per_s" in md else None,
        "throughputs": tp,
        "roofline": {
            "kernel": ("qmoe_moe_decode_block: block_fused_kernel (one launch)" if a.tokens == 1 else
                       "qmoe_moe_decode_block: block_logits_kernel + block_expert_kernel + "
                       "block_reduce_kernel (one call, 3 launches)") if a.tokens <= 8 else
                      ("MoE block (route + moe_gateup_gemv_kernel + moe_down_mfma_kernel + combine)"
                       if a.tokens <= _gemv_max_tokens() else
                       "MoE block (route + permute + moe_gateup_grouped_kernel + moe_down_grouped_kernel + combine)"),
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": (round(traffic["FETCH_SIZE"]["bytes_per_call"] + traffic["WRITE_SIZE"]["bytes_per_call"])
                        if traffic else None),
            "traffic_detail": ({k: {"bytes": round(v["bytes_per_call"]), "scale": round(v["scale"], 4)}
                                for k, v in traffic.items()} if traffic else None),
            "algorithmic_bytes_per_launch": dec["block_bytes"],
            "launch_us_mean": round(dec["us_per_block"], 3),
            "frac_of_measured_copy": round(achieved / peaks["hbm_copy_GBps"], 4),
        },
        "measured_peaks": peaks,
        "cpu_baseline": cpu,
        "extra": extra or None,
        "git": git_sha(),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
