"""Benchmark of the Library read on one MI355X.

Default workload: batched paged decode — B = 64 sequences, each reading its own Library of
U{8..64} chunks x 512 slots (chunk = page, pages placed by a seeded shuffle), d_s = 2048, fp16
K = V slots with ragged tails, top-8 routing.  One step = routing (q.S scores + top-k + softmax)
plus the split-K masked-softmax read of the routed pages for all 64 query rows, inputs resident
in HBM.  Prints ONE JSON line.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--workload batched_paged_decode]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

import torch

METRIC = "Library-read query tokens/sec + achieved HBM GB/s (% peak) at B=64 paged decode"
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="batched_paged_decode",
                    choices=["batched_paged_decode", "single_decode", "prefill", "multi_depth",
                             "pool_build", "d18", "op_b"])
    ap.add_argument("--nsplit", type=int, default=None)
    ap.add_argument("--rows", type=int, default=32, help="op_b: decode rows (requests) per call")
    ap.add_argument("--cpu-sample", type=int, default=16, help="sequences in the CPU baseline sample (0 = skip)")
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--no-graph", action="store_true", help="time the eager step only (no HIP graph replay)")
    ap.add_argument("--no-prefill", action="store_true",
                    help="batched_paged_decode: leave out the prefill block of the JSON line")
    ap.add_argument("--prefill-steps", type=int, default=20,
                    help="batched_paged_decode: timed steps of the prefill block (10 warm-up steps)")
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="after the timed loop, copy a buffer of this size 3 times (a plain copy "
                         "kernel of known bytes, to scale rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def traffic_from_profile(workload: str, name: str | None = None):
    """HBM bytes per launch of the workload's kernels measured offline with rocprofv3 --pmc
    (FETCH_SIZE and WRITE_SIZE, scaled by the same counters on a copy of known size); the
    summary lives in profiles/ next to the command that produced it.  None when absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        name or f"decode_read_{workload}_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def cpu_baseline(P, q, top_k, n_seq, reps):
    """The reference path on the host cores: per sequence one call of route + read over ALL of its
    chunks in fp32 (the reference's order, xenc/injector.py:220-265), via the CPU oracle."""
    import oracle as O
    torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
    B = q.shape[0]
    n_seq = min(n_seq, B)
    qc = q.cpu()

    def routed_only(qv, K, M, S):
        # Route over every chunk, then read only the kept ones (the others carry weight 0): per
        # kept chunk a masked softmax of K_c q and its weighted sum of K_c rows (views, no copies).
        logit = (qv @ S.T) * 10.0
        C = S.shape[0]
        k = C if not top_k or top_k >= C else top_k
        order = O.topk_order(logit, k)[0].tolist()
        w = O.route(qv, S, 10.0, top_k)[0]
        r = torch.zeros(K.shape[-1])
        for c in order:
            a = torch.softmax((K[c] @ qv[0] * 12.0).masked_fill(~M[c], float("-inf")), -1)
            r += w[c] * (a @ K[c])
        return r

    def median_time(fn):
        fn()                                                  # warm-up
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    times, times_routed, slots = [], [], 0
    for b in range(n_seq):
        K, M, S = P.library(b)
        K, M, S = K.cpu(), M.cpu(), S.cpu()
        qb = qc[b].view(1, 1, -1)
        times.append(median_time(lambda: O.branch_read(qb, K, M, S, top_k=top_k)))
        times_routed.append(median_time(lambda: routed_only(qc[b].view(1, -1), K, M, S)))
        slots += int(M.sum())
        del K, M, S
    total = sum(times)
    return {"value": n_seq / total, "unit": "query tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"first {n_seq} of {B} sequences, one fp32 route+read call each over all of the "
                       f"sequence's chunks ({slots} slots), median of {reps} reps after 1 warm-up; "
                       f"CPU oracle on {cpu_model()}, os.cpu_count()={os.cpu_count()}"),
            "routed_only": {"value": n_seq / sum(times_routed), "unit": "query tokens/s",
                            "sample": (f"the same sequences: route over all chunks, then read only the "
                                       f"top-{top_k} routed chunks, fp32")}}


MFMA_FP16_PEAK_TFLOPS = 2500.0


def measured_mfma_peak(dev) -> float:
    """fp16 MFMA TFLOP/s the device sustains on a pure register-operand MFMA loop
    (xenc_calibrate_mfma: 2 waves per SIMD on every CU, random operands), best of 3 after a
    warm-up: the ceiling the vendor peak's clock does not hold under sustained load."""
    from kv_skill_v2_amd._lib import check, lib, stream_handle
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    src = (torch.rand(65536 * 8, generator=torch.Generator().manual_seed(1)) - 0.5).to(torch.float16).to(dev)
    waves, rounds = 8, 4000
    out = torch.empty(cus * waves * 64, dtype=torch.float32, device=dev)
    L, st = lib(), stream_handle(dev)
    best = 0.0
    for rep in range(4):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        check(L.xenc_calibrate_mfma(src.data_ptr(), 65536, waves, cus, rounds, out.data_ptr(), st),
              "xenc_calibrate_mfma")
        e1.record()
        torch.cuda.synchronize()
        if rep:
            best = max(best, cus * waves * rounds * 16 * 32768.0 / (e0.elapsed_time(e1) * 1e-3) / 1e12)
    return best


def measured_stream_peak(dev, gib: int = 2) -> float:
    """HBM GB/s of a nontemporal 16-byte streaming read over `gib` GiB (xenc_calibrate_stream),
    best of 3 after a warm-up: the read rate the decode kernels stream pages at."""
    from kv_skill_v2_amd._lib import check, lib, stream_handle
    buf = torch.ones(gib << 30, dtype=torch.uint8, device=dev)
    blocks = (gib << 30) >> 21          # 2 MiB per workgroup, like a page of the batched decode
    out = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
    L, st = lib(), stream_handle(dev)
    best = 0.0
    for rep in range(4):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        check(L.xenc_calibrate_stream(buf.data_ptr(), buf.numel(), blocks, out.data_ptr(), st), "xenc_calibrate_stream")
        e1.record()
        torch.cuda.synchronize()
        if rep:
            best = max(best, buf.numel() / (e0.elapsed_time(e1) * 1e-3) / 1e9)
    del buf
    return best


def settle(step, min_ms: float = 30.0, max_calls: int = 4000) -> int:
    """Untimed calls of `step` until the GPU has been busy with them for `min_ms`, before a timed
    region: these boxes raise their clocks only after several milliseconds of sustained load (the
    op-B read timed 8 % slow after 10 warm-up calls of 0.34 ms, and a 16-step graph replayed once
    right after its capture and checks ran 3 % behind the same graph replayed warm).  Returns the
    number of calls; the workloads record it as config.settle_calls.  The W warm-up steps of the
    command line follow it unchanged."""
    step()                 # one-time set-up of a first call (allocations, code loading) stays
    torch.cuda.synchronize()   # out of the window
    n = 1
    t0 = time.perf_counter()
    while n < max_calls:
        for _ in range(4):
            step()
        n += 4
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= min_ms:
            break
    return n


def timed_steps(step, steps: int, stream, host: list | None = None):
    """Times `steps` back-to-back calls of `step` with nothing else queued between them, closed
    by a device synchronisation on each side.  Returns (wall ms per step, GPU ms per step): the
    second from ONE event pair around the whole region on `stream`, so it is the span the kernels
    of the K steps occupy, gaps between them included.  A timing event between steps would add
    GPU idle time of its own (about 10 us per pair on this stack), so none is recorded there.
    `host`, when given, receives the host time per step spent issuing the calls (the loop before
    the closing synchronisation): the step's host cost while the launch queue does not block."""
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    a.record(stream)
    for _ in range(steps):
        step()
    t_issue = time.perf_counter()
    b.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    if host is not None:
        host.append((t_issue - t0) * 1e3 / steps)
    return wall, a.elapsed_time(b) / steps


_GRAPH_LAUNCH = None


def _hip_graph_launch():
    """hipGraphLaunch of the HIP runtime torch has loaded (found by its path in /proc/self/maps,
    so no second runtime is ever opened), or None.  A graph replayed through it skips the
    per-replay bookkeeping of torch's CUDAGraph.replay(), which costs about 6 us of host time
    and 4 us of wall time per replay on this stack."""
    global _GRAPH_LAUNCH
    if _GRAPH_LAUNCH is None:
        _GRAPH_LAUNCH = False
        try:
            with open("/proc/self/maps") as f:
                paths = {ln.split()[-1] for ln in f if "libamdhip64" in ln and "/" in ln}
            if len(paths) == 1:
                import ctypes
                fn = ctypes.CDLL(paths.pop()).hipGraphLaunch
                fn.argtypes, fn.restype = [ctypes.c_void_p, ctypes.c_void_p], ctypes.c_int
                _GRAPH_LAUNCH = fn
        except (OSError, AttributeError):
            _GRAPH_LAUNCH = False
    return _GRAPH_LAUNCH or None


def graph_replayer(gph, dev):
    """A callable that launches the instantiated graph on the current stream of `dev`."""
    launch = _hip_graph_launch()
    if launch is None:
        return gph.replay
    exe = gph.raw_cuda_graph_exec()
    from kv_skill_v2_amd._lib import stream_handle
    st = stream_handle(dev)

    def replay():
        rc = launch(exe, st)
        if rc:
            raise RuntimeError(f"hipGraphLaunch failed: {rc}")
    return replay


def graph_timings(step, same, steps: int, dev, per_graph: int = 16) -> dict:
    """HIP-graph timings of `step` (returning its output tensor): one step per graph, and
    `per_graph` steps captured back to back in one graph (the per-step cost inside a larger
    captured sequence, as a captured serving step sees it).  Every replay is first checked
    against the eager result (graph_of).  Returns {"ms", "span_ms", "ms_in_graph",
    "span_ms_in_graph"}; values are None where a check failed."""
    stream = torch.cuda.current_stream(dev)
    out = {"ms": None, "span_ms": None, "ms_in_graph": None, "span_ms_in_graph": None}
    gph, _ = graph_of(step, same)
    if gph is not None:
        settle(graph_replayer(gph, dev))
        out["ms"], out["span_ms"] = timed_steps(graph_replayer(gph, dev), steps, stream)
    gph16, _ = graph_of(lambda: [step() for _ in range(per_graph)][-1], same)
    if gph16 is not None:
        settle(graph_replayer(gph16, dev))
        ms, span = timed_steps(graph_replayer(gph16, dev), max(1, steps // per_graph), stream)
        out["ms_in_graph"], out["span_ms_in_graph"] = ms / per_graph, span / per_graph
    return out


def fastest_timing(eager_ms: float, eager_span: float, gt: dict):
    """(name, ms per step, GPU span per step) of the fastest measured way to run the step: eager
    launches, one step per graph, or 16 steps per graph."""
    cands = [("eager", eager_ms, eager_span)]
    if gt.get("ms") is not None:
        cands.append(("hip_graph", gt["ms"], gt["span_ms"]))
    if gt.get("ms_in_graph") is not None:
        cands.append(("hip_graph_16_steps", gt["ms_in_graph"], gt["span_ms_in_graph"]))
    return min(cands, key=lambda c: c[1])


def graph_of(step, same):
    """`step` captured once in a HIP graph after a warm-up call on a side stream.  Returns (graph,
    the captured call's output), or (None, None) when a replay does not reproduce the eager
    result: three replays, each followed by a synchronisation, `same(captured output)`, an eager
    call and another synchronisation."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    gph = torch.cuda.CUDAGraph()
    # Captured on the warm-up stream: the per-stream decode workspace already exists there, so
    # its one-time counter initialisation is not captured into the graph.
    with torch.cuda.graph(gph, stream=s):
        out = step()
    for _ in range(3):
        gph.replay()
        torch.cuda.synchronize()
        if not same(out):
            return None, None
        step()
        torch.cuda.synchronize()
    return gph, out


def measure_prefill(steps: int, warmup: int, cpu_sample: int) -> dict:
    """Prefill/registration read: 4 documents x 2048 query rows, each document a Library of 32 x 512
    slots (ragged tail), d_s = 2048, dense routing (every chunk read), fp16 MFMA with fp32
    accumulation; forward (route + read) and the dQ backward (read + route) against a seeded
    upstream gradient ~N(0,1).  Algorithmic FLOPs per document and direction: 4 * T * sum(n_valid) * d
    (two GEMMs of 2 FLOPs per multiply-add; recomputation is not counted).  Returns the timings,
    TFLOP/s and fractions of the fp16 MFMA peak (vendor and measured) plus the CPU baseline."""
    from kv_skill_v2_amd import ops, synth

    dev = torch.device("cuda:0")
    G, T, C, N, d = 4, 2048, 32, 512, 2048
    P = synth.pool([C] * G, N, d, device=dev)
    lib = ops.PagedLibrary(P.pages, P.chunk_page, P.chunk_nvalid, P.chunk_ptr, P.S,
                           n_chunks=P.n_chunks, nvalid=P.nvalid)
    plan = ops.row_plan(lib, [T] * G)
    q = synth.queries(G * T, d, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    g_up = torch.randn(G * T, d, generator=gen, device=dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    lib.fragment_pages(0), lib.fragment_pages(1)  # one-time fragment-ordered copies of the pages
    torch.cuda.synchronize()
    frag_ms = (time.perf_counter() - t0) * 1e3

    def fwd():
        w, _, _, qh = ops.route_topk_rows(q, lib, plan, top_k=0, emit_f16=True)
        r, p = ops.prefill_forward(q, w, lib, plan, qh=qh)
        return w, r, p

    def bwd(w, p):
        return ops.prefill_backward_routed(g_up, w, p, lib, plan, route_temp=10.0)

    def step():
        w, _, p = fwd()
        bwd(w, p)

    settle_calls = settle(step)
    for _ in range(warmup):
        step()
    stream = torch.cuda.current_stream(dev)
    ms_step, gpu_ms_step = timed_steps(step, steps, stream)
    # The split between the directions, from a second loop of K steps with events between the
    # forward and the backward (outside the timed region above: the events add idle time).
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for i in range(steps):
        evs[i][0].record(stream)
        w, r, p = fwd()
        evs[i][1].record(stream)
        bwd(w, p)
        evs[i][2].record(stream)
    torch.cuda.synchronize()
    fwd_ms = statistics.mean(e[0].elapsed_time(e[1]) for e in evs)
    bwd_ms = statistics.mean(e[1].elapsed_time(e[2]) for e in evs)
    nvalid = sum(P.nvalid)
    flops = 4.0 * T * nvalid * d                  # per direction, all documents
    fwd_tf = flops / (fwd_ms * 1e-3) / 1e12
    bwd_tf = flops / (bwd_ms * 1e-3) / 1e12
    mfma_meas = measured_mfma_peak(dev)

    cpu = None
    if cpu_sample > 0:
        import oracle as O
        torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
        K, M, S = P.library(0)
        K, M, S = K.cpu(), M.cpu(), S.cpu()
        qc = q[:T].cpu().view(1, T, d).requires_grad_(True)
        gc = g_up[:T].cpu().view(1, T, d)
        t0 = time.perf_counter()
        rr, _ = O.branch_read(qc, K, M, S, top_k=0)
        (rr * gc).sum().backward()
        cpu_s = time.perf_counter() - t0
        cpu = {"value": 2 * 4.0 * T * sum(P.nvalid[:C]) * d / cpu_s / 1e12, "unit": "TFLOP/s (fwd+bwd)",
               "cores": torch.get_num_threads(), "kind": "port",
               "sample": (f"1 of {G} documents ({T} rows x {C} chunks), fp32 route+read forward and torch "
                          f"autograd backward in the reference's operation order, 1 rep ({cpu_s:.2f} s); "
                          f"CPU oracle on {cpu_model()}, os.cpu_count()={os.cpu_count()}")}
    del lib, P, q, g_up
    torch.cuda.empty_cache()
    return {"steps": steps, "warmup": warmup, "ms_per_step": ms_step, "gpu_ms_per_step": gpu_ms_step,
            "tflops_fwd_bwd": 2 * flops / (ms_step * 1e-3) / 1e12, "algorithmic_flops_per_direction": flops,
            "config": {"documents": G, "rows_per_document": T, "chunks": C, "slots_per_page": N, "d_s": d,
                       "routing": "dense (top_k=0)", "accumulate": "fp32", "fragment_pages_ms_once": frag_ms,
                       "settle_calls": settle_calls},
            "fwd": {"ms": fwd_ms, "tflops": fwd_tf, "frac": fwd_tf / MFMA_FP16_PEAK_TFLOPS,
                    "frac_of_measured": fwd_tf / mfma_meas if mfma_meas else None},
            "bwd": {"ms": bwd_ms, "tflops": bwd_tf, "frac": bwd_tf / MFMA_FP16_PEAK_TFLOPS,
                    "frac_of_measured": bwd_tf / mfma_meas if mfma_meas else None},
            "peak_tflops": MFMA_FP16_PEAK_TFLOPS, "measured_peak_tflops": mfma_meas,
            "cpu_baseline": cpu}


def bench_prefill(args):
    """The prefill/registration read (measure_prefill) as its own JSON line."""
    pf = measure_prefill(args.steps, args.warmup, args.cpu_sample)
    fwd_tf = pf["fwd"]["tflops"]
    traffic = traffic_from_profile("prefill", "prefill_read_traffic.json")
    out = {
        "metric": "Prefill/registration read TFLOP/s (fwd and dQ bwd), 4 docs x 2048 rows x 32x512 slots",
        "value": pf["tflops_fwd_bwd"], "unit": "TFLOP/s (fwd+bwd)", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": pf["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "prefill", **pf["config"]},
        "fwd": pf["fwd"], "bwd": pf["bwd"],
        "roofline": {"bound": "mfma", "kernel": "scores_kernel + readout_kernel (fwd)",
                     "achieved": fwd_tf, "peak": MFMA_FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": fwd_tf / MFMA_FP16_PEAK_TFLOPS,
                     "traffic": traffic["bytes_per_launch"] if traffic else None,
                     "traffic_source": traffic["source"] if traffic else None,
                     "algorithmic_flops": pf["algorithmic_flops_per_direction"],
                     "measured_peak": pf["measured_peak_tflops"],
                     "frac_of_measured": pf["fwd"]["frac_of_measured"]},
        "cpu_baseline": pf["cpu_baseline"],
    }
    print(json.dumps(out), flush=True)


def bench_multi_depth(args):
    """Multi-depth selector decode: 8 depth Libraries (64 x 512 slots, d_s = 2560) shared by a batch
    of 32 tokens; the selector keeps the top-2 depths per token (seeded logits), so 64 (token,
    depth) query rows are routed (top-8 chunks of their depth) and read in ONE route and ONE read
    launch (the depth is the row's library).  Each read is written back through its depth's
    B [5120, 2560] fp32 with gate and gain folded in (one xenc_write_back launch streams the B of
    every selected depth once), then
    rescaled to the selector's matched norm and weighted.  The unselected depths are not read (the
    reference reads all 8 and multiplies 6 by zero).  Step = everything after the selector logits;
    the two updates of a token (one per selected depth, applied at different layers in a model)
    are summed into one [32, 5120] output here.  Algorithmic bytes: the unique routed pages of each
    depth (union over the batch) x valid slots x d x 2, the S of the 8 Libraries, every B read,
    and the activations."""
    from kv_skill_v2_amd import ops, synth
    from kv_skill_v2_amd.multi_depth import MultiDepthDecode
    from kv_skill_v2_amd.selector import LayerSelector, rms_norm

    c = synth.MULTI_DEPTH
    dev = torch.device("cuda:0")
    P, z, q_all, h, BwT = synth.multi_depth_workload(dev)
    Bw = BwT.transpose(1, 2).contiguous()                            # [L, d_r, d] out-major rows
    del BwT
    lib = ops.PagedLibrary(P.pages, P.chunk_page, P.chunk_nvalid, P.chunk_ptr, P.S,
                           n_chunks=P.n_chunks, nvalid=P.nvalid)
    B, L, d, dr, k = c["B"], c["depths"], c["d"], c["d_r"], c["top_k"]
    sel = LayerSelector(dr, list(range(L)), k=c["k_sel"]).to(dev)
    gate_w = torch.zeros(dr, device=dev)
    gate_b = torch.full((L,), -2.0, device=dev)
    log_gain = torch.zeros(L, device=dev)
    hn = rms_norm(h)
    md = MultiDepthDecode(lib, Bw, gate_w, gate_b, log_gain, sel.log_alpha, k_sel=c["k_sel"], top_k=k,
                          nsplit=args.nsplit)

    def step():
        return md(z, q_all, h, hn)

    _, idx0, qg0 = step()
    torch.cuda.synchronize()
    pages = set()
    ptr_h = P.chunk_ptr.cpu().tolist()
    for row, (g, cs) in enumerate(zip(qg0.cpu().tolist(), idx0.cpu().tolist())):
        pages.update((g, ch) for ch in cs if ch >= 0)
    page_bytes = sum(P.nvalid[ptr_h[g] + ch] for g, ch in pages) * d * 2
    used = len(set(qg0.cpu().tolist()))
    bytes_step = (page_bytes + L * c["chunks"] * d * 4 + used * d * dr * 4
                  + 2 * B * c["k_sel"] * (d + dr) * 4 + B * dr * 4 * 2)
    settle_calls = settle(step)
    for _ in range(args.warmup):
        step()
    stream = torch.cuda.current_stream(dev)
    host = []
    ms_eager, span_eager = timed_steps(step, args.steps, stream, host)

    # The step captured once in a HIP graph and replayed.  Every replay is checked against the
    # eager result (bit for bit) with eager work and synchronisation in between; on
    # any mismatch the eager time is reported.
    gt = {"ms": None, "span_ms": None, "ms_in_graph": None, "span_ms_in_graph": None}
    if not args.no_graph:
        ref_out = step()[0].clone()
        gt = graph_timings(lambda: step()[0], lambda o: torch.equal(o, ref_out), args.steps, dev)
    ms_graph = gt["ms"]
    # The step runs every way; report the fastest measured one (named in config).
    timing, ms_step, span = fastest_timing(ms_eager, span_eager, gt)
    achieved = bytes_step / (span * 1e-3) / 1e9

    cpu = None
    if args.cpu_sample > 0:
        import oracle as O
        torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
        K, M, S = P.library(0)
        K, M, S = K.cpu(), M.cpu(), S.cpu()
        ql0 = q_all[0].cpu().view(B, 1, d)
        Bw0 = Bw[0].cpu()
        hc = h.cpu().view(B, 1, dr)
        O.branch_read(ql0[:1], K, M, S, top_k=k)                       # warm-up
        t0 = time.perf_counter()
        r0, _ = O.branch_read(ql0, K, M, S, top_k=k)
        dl0 = O.epilogue(O.rms_norm(hc), r0, Bw0, None, gate_w.cpu(), gate_b[0].cpu(), log_gain[0].cpu())
        O.selector_apply(dl0, hc, torch.ones(B, 1), math.log(0.02))
        t_layer = time.perf_counter() - t0
        cpu = {"value": B / (L * t_layer), "unit": "query tokens/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": (f"1 of the {L} depth layers the reference reads per token (all 64 chunks, fp32, "
                          f"route + read + B write-back + selector rescale for the batch of {B}), "
                          f"{t_layer:.2f} s, scaled by {L}; CPU oracle on {cpu_model()}, "
                          f"os.cpu_count()={os.cpu_count()}")}
    out = {
        "metric": "Multi-depth selector decode query tokens/sec + achieved HBM GB/s (% peak)",
        "value": B / (ms_step * 1e-3), "unit": "query tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "multi_depth", "depths": L, "chunks_per_depth": c["chunks"],
                   "slots_per_page": c["N"], "d_s": d, "d_reader": dr, "batch": B,
                   "selector_top_k": c["k_sel"], "top_k": k, "B_dtype": "fp32", "accumulate": "fp32",
                   "settle_calls": settle_calls,
                   "timing": timing, "ms_per_step_eager": ms_eager, "ms_per_step_graph": ms_graph,
                   "ms_per_step_in_16_step_graph": gt["ms_in_graph"],
                   "host_issue_us_per_step": host[0] * 1e3},
        "roofline": {"bound": "hbm", "kernel": "whole step (route + read + write-back + epilogue)",
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "algorithmic_bytes": bytes_step, "avg_launch_ms": span, "unique_routed_pages": len(pages),
                     "routed_page_reads": int((idx0 >= 0).sum()), "depths_used": used},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def bench_pool_build(args):
    """Library pool build from document caches: the batched-decode page set (64 documents of
    U{8..64} chunks x 512 slots, ragged tails, d_s = 2048) as back-to-back fp16 slot rows already
    in HBM, centred by a seeded mu; one step = one xenc_build_pages launch writing the fp16 pages,
    fp32 summary keys and valid counts.  Algorithmic bytes per launch: the slot rows read once
    (R x d x 2) plus the pages (C x 512 x d x 2, zero tails included), S (C x d x 4) and counts."""
    from kv_skill_v2_amd import ops, synth

    dev = torch.device("cuda:0")
    P, _, _, _ = synth.decode_workload("batched_paged_decode", device=dev)
    C, N, d = len(P.nvalid), P.pages.shape[1], P.pages.shape[2]
    by_chunk = P.pages[P.chunk_page.long()]                   # chunk order
    keep = torch.arange(N, device=dev).view(1, N) < P.chunk_nvalid.view(-1, 1)
    rows = by_chunk[keep].contiguous()                         # [R, d] fp16, chunks back to back
    off = torch.zeros(C + 1, dtype=torch.int64, device=dev)
    off[1:] = torch.cumsum(P.chunk_nvalid.long(), 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    mu = (0.05 * torch.randn(d, generator=gen, device=dev)).contiguous()
    del by_chunk, keep
    R = rows.shape[0]
    alg_bytes = R * d * 2 + C * N * d * 2 + C * d * 4 + C * 4 + (C + 1) * 8 + d * 4
    def step():
        ops.build_pages(rows, off, d, N, d, mu)

    settle_calls = settle(step)
    for _ in range(args.warmup):
        step()
    stream = torch.cuda.current_stream(dev)
    ms_step, k_ms = timed_steps(step, args.steps, stream)
    achieved = alg_bytes / (k_ms * 1e-3) / 1e9
    # Read + write ceiling for reference: torch's device copy of the slot rows (same order of
    # bytes read and written as the build).
    dst = torch.empty_like(rows)
    cev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(5)]
    for a, b in cev:
        a.record(stream)
        dst.copy_(rows)
        b.record(stream)
    torch.cuda.synchronize()
    copy_gbs = 2 * rows.numel() * 2 / (statistics.mean(a.elapsed_time(b) for a, b in cev[1:]) * 1e-3) / 1e9
    del dst

    cpu = None
    if args.cpu_sample > 0:
        import oracle as O
        torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
        nc = sum(P.n_chunks[:8])
        r_cpu = rows[: int(off[nc])].cpu()
        o = off[: nc + 1].cpu().tolist()
        chunk_rows = [r_cpu[o[c]:o[c + 1]] for c in range(nc)]
        mu_c = mu.cpu()
        t0 = time.perf_counter()
        for g in range(8):
            a, b = sum(P.n_chunks[:g]), sum(P.n_chunks[:g + 1])
            O.library_tensors(chunk_rows[a:b], dtype=torch.float32, center_mu=mu_c)
        cpu_s = time.perf_counter() - t0
        cpu = {"value": nc / cpu_s, "unit": "chunks/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": (f"documents 0-7 ({nc} chunks x {N} slots x {d}), fp32 Library padding + "
                          f"centring + summaries in the reference's operation order, one pass "
                          f"({cpu_s:.2f} s); CPU oracle on {cpu_model()}")}
    out = {
        "metric": "Library pool build from document caches: chunks/s and HBM GB/s (% peak)",
        "value": C / (ms_step * 1e-3), "unit": "chunks/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32 (fp16 in/out)", "data": "synthetic",
        "config": {"workload": "pool_build", "documents": len(P.n_chunks), "chunks": C,
                   "slot_rows": R, "slots_per_page": N, "d_s": d, "centred": True,
                   "settle_calls": settle_calls},
        "roofline": {"bound": "hbm", "kernel": "build_pages_kernel", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": None, "algorithmic_bytes": alg_bytes, "avg_launch_ms": k_ms,
                     "device_copy_gbs": copy_gbs},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def bench_d18(args):
    """D18 multi-document read at a decode step of a Qwen3.5-shaped reader layer: one reader row,
    6 document operators of 2048 rows each (bf16, Hkv = 2, hd = 256), 16 query heads (G = 8), 512
    own rows before it; soft routing over the documents (skip 16).  One step = one xenc_d18_read
    call (partials over (kv head, document | own rows, key split), then the merge + routing).
    Algorithmic bytes: every operator row's K and V once per kv head, the own rows' K and V (fp32),
    the rotated queries and the outputs."""
    from kv_skill_v2_amd import ops
    from kv_skill_v2_amd._lib import lib, ptr, stream_handle

    dev = torch.device("cuda:0")
    D, N, hkv, G, hd, P, T, skip = 6, 2048, 2, 8, 256, 512, 1, 16
    hq = hkv * G
    g = torch.Generator(device=dev)
    g.manual_seed(18)
    docs = [(torch.randn(hkv, N, hd, generator=g, device=dev).bfloat16(),
             torch.randn(hkv, N, hd, generator=g, device=dev).bfloat16()) for _ in range(D)]
    pk = ops.d18_pack(docs)
    qd = torch.randn(D, T, hq, hd, generator=g, device=dev)
    qo = torch.randn(T, hq, hd, generator=g, device=dev)
    ko = torch.randn(hkv, P + T, hd, generator=g, device=dev)
    vo = torch.randn(hkv, P + T, hd, generator=g, device=dev)
    S = ops.d18_nsplit(T, hkv, pk.lengths, P + T) if args.nsplit is None else args.nsplit
    out = torch.empty(T, hq, hd, device=dev)
    w = torch.empty(hkv, G, T, D, device=dev)
    r, rmax = torch.empty_like(w), torch.empty_like(w)
    ws = torch.empty(int(lib().xenc_d18_workspace_bytes(T, hq, D, hd, S)), dtype=torch.uint8, device=dev)
    st = stream_handle(dev)
    scale = hd ** -0.5

    def call():
        rc = lib().xenc_d18_read(1, T, hq, hkv, hd, D, ptr(qd), ptr(qo), ptr(pk.K), ptr(pk.V), pk.K.stride(0),
                                 pk.K.stride(1), ptr(pk.doc_ptr), ptr(ko), ptr(vo), ko.stride(0), ko.stride(1), P,
                                 scale, skip, 1.0, 0, -1, None, S, ptr(out), ptr(w), ptr(r), ptr(rmax),
                                 ptr(ws), ws.numel(), stream_handle(dev))
        if rc:
            raise RuntimeError(f"xenc_d18_read failed: {rc}")

    alg_bytes = (D * N * hkv * hd * 2 * 2 + (P + T) * hkv * hd * 2 * 4 + (D + 1) * T * hq * hd * 4
                 + T * hq * hd * 4 + 3 * hkv * G * T * D * 4)
    settle_calls = settle(call)
    for _ in range(args.warmup):
        call()
    stream = torch.cuda.current_stream(dev)
    ms_eager, k_ms_eager = timed_steps(call, args.steps, stream)
    # The call (two launches) captured once in a HIP graph and replayed: every replay's output
    # checked against the eager one.  The faster of the two ways is reported (named in config).
    gt = {"ms": None, "span_ms": None, "ms_in_graph": None, "span_ms_in_graph": None}
    if not args.no_graph:
        ref = (out.clone(), w.clone())
        gt = graph_timings(lambda: (call(), out)[1], lambda _: torch.equal(out, ref[0]) and torch.equal(w, ref[1]),
                           args.steps, dev)
        if not torch.equal(out, ref[0]):
            gt = {k: None for k in gt}
    ms_graph = gt["ms"]
    timing, ms_step, k_ms = fastest_timing(ms_eager, k_ms_eager, gt)
    achieved = alg_bytes / (k_ms * 1e-3) / 1e9
    cpu = None
    if args.cpu_sample > 0:
        import oracle as O
        torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
        qd_c = qd.cpu().permute(0, 2, 1, 3).reshape(D, hkv, G, T, hd)
        qo_c = qo.cpu().permute(1, 0, 2).reshape(hkv, G, T, hd)
        docs_c = [(K.cpu().float(), V.cpu().float()) for K, V in docs]
        ko_c, vo_c = ko.cpu(), vo.cpu()
        O.d18_core(qd_c, qo_c, docs_c, ko_c, vo_c, P, scale, skip)          # warm-up
        ts = []
        for _ in range(max(1, args.cpu_reps)):
            t1 = time.perf_counter()
            O.d18_core(qd_c, qo_c, docs_c, ko_c, vo_c, P, scale, skip)
            ts.append(time.perf_counter() - t1)
        cpu_s = statistics.median(ts)
        cpu = {"value": 1.0 / cpu_s, "unit": "reader rows/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": (f"the same call: the reference's per-document loop (xenc/d18_library.py:63-90) in "
                          f"fp32 on the CPU oracle, median of {max(1, args.cpu_reps)} reps after 1 warm-up; "
                          f"{cpu_model()}")}
    res = {
        "metric": "D18 multi-document read: reader rows/s and HBM GB/s (% peak)",
        "value": T / (ms_step * 1e-3), "unit": "reader rows/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32 (bf16 operators)", "data": "synthetic",
        "config": {"workload": "d18", "settle_calls": settle_calls, "documents": D, "rows_per_document": N,
                   "hkv": hkv, "hq": hq,
                   "head_dim": hd, "own_rows": P, "reader_rows": T, "skip": skip, "key_splits": S,
                   "timing": timing, "ms_per_call_eager": ms_eager, "ms_per_call_graph": ms_graph,
                   "ms_per_call_in_16_call_graph": gt["ms_in_graph"]},
        "roofline": {"bound": "hbm", "kernel": "d18_partials_kernel + d18_merge_kernel", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "algorithmic_bytes": alg_bytes, "avg_launch_ms": k_ms},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


def bench_op_b(args):
    """Op B, the vLLM plugin's decode read (DecodeReader, xenc/d23_read_kernels.py:134-160), at the
    serving shape of the reference's batch benchmark (xenc's scripts/bench_d23_vllm.py: Qwen3.5-9B
    reader, batches up to 32, documents of 16k tokens): 32 decode rows (--rows; 1 is the
    reference's batch-1 latency case), each over its own
    16,384-row document operator joined with 64 own rows; hq 16, hkv 4, head dim 256, bf16 pools of
    16-row blocks, block tables a seeded shuffle of the pools.  One step = one DecodeReader call (a
    single xenc_paged_decode_joint launch).  Algorithmic bytes: every routed K and V row once
    (rows x hkv x d x 2 B x 2), plus q and the fp32 outputs."""
    from kv_skill_v2_amd.decode_reader import DecodeReader

    dev = torch.device("cuda:0")
    B, hq, hkv, d, bs, op_len, own_len = max(1, args.rows), 16, 4, 256, 16, 16384, 64
    dt = torch.bfloat16
    g = torch.Generator(device=dev)
    g.manual_seed(23)
    nb_op, nb_own = B * op_len // bs, B * own_len // bs
    op_k = torch.randn(nb_op, bs, hkv, d, generator=g, device=dev).to(dt)
    op_v = torch.randn(nb_op, bs, hkv, d, generator=g, device=dev).to(dt)
    own_k = torch.randn(nb_own, bs, hkv, d, generator=g, device=dev).to(dt)
    own_v = torch.randn(nb_own, bs, hkv, d, generator=g, device=dev).to(dt)
    gc = torch.Generator().manual_seed(4)
    op_bt = torch.randperm(nb_op, generator=gc).to(torch.int32).view(B, op_len // bs).to(dev)
    own_bt = torch.randperm(nb_own, generator=gc).to(torch.int32).view(B, own_len // bs).to(dev)
    op_l = torch.full((B,), op_len, dtype=torch.int32, device=dev)
    own_l = torch.full((B,), own_len, dtype=torch.int32, device=dev)
    q = torch.randn(B, hq, d, generator=g, device=dev).to(dt)
    scale = d ** -0.5
    dec = DecodeReader(B, hq, hkv, d, max_keys=op_len + own_len, device=dev, chunk=None)
    chunk = dec.chunk

    def call():
        return dec(q, op_k, op_v, op_bt, op_l, own_k, own_v, own_bt, own_l, scale)

    alg_bytes = B * (op_len + own_len) * hkv * d * 2 * 2 + B * hq * d * (2 + 4)
    settle_calls = settle(call)
    for _ in range(args.warmup):
        call()
    stream = torch.cuda.current_stream(dev)
    ms_step, k_ms = timed_steps(call, args.steps, stream)
    achieved = alg_bytes / (k_ms * 1e-3) / 1e9
    cpu = None
    if args.cpu_sample > 0:
        import oracle as O
        torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
        rows = min(B, max(1, args.cpu_sample // 4))
        need_op = op_bt[:rows].cpu().long()
        need_own = own_bt[:rows].cpu().long()
        # Only the blocks of the sampled rows go to the host, renumbered in table order.
        a_op = (op_k[need_op.flatten()].cpu(), op_v[need_op.flatten()].cpu())
        a_own = (own_k[need_own.flatten()].cpu(), own_v[need_own.flatten()].cpu())
        bt_op = torch.arange(need_op.numel(), dtype=torch.int32).view(rows, -1)
        bt_own = torch.arange(need_own.numel(), dtype=torch.int32).view(rows, -1)
        qc, lo_c, lw_c = q[:rows].cpu(), op_l[:rows].cpu(), own_l[:rows].cpu()

        def cpu_call():
            O.decode_read_ref(qc, a_op[0], a_op[1], bt_op, lo_c, a_own[0], a_own[1], bt_own, lw_c, scale)

        cpu_call()
        ts = []
        for _ in range(max(1, args.cpu_reps)):
            t1 = time.perf_counter()
            cpu_call()
            ts.append(time.perf_counter() - t1)
        cpu_s = statistics.median(ts)
        cpu = {"value": rows / cpu_s, "unit": "decode rows/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": (f"{rows} of the {B} rows: the reference's pure-torch decode read "
                          f"(xenc/d23_read_kernels.py:31-47) in fp32 on the CPU oracle, median of "
                          f"{max(1, args.cpu_reps)} reps after 1 warm-up; {cpu_model()}")}
    res = {
        "metric": "Op B decode read (DecodeReader): decode rows/s and HBM GB/s (% peak)",
        "value": B / (ms_step * 1e-3), "unit": "decode rows/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32 (bf16 pools)", "data": "synthetic",
        "config": {"workload": "op_b", "rows": B, "operator_rows": op_len, "own_rows": own_len, "hq": hq,
                   "hkv": hkv, "head_dim": d, "block_size": bs, "key_splits": dec.S, "chunk": chunk,
                   "settle_calls": settle_calls},
        "roofline": {"bound": "hbm", "kernel": "joint_read_mfma_kernel + joint_merge_kernel", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "algorithmic_bytes": alg_bytes, "avg_launch_ms": k_ms},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the "
              "multi-GPU sharding of the read is designed but not built", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    fn = {"prefill": bench_prefill, "op_b": bench_op_b, "multi_depth": bench_multi_depth,
          "pool_build": bench_pool_build, "d18": bench_d18}.get(args.workload, bench_decode)
    fn(args)
    if args.calibration_copy_mib > 0:
        calibration_copy(torch.device("cuda:0"), args.calibration_copy_mib)


def calibration_copy(dev, mib: int):
    """Three device-to-device copies of `mib` MiB after the workload: the blit kernel
    (`__amd_rocclr_copyBuffer`) reads and writes a known byte count, which scales the rocprofv3
    FETCH_SIZE / WRITE_SIZE readings of the workload's kernels in the same run."""
    n = mib * (1 << 20) // 2
    src = torch.ones(n, dtype=torch.float16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def bench_decode(args):
    """Batched (or single-sequence) paged decode step: route over every chunk of each sequence's
    Library, top-k, the paged split-K read of the routed pages and the LSE merge."""
    from kv_skill_v2_amd import ops, synth

    dev = torch.device("cuda:0")
    P, q, qg, top_k = synth.decode_workload(args.workload, device=dev)
    lib = ops.PagedLibrary(P.pages, P.chunk_page, P.chunk_nvalid, P.chunk_ptr, P.S,
                           n_chunks=P.n_chunks, nvalid=P.nvalid)
    B, d = q.shape
    read_temp, route_temp = 12.0, 10.0

    def step():
        return ops.route_read_decode(q, lib, qg, top_k=top_k, route_temp=route_temp, read_temp=read_temp,
                                     nsplit=args.nsplit)[3]

    # Algorithmic bytes of the read: each routed page's valid slot rows once (K = V tied), the
    # query rows and the output rows.  Routing is deterministic, so read it once off the clock.
    _, idx0, wsel0 = ops.route_topk(q, lib, qg, top_k=top_k, route_temp=route_temp)
    idx_h = idx0.cpu()
    nv_h = P.nvalid
    ptr_h = P.chunk_ptr.cpu().tolist()
    routed_slots = sum(nv_h[ptr_h[b] + c] for b in range(B) for c in idx_h[b].tolist() if c >= 0)
    read_bytes = routed_slots * d * 2 + 2 * B * d * 4
    route_bytes = sum(P.n_chunks) * d * 4 + B * d * 4

    settle_calls = settle(step)
    for _ in range(args.warmup):
        step()
    stream = torch.cuda.current_stream(dev)
    # Eager steps: the q . S dots, the read kernel with the top-k in its prologue and the merge,
    # K steps back to back.  The roofline figure counts the step's algorithmic bytes (routed
    # pages, S, q and r) over the GPU span per step of the timed region.
    host = []
    ms_eager, span_eager = timed_steps(step, args.steps, stream, host)

    # The step captured once in a HIP graph and replayed.  Every replay is checked bit for bit
    # against the eager result, with eager work and a synchronisation in between; on any
    # mismatch the eager time is reported.
    gt = {"ms": None, "span_ms": None, "ms_in_graph": None, "span_ms_in_graph": None}
    if not args.no_graph:
        ref_out = step().clone()
        gt = graph_timings(step, lambda o: torch.equal(o, ref_out), args.steps, dev)
    ms_graph = gt["ms"]
    # The step runs every way; report the fastest measured one (named in config).
    timing, ms_step, span = fastest_timing(ms_eager, span_eager, gt)
    achieved = (read_bytes + route_bytes) / (span * 1e-3) / 1e9

    traffic = traffic_from_profile(args.workload)
    stream_meas = measured_stream_peak(dev)

    cpu = None
    if args.cpu_sample > 0:
        cpu = cpu_baseline(P, q, top_k, args.cpu_sample, args.cpu_reps)

    out = {
        "metric": METRIC,
        "value": B / (ms_step * 1e-3),
        "unit": "query tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": args.workload, "sequences": B, "d_s": d,
                   "chunks_per_library": f"U{{8..64}} (total {sum(P.n_chunks)})" if B > 1 else str(P.n_chunks[0]),
                   "slots_per_page": P.pages.shape[1], "top_k": top_k, "read_temp": read_temp,
                   "route_temp": route_temp, "accumulate": "fp32", "page_table": "seeded shuffle",
                   "settle_calls": settle_calls,
                   "nsplit": args.nsplit or ops.default_nsplit(B * idx_h.shape[1], P.pages.shape[1]),
                   "timing": timing, "ms_per_step_eager": ms_eager, "ms_per_step_graph": ms_graph,
                   "ms_per_step_in_16_step_graph": gt["ms_in_graph"],
                   "host_issue_us_per_step": host[0] * 1e3},
        "roofline": {"bound": "hbm",
                     "kernel": "route_dots_kernel + decode_read_kernel (top-k in its prologue) + merge_kernel",
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": traffic["bytes_per_launch"] if traffic else None,
                     "traffic_source": traffic["source"] if traffic else None,
                     "algorithmic_bytes": read_bytes + route_bytes, "avg_launch_ms": span,
                     "routed_slots": routed_slots, "read_bytes": read_bytes, "route_bytes": route_bytes,
                     "measured_peak": stream_meas, "frac_of_measured": achieved / stream_meas},
        "cpu_baseline": cpu,
    }
    if args.workload == "batched_paged_decode" and not args.no_prefill:
        # The north star's second target, measured in the same run: the prefill/registration read
        # (4 documents x 2048 rows x 32 x 512 slots, forward and dQ backward) against the fp16
        # MFMA peak.  `metric` and `value` stay the batched decode's.
        out["prefill"] = measure_prefill(args.prefill_steps, 10, min(args.cpu_sample, 1))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
