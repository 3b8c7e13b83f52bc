"""Benchmark: QPS of the IVF-PQ search hot path on one MI355X.

Workload: 1M x 128 fp32 base vectors from a
256-component Gaussian mixture (centres U[-1,1], sigma 0.08, seeded), 1024
inverted lists, PQ M=32 x 256 codewords, 10k queries in one batch, nprobe=32,
k=10.  The index is built in-run by this framework's GPU build path (k-means++
seeding, 20 Lloyd iterations, PQ 15 iterations on a 50k sample); that build is
not timed.

One step = one fgpu_search of the 10k-query batch with queries already in
HBM: coarse quantizer (MFMA GEMM + exact re-score + top-32), then the MFMA
screen (bf16 distance bounds: a threshold per query from its first list, then
every probed list whose bound can reach it) and the exact rescore of the
candidates with the reference's LUT arithmetic, top-10; queries the screen
hands over run the LUT + ADC scan.  value = 10k / step time.  `stages_ms`
holds HIP events fgpu_search records between its kernels on its own stream.

The roofline entry is for the step's longest kernel, a screen round: achieved
= its algorithmic flops (2 (dim + 16) per (query, vector) pair it screens) over
its event-timed duration, against the dense bf16 MFMA peak; `traffic` is the
copy-calibrated FETCH_SIZE + WRITE_SIZE from profiles/.  `adc_scan` is the
metric's ADC-scan HBM GB/s: the LUT + ADC scan kernel timed on the same probes
with HIP events on its stream, achieved = the code and id bytes of the lists
it reads (its own load count); its exact list bound skips most probed lists,
so the work-equivalent figure (the code bytes of every probed list, once per
(query, list)) is reported apart as `effective`, and `no_skip` times the same
kernel reading every probed list.  `measured_read_peak_gbs` is a streaming
read of 4 GiB.  `end_to_end` follows the reference's QPS definition (H2D +
search + D2H), on one stream and on two alternating streams.  The line also
carries `graph_coarse`: the same coarse step done the reference's way (a graph
walk over the centroids instead of the exact GEMM; not timed in `value`), with
its time, the share of the exact top-32 lists it finds and how often the
top-10 stays identical.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-queries N] [--workload c2|c3|c4|c5]

--workload c3 prints a supplementary line for BASELINE config 3 instead: 10M x
96 fp32 (1024-component mixture, per-component sigma U[0.05, 0.15]), 4096
lists, PQ M=48, 10k queries, nprobe=64, the two-phase pruned scan (p1_lists 12,
limit_k 50, threshold_coeff 1.0) compacted to the top 1000 candidates, then the
early-stopping exact rerank (mini-batch 128, eps 0.1, beta 2) to k=100.  Its
index is built in-run too (k-means on a 1M-row sample, then every row
assigned), not timed.  Phase 1 of the two-phase scan runs as the MFMA screen
over one single-probe query per (query, phase-1 probe); the line's roofline is
that screen's longer round, measured like config 2's, and `two_phase` holds
the call's stage times and counters.

--workload c4 prints a supplementary line for BASELINE config 4, the index
build: 10M x 128 fp32 (1024-component mixture); k-means++ seeding and 20 Lloyd
iterations of 4096 centroids on a 1M-row sample; assignment of all 10M rows;
PQ M=32 training (15 iterations, 50k sample) and encoding of all rows; and an
elbow sweep over 1024/2048/4096 lists (k-means SSE on the sample, Kneedle
knee).  value = rows built per second over the whole build.

--workload c5 prints a supplementary line for BASELINE config 5: graph search
over 5M x 128 fp32 (256-component mixture) with a fixed out-degree-32 graph,
10k queries, itopk 64, search width 4, at most 64 steps, k=10.  The graph is
built in-run, untimed: each base vector's nearest other vectors by this
framework's IVF-PQ search (2048 lists, M=32, nprobe 8, ADC top-64 reranked
exactly), optionally with seeded random long-range edges.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "QPS at fixed nprobe, 1M×128 IVF-PQ k=10 (1 GPU); ADC-scan HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2500.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "adc_flow_c2_traffic.txt")
TRAFFIC_FILE_C3 = os.path.join(ROOT, "profiles", "two_phase_c3_traffic.txt")
SCREEN_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "screen_c2_traffic.txt")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def read_traffic(path=TRAFFIC_FILE, key="traffic_bytes_per_launch"):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, copy-calibrated)."""
    try:
        for line in open(path):
            if line.startswith(key + ":"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def timed_ms(torch, stream, reps, fn):
    """Average time of fn() over reps launches, from HIP events recorded on the stream the work runs on."""
    fn()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def stream_read_peak(torch, fg, dev, gib=4, reps=10):
    """Measured HBM read rate: 16-byte streaming loads over a buffer far larger than the MALL."""
    a = torch.empty(gib << 30, dtype=torch.uint8, device=dev)
    ms = timed_ms(torch, torch.cuda.current_stream(), reps, lambda: fg.stream_read(a))
    del a
    return (gib << 30) / (ms * 1e-3) / 1e9


def row_gather_peak(torch, fg, rows, nreads, lanes_per_row=8, reps=5, seed=5):
    """Measured random-row read rate over a 2-D device tensor: nreads whole rows at seeded random ids, eight lanes a
    row (the rerank's and graph search's pattern) or one lane a row, all loads in flight."""
    g = torch.Generator(device=rows.device)
    g.manual_seed(seed)
    idx = torch.randint(0, rows.shape[0], (nreads,), generator=g, device=rows.device, dtype=torch.int32)
    ms = timed_ms(torch, torch.cuda.current_stream(), reps, lambda: fg.row_gather(rows, idx, lanes_per_row))
    return nreads * rows.shape[1] * rows.element_size() / (ms * 1e-3) / 1e9


def cpu_timed(fn, warm, runs=3):
    """Median wall time of `runs` calls of fn after one warm-up call of warm; returns (seconds, last result)."""
    warm()
    ts, r = [], None
    for _ in range(runs):
        t0 = time.perf_counter()
        r = fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), r


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-queries", type=int, default=10000, help="query sample for the CPU baseline (0 = skip)")
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--nq", type=int, default=10_000)
    ap.add_argument("--copy-probe", action="store_true", help="also run a 1 GiB device copy (PMC calibration)")
    ap.add_argument("--workload", choices=["c1", "c2", "c3", "c4", "c5", "batch128"], default="c2")
    ap.add_argument("--c5-components", type=int, default=256, help="mixture components of the C5 data")
    ap.add_argument("--c5-random-edges", type=int, default=8,
                    help="C5: out-edges per vector replaced by seeded random long-range edges")
    ap.add_argument("--c5-no-reverse", action="store_true", help="C5: forward kNN edges only (no reverse edges)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is not supported "
              "(the search shards by queries, with no exchange between GPUs)", file=sys.stderr)
        sys.exit(2)

    import torch

    import fusiongpu_amd as fg

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload == "c1":
        return run_c1(args, torch, fg, dev)
    if args.workload == "c3":
        return run_c3(args, torch, fg, dev)
    if args.workload == "c5":
        return run_c5(args, torch, fg, dev)
    if args.workload == "c4":
        return run_c4(args, torch, fg, dev)
    if args.workload == "batch128":
        return run_batch128(args, torch, fg, dev)
    dim, nlist, m, nprobe, k = 128, 1024, 32, 32, 10
    t0 = time.time()
    x = fg.gen_gmm(args.n, dim, 256, seed=2024, set=0, sig_lo=0.08)
    q = fg.gen_gmm(args.nq, dim, 256, seed=2024, set=1, sig_lo=0.08)
    log(f"generated {args.n}x{dim} base + {args.nq} queries in {time.time() - t0:.1f}s")
    t0 = time.time()
    dx = torch.from_numpy(x).to(dev)
    offs, ids, codes, cent, cb = fg.build_ivfpq(dx, nlist, m, kmeans_iters=20, init_mode=1, seed=42, pq_iters=15,
                                                sample_size=50000)
    del dx
    log(f"index built on GPU in {time.time() - t0:.1f}s (max list {np.diff(offs).max()}, "
        f"empty lists {(np.diff(offs) == 0).sum()})")
    idx = fg.Index.from_arrays(dim, m, offs, ids, codes, cent, cb)
    dq = torch.from_numpy(q).to(dev)
    ws = torch.empty(idx.search_workspace_bytes(args.nq, nprobe), dtype=torch.uint8, device=dev)
    out = (torch.empty((args.nq, k), dtype=torch.int32, device=dev),
           torch.empty((args.nq, k), dtype=torch.float32, device=dev))
    stream = torch.cuda.current_stream()

    # ---- whole-path timing (the metric): fgpu_search = coarse step, MFMA screen, exact rescore
    for _ in range(args.warmup):
        idx.search(dq, nprobe, k, workspace=ws, out=out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        idx.search(dq, nprobe, k, workspace=ws, out=out)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = 1e3 * wall / args.steps
    qps = args.nq / (wall / args.steps)
    log(f"search: {ms_per_step:.3f} ms/step, {qps:,.0f} QPS (screen path: {idx.screen_ready})")

    # ---- per-stage times: HIP events fgpu_search records on its own stream between its kernels
    reps = max(args.steps, 5)
    idx.set_option(fg.Index.OPT_STAGE_EVENTS, 1)
    stage_ms = {kk: 0.0 for kk in fg.Index.STAGES}
    for _ in range(reps):
        idx.search(dq, nprobe, k, workspace=ws, out=out)
        for kk, v in idx.search_stage_times().items():
            stage_ms[kk] += v / reps
    idx.set_option(fg.Index.OPT_STAGE_EVENTS, 0)
    sst = idx.search_screen_stats(args.nq, nprobe, ws)
    log("stages (ms): " + ", ".join(f"{kk} {v:.4f}" for kk, v in stage_ms.items()))
    log(f"screen: {sst['pairs_round2']} (query, list) pairs in round 2 over {sst['lists_round2']} lists, "
        f"{sst['candidates'] / args.nq:.1f} candidates a query (max {sst['max_candidates']}), "
        f"{sst['queries_to_lut_kernel']} queries to the LUT kernel")
    # The roofline kernel: the larger screen round (both are screen_kernel<128,32,round>).  Its
    # algorithmic work is the bound GEMM, 2 (dim + 16) flops per (query, vector) pair screened; the
    # MFMA tiles it runs pad each list's queries to 32 rows.
    rnd = 2 if stage_ms["screen_round2"] >= stage_ms["screen_round1"] else 1
    scr_ms = stage_ms[f"screen_round{rnd}"]
    scr_flop = 2.0 * (dim + 16) * sst[f"vector_pairs_round{rnd}"]
    scr_exec_flop = 2.0 * (dim + 16) * 32 * 32 * sst[f"tiles_round{rnd}"]
    scr_bytes = sst[f"tiles_round{rnd}"] * 32 * (m + 16)  # codes + 16-byte extra block of each vector row read
    scr_tflops = scr_flop / (scr_ms * 1e-3) / 1e12
    log(f"screen round {rnd}: {scr_ms:.4f} ms, {scr_flop / 1e9:.2f} GFLOP algorithmic ({scr_tflops:.1f} TFLOP/s), "
        f"{scr_exec_flop / 1e9:.2f} GFLOP in MFMA tiles, {scr_bytes / 1e6:.1f} MB of codes + blocks read")

    # ---- the LUT scan (the fallback kernel; what fgpu_adc_search runs), timed on its own
    probes, pd = idx.coarse_search(dq, nprobe)
    cnt, _ = fg.probe_counts(idx, probes)
    n_probed_vecs = int(cnt.to(torch.int64).sum().item())
    adc_bytes = n_probed_vecs * m  # code bytes of every probed list, once per (query, list)
    pruned = int((probes == -1).sum().item())
    coarse_ms = timed_ms(torch, stream, reps, lambda: idx.coarse_search(dq, nprobe, workspace=ws))
    lut_out = (torch.empty_like(out[0]), torch.empty_like(out[1]))
    adc_ms = timed_ms(torch, stream, reps, lambda: idx.adc_search(dq, probes, k, out=lut_out, probe_dists=pd))
    assert torch.equal(lut_out[0], out[0]) and torch.equal(lut_out[1], out[1]), "LUT scan and screen path differ"
    gemm_flop = 2.0 * args.nq * nlist * dim
    log(f"coarse {coarse_ms:.3f} ms ({gemm_flop / coarse_ms / 1e9:.1f} TFLOP/s incl. select), LUT scan "
        f"{adc_ms:.3f} ms; {pruned} of {args.nq * nprobe} probes pruned (prune_ratio 100)")
    # What the LUT scan moves: the codes and ids of the lists it does not skip.
    sid, sd, st = idx.adc_search_stats(dq, probes, k, probe_dists=pd)
    assert torch.equal(sid, out[0]) and torch.equal(sd, out[1]), "instrumented scan differs"
    loaded_bytes = st["vectors_loaded"] * (m + 4)  # code bytes + the 4-byte vector id loaded with them
    loaded_gbs = loaded_bytes / (adc_ms * 1e-3) / 1e9
    eff_gbs = adc_bytes / (adc_ms * 1e-3) / 1e9
    log("LUT scan clocks per query: " + ", ".join(f"{kk} {st[kk] / args.nq:.0f}" for kk in
                                                     ("clk_setup", "clk_builder", "clk_scanner", "clk_total")))
    log(f"LUT scan moves {st['vectors_loaded'] * m / 1e9:.2f} GB of codes (+ids {st['vectors_loaded'] * 4 / 1e9:.2f}"
        f" GB) = {loaded_gbs:.0f} GB/s; LUTs built {st['luts_built']}, probed lists skipped {st['lists_skipped']} "
        f"of {int((probes != -1).sum().item())}; every probed list once would be {adc_bytes / 1e9:.2f} GB "
        f"({eff_gbs:.0f} GB/s work-equivalent)")
    # The same scan with the list bound off: it reads every probed list.
    idx.set_option(fg.Index.OPT_LIST_SKIP, 0)
    nid, nd = idx.adc_search(dq, probes, k, probe_dists=pd)
    ns_ms = timed_ms(torch, stream, reps, lambda: idx.adc_search(dq, probes, k, out=lut_out, probe_dists=pd))
    idx.set_option(fg.Index.OPT_LIST_SKIP, 1)
    assert torch.equal(nid, sid) and torch.equal(nd, sd), "the scan without list skipping differs"
    ns_bytes = n_probed_vecs * (m + 4)
    ns_gbs = ns_bytes / (ns_ms * 1e-3) / 1e9
    log(f"LUT scan without list skipping: {ns_ms:.3f} ms, {ns_bytes / 1e9:.2f} GB (codes + ids of every probed "
        f"list) = {ns_gbs:.0f} GB/s; ids identical")
    assert idx.faults() == 0, "a bounded wait of the scan gave up"
    peak_gbs = stream_read_peak(torch, fg, dev)
    log(f"measured stream-read rate: {peak_gbs:.0f} GB/s (16-byte loads over 4 GiB)")

    # ---- end to end, the reference's QPS definition (search_pipeline.cu:621-636): queries
    # from pinned host memory, search, results back to pinned host memory, all steps enqueued.
    # Serial: every step on one stream.  Two streams: steps alternate between two streams, each
    # with its own buffers, so one step's copies can run beside the other's search (the
    # reference's multi-stream pipeline, search_pipeline.cu:168-214, 311-377).
    def e2e_bufs():
        b = {"hq": torch.empty((args.nq, dim), dtype=torch.float32, pin_memory=True),
             "hid": torch.empty((args.nq, k), dtype=torch.int32, pin_memory=True),
             "hdd": torch.empty((args.nq, k), dtype=torch.float32, pin_memory=True),
             "dq": torch.empty_like(dq), "ws": torch.empty_like(ws),
             "out": (torch.empty_like(out[0]), torch.empty_like(out[1]))}
        b["hq"].copy_(torch.from_numpy(q))
        return b

    def e2e_step(b, ev=None):
        if ev:
            ev[0].record()
        b["dq"].copy_(b["hq"], non_blocking=True)
        if ev:
            ev[1].record()
        idx.search(b["dq"], nprobe, k, workspace=b["ws"], out=b["out"])
        if ev:
            ev[2].record()
        b["hid"].copy_(b["out"][0], non_blocking=True)
        b["hdd"].copy_(b["out"][1], non_blocking=True)
        if ev:
            ev[3].record()

    bufs = [e2e_bufs(), e2e_bufs()]
    for _ in range(2):
        e2e_step(bufs[0])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        e2e_step(bufs[0])
    torch.cuda.synchronize()
    e2e_ms = 1e3 * (time.perf_counter() - t0) / args.steps
    assert torch.equal(bufs[0]["hid"], out[0].cpu()), "end-to-end results differ"
    # where a serial step's time goes: events on its stream around the copies and the search
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    part = [0.0, 0.0, 0.0]
    for _ in range(reps):
        e2e_step(bufs[0], evs)
        evs[3].synchronize()
        for t in range(3):
            part[t] += evs[t].elapsed_time(evs[t + 1]) / reps
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        with torch.cuda.stream(streams[i % 2]):
            e2e_step(bufs[i % 2])
    torch.cuda.synchronize()
    e2e2_ms = 1e3 * (time.perf_counter() - t0) / args.steps
    for b in bufs:
        assert torch.equal(b["hid"], out[0].cpu()) and torch.equal(b["hdd"], out[1].cpu()), \
            "end-to-end results differ"
    h2d_gbs = args.nq * dim * 4 / (part[0] * 1e-3) / 1e9
    log(f"end to end (H2D queries + search + D2H results): {e2e_ms:.3f} ms/step serial "
        f"(H2D {part[0]:.4f} ms = {h2d_gbs:.1f} GB/s, search {part[1]:.4f}, D2H {part[2]:.4f}); "
        f"{e2e2_ms:.3f} ms/step on two streams, {args.nq / e2e2_ms * 1e3:,.0f} QPS")

    # ---- the graph coarse mode (the reference's CAGRA-over-centroids step): time and
    # how many of the exact top-nprobe lists it finds, and the end-to-end top-10 it gives;
    # the reference's graph degree (8) and a denser graph (32), its search parameters
    graph_coarse = []
    ep = probes.cpu().numpy().view(np.uint32)
    for degree in (8, 32):
        t0 = time.perf_counter()
        cgraph = idx.coarse_graph_build(degree)
        torch.cuda.synchronize()
        graph_build_ms = 1e3 * (time.perf_counter() - t0)
        gprobes, _ = idx.coarse_graph_search(dq, nprobe, cgraph)
        graph_ms = timed_ms(torch, stream, reps, lambda: idx.coarse_graph_search(dq, nprobe, cgraph))
        gp = gprobes.cpu().numpy().view(np.uint32)
        probe_recall = float(np.mean([len(set(a_) & set(b_)) / nprobe for a_, b_ in zip(gp, ep)]))
        gids, _ = idx.adc_search(dq, gprobes, k)
        same_topk = float((gids == out[0]).all(dim=1).float().mean().item())
        graph_coarse.append({"degree": degree, "itopk": 32, "width": 4, "max_iter": 200,
                             "coarse_ms": round(graph_ms, 4), "graph_build_ms": round(graph_build_ms, 2),
                             "probe_recall_vs_exact": round(probe_recall, 4),
                             "queries_with_identical_top10": round(same_topk, 4)})
        log(f"graph coarse mode, degree {degree}: {graph_ms:.3f} ms (build {graph_build_ms:.1f} ms), finds "
            f"{probe_recall:.4f} of the exact top-{nprobe} lists; top-10 identical for {same_topk:.4f} of the queries")

    if args.copy_probe:
        a = torch.empty(1 << 28, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        log("copy probe: 1 GiB device-to-device copy done")

    gid = out[0].cpu().numpy()
    gd = out[1].cpu().numpy()

    # ---- CPU baseline: the oracle (C++/OpenMP restatement of the same search) on the same index
    cpu = None
    parity = None
    if args.cpu_queries > 0:
        import oracle
        ns = min(args.cpu_queries, args.nq)

        def cpu_search(qq):
            op, _ = oracle.coarse(qq, cent, nprobe)
            return oracle.search_plain(qq, cent, cb, offs, ids, codes, op, k)

        cpu_s, (oid, od) = cpu_timed(lambda: cpu_search(q[:ns]), warm=lambda: cpu_search(q[:min(ns, 500)]))
        threads = oracle.lib.orc_max_threads()
        cpu = {"value": round(ns / cpu_s, 1), "unit": "queries/s", "cores": threads, "kind": "port",
               "cpu_model": cpu_model(),
               "sample": f"first {ns} of the 10k queries, same index: coarse + LUT/ADC + top-10 (the oracle's "
                         f"exhaustive scan); median of 3 runs after a warm-up, {cpu_s:.2f}s each, "
                         f"{threads} OpenMP threads"}
        parity = {"queries": ns, "ids_equal": bool(np.array_equal(gid[:ns], oid)),
                  "dists_bit_equal": bool(np.array_equal(gd[:ns].view(np.uint32), od.view(np.uint32)))}
        log(f"cpu baseline {cpu['value']} QPS on {threads} threads ({cpu['cpu_model']}); parity {parity}")

    traffic = read_traffic()
    res = {
        "metric": METRIC,
        "value": round(qps, 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded Gaussian mixture; index built in-run by this framework's GPU build path",
        "config": {"workload": "BASELINE config 2: 1M x 128 fp32, 1024 lists, PQ M=32 x 256 (8-bit), "
                               "10k queries in one batch, nprobe=32, k=10",
                   "n": args.n, "dim": dim, "nlist": nlist, "pq_m": m, "nq": args.nq, "nprobe": nprobe, "k": k,
                   "prune_ratio": 100.0, "probes_pruned": pruned, "probes_total": args.nq * nprobe},
        "roofline": {"bound": "mfma", "kernel": f"screen_kernel<128,32,{rnd}> (screen round {rnd})",
                     "achieved": round(scr_tflops, 2), "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(scr_tflops / BF16_MFMA_PEAK_TFLOPS, 4),
                     "traffic": read_traffic(SCREEN_TRAFFIC_FILE, f"traffic_bytes_per_launch_round{rnd}"),
                     "avg_launch_ms": round(scr_ms, 4), "flop_per_launch": scr_flop,
                     "mfma_tile_flop_per_launch": scr_exec_flop,
                     "mfma_tile_frac": round(scr_exec_flop / (scr_ms * 1e-3) / 1e12 / BF16_MFMA_PEAK_TFLOPS, 4),
                     "bytes_read_per_launch": scr_bytes,
                     "hbm_gbs": round(scr_bytes / (scr_ms * 1e-3) / 1e9, 1),
                     "note": "the step's longest kernel: bf16 MFMA distance bounds of (query, vector) pairs; "
                             "achieved = 2 (dim + 16) flops per pair screened (the bound GEMM, K = dim plus a "
                             "16-wide block of constants) / its event-timed duration, against the dense bf16 "
                             "peak; mfma_tile_frac counts the 32 x 32 tiles it runs (a list's queries padded to "
                             "32 rows); bytes_read = codes + 16-byte block of each vector row a tile reads; "
                             "traffic = copy-calibrated FETCH_SIZE + WRITE_SIZE per launch "
                             "(profiles/screen_c2_traffic.txt)"},
        "adc_scan": {"bound": "hbm", "kernel": "adc_flow_kernel<128,32>", "achieved": round(loaded_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(loaded_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "bytes_per_launch": loaded_bytes, "avg_launch_ms": round(adc_ms, 4),
                     "note": "the LUT + ADC scan (fgpu_adc_search; fgpu_search's kernel for the queries the "
                             "screen hands over, and its whole scan with the screen off), timed on the same "
                             "probes; achieved = codes + ids of the lists the scan reads (its own load count "
                             "in this run) / kernel time; traffic = copy-calibrated FETCH_SIZE + WRITE_SIZE per "
                             "launch (profiles/adc_flow_c2_traffic.txt)",
                     "traffic_rate_gbs": round(traffic / (adc_ms * 1e-3) / 1e9, 1) if traffic else None,
                     "measured_read_peak_gbs": round(peak_gbs, 1),
                     "frac_of_measured_peak": round(loaded_gbs / peak_gbs, 4),
                     "effective": {"bytes_per_launch": adc_bytes, "gbs": round(eff_gbs, 1),
                                   "lists_skipped": st["lists_skipped"], "luts_built": st["luts_built"],
                                   "note": "work-equivalent rate: code bytes of every probed list once per (query, "
                                           "list) over the kernel time; the exact list bound skips lists that "
                                           "cannot reach the top-10, so this exceeds the HBM peak"},
                     "no_skip": {"avg_launch_ms": round(ns_ms, 4), "bytes_per_launch": ns_bytes,
                                 "achieved": round(ns_gbs, 1), "frac": round(ns_gbs / HBM_PEAK_GBS, 4),
                                 "ids_identical": True,
                                 "traffic": read_traffic(TRAFFIC_FILE, "traffic_bytes_per_launch_no_skip"),
                                 "note": "the same kernel with the list bound off: it reads the codes and ids of "
                                         "every probed list (32 MB of codes, so mostly from the MALL)"},
                     "clocks_per_query": {kk: round(st[kk] / args.nq) for kk in
                                          ("clk_setup", "clk_builder", "clk_scanner", "clk_total")}},
        "lut_path_ms": {"coarse": round(coarse_ms, 4), "adc_scan": round(adc_ms, 4),
                        "coarse_tflops_incl_select": round(gemm_flop / coarse_ms / 1e9, 2)},
        "stages_ms": dict({kk: round(v, 4) for kk, v in stage_ms.items()},
                          note="HIP events fgpu_search records on its stream between its stages "
                               "(FGPU_OPT_STAGE_EVENTS), averaged over the stage-timing launches; screen_pairs1 "
                               "includes the zeroing kernel"),
        "screen": {kk: sst[kk] for kk in ("pairs_round1", "pairs_round2", "lists_round2", "candidates",
                                          "max_candidates", "queries_to_lut_kernel", "queries_with_threshold",
                                          "vector_pairs_round1", "vector_pairs_round2", "tiles_round1",
                                          "tiles_round2")},
        "end_to_end": {"ms_per_step": round(min(e2e_ms, e2e2_ms), 4),
                       "qps": round(args.nq / min(e2e_ms, e2e2_ms) * 1e3, 1),
                       "serial_ms_per_step": round(e2e_ms, 4), "two_stream_ms_per_step": round(e2e2_ms, 4),
                       "serial_parts_ms": {"h2d": round(part[0], 4), "search": round(part[1], 4),
                                           "d2h": round(part[2], 4)},
                       "h2d_gbs": round(h2d_gbs, 1),
                       "note": "the reference's QPS definition: queries H2D from pinned memory + search + "
                               "results D2H, every step enqueued, one wait at the end; ms_per_step is the faster "
                               "of one stream and two alternating streams; the parts are events around a serial "
                               "step's copies and search"},
        "cpu_baseline": cpu,
        "parity": parity,
        "graph_coarse": graph_coarse,
    }
    print(json.dumps(res), flush=True)


def run_batch128(args, torch, fg, dev):
    """The reference pipeline's per-batch path at its defaults (search_pipeline.cu:562-569: batch 128,
    top_m 20, p1_lists 12, limit_k 50, threshold_coeff 1.0, rerank_m 10000, mini_batch 128, eps 0.1,
    beta 2, k 10) on the C2 data: coarse + two-phase + exact rerank, each stage timed with HIP events
    over repeated launches on one batch, with the small-batch kernels (phase 1 split over workgroups,
    four rerank mini-batches a step) and with them off.  Results are identical either way and checked
    against the oracle on the first batch."""
    dim, nlist, m, k = 128, 1024, 32, 10
    nb, top_m, p1, limit_k, coeff, rm, mb, eps, beta = 128, 20, 12, 50, 1.0, 10000, 128, 0.1, 2
    x = fg.gen_gmm(args.n, dim, 256, seed=2024, set=0, sig_lo=0.08)
    q = fg.gen_gmm(args.nq, dim, 256, seed=2024, set=1, sig_lo=0.08)
    dx = torch.from_numpy(x).to(dev)
    offs, ids, codes, cent, cb = fg.build_ivfpq(dx, nlist, m, kmeans_iters=20, init_mode=1, seed=42, pq_iters=15,
                                                sample_size=50000)
    idx = fg.Index.from_arrays(dim, m, offs, ids, codes, cent, cb)
    dq = torch.from_numpy(q[:nb]).to(dev)
    stream = torch.cuda.current_stream()
    tp_ws = torch.empty(fg.lib.fgpu_two_phase_workspace_bytes(nb, top_m, p1, limit_k, rm), dtype=torch.uint8,
                        device=dev)
    probes, _ = idx.coarse_search(dq, top_m)
    runs = {}
    for label, split, spec in (("small_batch_kernels", 0, 0), ("one_workgroup_a_query", 1, 1)):
        idx.set_option(fg.Index.OPT_TWO_PHASE_SPLIT, split)
        tid, td, tc, _, _ = idx.two_phase_search(dq, probes, p1, limit_k, coeff, rm, workspace=tp_ws)
        fid, fd, fvis = fg.rerank(dq, dx, tid, tc, k, mb, eps, beta, spec=spec)
        t_coarse = timed_ms(torch, stream, 50, lambda: idx.coarse_search(dq, top_m))
        t_tp = timed_ms(torch, stream, 50, lambda: idx.two_phase_search(dq, probes, p1, limit_k, coeff, rm,
                                                                         workspace=tp_ws))
        t_rr = timed_ms(torch, stream, 50, lambda: fg.rerank(dq, dx, tid, tc, k, mb, eps, beta, spec=spec))
        idx.set_option(fg.Index.OPT_TWO_PHASE_SPLIT, 0)
        runs[label] = {"coarse_ms": round(t_coarse, 4), "two_phase_ms": round(t_tp, 4), "rerank_ms": round(t_rr, 4),
                       "batch_ms": round(t_coarse + t_tp + t_rr, 4),
                       "qps": round(nb / (t_coarse + t_tp + t_rr) * 1e3, 1),
                       "ids": fid.cpu().numpy(), "dists": fd.cpu().numpy().view(np.uint32)}
        log(f"batch {nb}, {label}: coarse {t_coarse:.4f} + two-phase {t_tp:.4f} + rerank {t_rr:.4f} ms = "
            f"{runs[label]['batch_ms']:.4f} ms a batch, {runs[label]['qps']:,.0f} QPS (device stages)")
    a, b = runs["small_batch_kernels"], runs["one_workgroup_a_query"]
    same = bool(np.array_equal(a["ids"], b["ids"]) and np.array_equal(a["dists"], b["dists"]))
    parity = None
    if args.cpu_queries > 0:
        import oracle

        oprobes, _ = oracle.coarse(q[:nb], cent, top_m, 100.0)
        otid, _, otcnt, _, _ = oracle.search_two_phase(q[:nb], cent, cb, offs, ids, codes, oprobes, p1, limit_k, coeff,
                                                       rm)
        oid, od, _ = oracle.rerank(q[:nb], x, otid, otcnt, k, mb, eps, beta)
        parity = {"queries": nb, "ids_equal": bool(np.array_equal(a["ids"], oid)),
                  "dists_bit_equal": bool(np.array_equal(a["dists"], np.asarray(od, np.float32).view(np.uint32)))}
    log(f"small-batch kernels give identical results: {same}; parity vs oracle {parity}")
    res = {
        "metric": "device QPS of the reference pipeline's per-batch path at batch 128 (coarse + two-phase + rerank)",
        "value": a["qps"], "unit": "queries/s", "n_gpus": 1, "steps": 50, "warmup": 1,
        "ms_per_step": a["batch_ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic: the C2 mixture; index built in-run by this framework's GPU build path",
        "config": {"workload": "C2 data at the reference pipeline's defaults: batch 128, top_m 20, p1_lists 12, "
                               "limit_k 50, threshold_coeff 1.0, rerank_m 10000, mini_batch 128, eps 0.1, beta 2, k 10",
                   "n": args.n, "dim": dim, "nlist": nlist, "pq_m": m},
        "stages_ms": {kk: {f: v[f] for f in ("coarse_ms", "two_phase_ms", "rerank_ms", "batch_ms", "qps")}
                      for kk, v in runs.items()},
        "identical_with_and_without_small_batch_kernels": same,
        "parity": parity,
    }
    print(json.dumps(res), flush=True)


def run_c1(args, torch, fg, dev):
    """BASELINE config 1, the reference's CPU-runnable case: 100k x 128, 256 lists, PQ M=16, nprobe 16, k=10,
    1000 queries; the whole query set through the oracle's CPU search beside it."""
    from fusiongpu_amd import workloads as W
    cfg = W.C1
    dim, m, nprobe, k, nq = cfg.dim, cfg.pq_m, cfg.nprobe, cfg.k, cfg.nq
    x, q = W.base(cfg), W.queries(cfg)
    t0 = time.time()
    offs, ids, codes, cent, cb = W.build_index(cfg, torch.from_numpy(x).to(dev))
    log(f"C1 index built on GPU in {time.time() - t0:.1f}s (max list {np.diff(offs).max()})")
    idx = fg.Index.from_arrays(dim, m, offs, ids, codes, cent, cb)
    dq = torch.from_numpy(q).to(dev)
    ws = torch.empty(idx.search_workspace_bytes(nq, nprobe), dtype=torch.uint8, device=dev)
    out = (torch.empty((nq, k), dtype=torch.int32, device=dev), torch.empty((nq, k), dtype=torch.float32, device=dev))
    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        idx.search(dq, nprobe, k, workspace=ws, out=out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        idx.search(dq, nprobe, k, workspace=ws, out=out)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = 1e3 * wall / args.steps
    qps = nq / (wall / args.steps)
    probes, pd = idx.coarse_search(dq, nprobe)
    reps = max(args.steps, 5)
    coarse_ms = timed_ms(torch, stream, reps, lambda: idx.coarse_search(dq, nprobe, workspace=ws))
    adc_ms = timed_ms(torch, stream, reps, lambda: idx.adc_search(dq, probes, k, probe_dists=pd))
    sid, sd, st = idx.adc_search_stats(dq, probes, k, probe_dists=pd)
    loaded_bytes = st["vectors_loaded"] * (m + 4)
    loaded_gbs = loaded_bytes / (adc_ms * 1e-3) / 1e9
    log(f"C1 search: {ms_per_step:.3f} ms/step, {qps:,.0f} QPS; coarse {coarse_ms:.3f} ms, scan {adc_ms:.3f} ms "
        f"({loaded_gbs:.0f} GB/s loaded)")
    gid, gd = out[0].cpu().numpy(), out[1].cpu().numpy()
    cpu = parity = None
    if args.cpu_queries > 0:
        import oracle
        ns = min(args.cpu_queries, nq)
        threads = oracle.lib.orc_max_threads()

        def cpu_search(qq):
            op, _ = oracle.coarse(qq, cent, nprobe)
            return oracle.search_plain(qq, cent, cb, offs, ids, codes, op, k)

        cpu_s, (oid, od) = cpu_timed(lambda: cpu_search(q[:ns]), warm=lambda: cpu_search(q[:50]))
        cpu = {"value": round(ns / cpu_s, 1), "unit": "queries/s", "cores": threads, "kind": "port",
               "cpu_model": cpu_model(),
               "sample": f"all {ns} queries, same index: coarse + LUT/ADC + top-{k} (the oracle's exhaustive scan); "
                         f"median of 3 runs after a warm-up, {cpu_s:.3f}s each, {threads} OpenMP threads"}
        parity = {"queries": ns, "ids_equal": bool(np.array_equal(gid[:ns], oid)),
                  "dists_bit_equal": bool(np.array_equal(gd[:ns].view(np.uint32), od.view(np.uint32)))}
        log(f"cpu baseline {cpu['value']} QPS on {threads} threads; parity {parity}")
    res = {
        "metric": "QPS at fixed nprobe, 100k x 128 IVF-PQ k=10 (1 GPU)",
        "value": round(qps, 1), "unit": "queries/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded Gaussian mixture; index built in-run by this framework's GPU build path",
        "config": {"workload": "BASELINE config 1: 100k x 128 fp32, 256 lists, PQ M=16 x 256, 1000 queries, "
                               "nprobe=16, k=10", "n": cfg.n, "dim": dim, "nlist": cfg.nlist, "pq_m": m, "nq": nq,
                   "nprobe": nprobe, "k": k, "prune_ratio": 100.0},
        "roofline": {"bound": "hbm", "kernel": "adc_flow_kernel<128,16>", "achieved": round(loaded_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(loaded_gbs / HBM_PEAK_GBS, 4),
                     "traffic": None, "bytes_per_launch": loaded_bytes, "avg_launch_ms": round(adc_ms, 4),
                     "note": "achieved = codes + ids of the lists the scan reads (its own count) / kernel time; "
                             "1000 queries are about four per workgroup of the persistent grid, so each query's set-up and first LUT "
                             "are a large share: a latency case"},
        "stages_ms": {"coarse": round(coarse_ms, 4), "adc": round(adc_ms, 4)},
        "cpu_baseline": cpu, "parity": parity,
    }
    print(json.dumps(res), flush=True)


def run_c3(args, torch, fg, dev):
    """two-phase pruned scan + compaction to top-1000 + exact rerank to k=100."""
    dim, nlist, m, nprobe, k = 96, 4096, 48, 64, 100
    p1, limit_k, coeff, rerank_m, mb, eps, beta = 12, 50, 1.0, 1000, 128, 0.1, 2
    n = args.n if args.n != 1_000_000 else 10_000_000
    t0 = time.time()
    x = fg.gen_gmm(n, dim, 1024, seed=2025, set=0, sig_lo=0.05, sig_hi=0.15)
    q = fg.gen_gmm(args.nq, dim, 1024, seed=2025, set=1, sig_lo=0.05, sig_hi=0.15)
    log(f"generated {n}x{dim} base + {args.nq} queries in {time.time() - t0:.1f}s")
    t0 = time.time()
    dx = torch.from_numpy(x).to(dev)
    offs, ids, codes, cent, cb = fg.build_ivfpq(dx, nlist, m, kmeans_iters=20, init_mode=1, seed=42, pq_iters=15,
                                                sample_size=50000, train_rows=min(n, 1_000_000))
    torch.cuda.synchronize()
    log(f"index built on GPU in {time.time() - t0:.1f}s (max list {np.diff(offs).max()}, "
        f"empty lists {(np.diff(offs) == 0).sum()})")
    idx = fg.Index.from_arrays(dim, m, offs, ids, codes, cent, cb)
    dq = torch.from_numpy(q).to(dev)
    nq = args.nq
    ws = torch.empty(idx.search_rerank_workspace_bytes(nq, nprobe, p1, limit_k, rerank_m), dtype=torch.uint8,
                     device=dev)
    out = (torch.empty((nq, k), dtype=torch.int32, device=dev), torch.empty((nq, k), dtype=torch.float32, device=dev))
    stream = torch.cuda.current_stream()

    def step():
        idx.search_rerank(dq, dx, nprobe, k, p1_lists=p1, limit_k=limit_k, threshold_coeff=coeff, rerank_m=rerank_m,
                          mini_batch=mb, eps=eps, beta=beta, workspace=ws, out=out)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = 1e3 * wall / args.steps
    qps = nq / (wall / args.steps)
    log(f"search+rerank: {ms_per_step:.3f} ms/step, {qps:,.0f} QPS")

    # stage timing with HIP events on the launch stream
    probes, _ = idx.coarse_search(dq, nprobe)
    cnt, _ = fg.probe_counts(idx, probes)
    adc_bytes = int(cnt.to(torch.int64).sum().item()) * m
    tp_ws = torch.empty(fg.lib.fgpu_two_phase_workspace_bytes(nq, nprobe, p1, limit_k, rerank_m), dtype=torch.uint8,
                        device=dev)
    tid, td, tc, _, _ = idx.two_phase_search(dq, probes, p1, limit_k, coeff, rerank_m, workspace=tp_ws)
    sid, sd, sc, tstats = idx.two_phase_stats(dq, probes, p1, limit_k, coeff, rerank_m, workspace=tp_ws)
    assert torch.equal(sid, tid) and torch.equal(sd, td) and torch.equal(sc, tc), "instrumented scan differs"
    loaded_bytes = tstats["vectors_loaded"] * (m + 4)
    log(f"two-phase counters: {tstats}; phase-2 loads {loaded_bytes / 1e9:.4f} GB (codes + ids)")
    # Phase 1 runs through the MFMA screen (one single-probe query per (query, phase-1 probe)); its
    # stages, from the events the call records with OPT_STAGE_EVENTS on.
    idx.set_option(fg.Index.OPT_STAGE_EVENTS, 1)
    tp_stage = {kk: 0.0 for kk in fg.Index.TP_STAGES}
    reps_st = max(args.steps, 3)
    for _ in range(reps_st):
        idx.two_phase_search(dq, probes, p1, limit_k, coeff, rerank_m, workspace=tp_ws)
        for kk, v in idx.two_phase_stage_times().items():
            tp_stage[kk] += v / reps_st
    idx.set_option(fg.Index.OPT_STAGE_EVENTS, 0)
    log("two-phase stages (ms): " + ", ".join(f"{kk} {v:.4f}" for kk, v in tp_stage.items()))
    rnd = 2 if tp_stage["screen_round2"] >= tp_stage["screen_round1"] else 1
    scr_ms = tp_stage[f"screen_round{rnd}"]
    scr_flop = 2.0 * (dim + 16) * tstats[f"screen_vector_pairs_round{rnd}"]
    scr_exec_flop = 2.0 * (dim + 16) * 32 * 32 * tstats[f"screen_tiles_round{rnd}"]
    scr_bytes = tstats[f"screen_tiles_round{rnd}"] * 32 * (m + 16)
    scr_tflops = scr_flop / (scr_ms * 1e-3) / 1e12
    log(f"screen round {rnd} of phase 1: {scr_ms:.4f} ms, {scr_flop / 1e9:.2f} GFLOP algorithmic "
        f"({scr_tflops:.1f} TFLOP/s), {scr_exec_flop / 1e9:.2f} GFLOP in MFMA tiles, {scr_bytes / 1e6:.1f} MB of "
        f"codes + blocks read")
    _, _, vis = fg.rerank(dq, dx, tid, tc, k, mb, eps, beta)
    visited = int(vis.to(torch.int64).sum().item())
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    reps = max(args.steps, 3)
    cws = torch.empty(idx.coarse_workspace_bytes(nq), dtype=torch.uint8, device=dev)
    ev[0].record(stream)
    for _ in range(reps):
        idx.coarse_search(dq, nprobe, workspace=cws)
    ev[1].record(stream)
    for _ in range(reps):
        idx.two_phase_search(dq, probes, p1, limit_k, coeff, rerank_m, workspace=tp_ws)
    ev[2].record(stream)
    for _ in range(reps):
        fg.rerank(dq, dx, tid, tc, k, mb, eps, beta)
    ev[3].record(stream)
    torch.cuda.synchronize()
    coarse_ms = ev[0].elapsed_time(ev[1]) / reps
    tp_ms = ev[1].elapsed_time(ev[2]) / reps
    rr_ms = ev[2].elapsed_time(ev[3]) / reps
    adc_gbs = adc_bytes / (tp_ms * 1e-3) / 1e9
    rr_bytes = visited * dim * 4
    log(f"coarse {coarse_ms:.3f} ms, two-phase {tp_ms:.3f} ms (algorithmic ADC bytes {adc_bytes / 1e9:.2f} GB -> "
        f"{adc_gbs:.0f} GB/s), rerank {rr_ms:.3f} ms ({visited} rows = {rr_bytes / 1e9:.2f} GB -> "
        f"{rr_bytes / (rr_ms * 1e-3) / 1e9:.0f} GB/s); candidates/query {tc.float().mean().item():.0f}")
    rows_peak = row_gather_peak(torch, fg, dx, visited)
    rows_one_lane = row_gather_peak(torch, fg, dx, visited, lanes_per_row=1)
    read_peak = stream_read_peak(torch, fg, dev)
    log(f"measured read rates: {rows_peak:.0f} GB/s for random {dim * 4}-byte rows of the base "
        f"({visited} rows, eight lanes a row; {rows_one_lane:.0f} GB/s one lane a row), {read_peak:.0f} GB/s streaming")
    if args.copy_probe:
        a = torch.empty(1 << 28, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b
        log("copy probe: 1 GiB device-to-device copy done")
    gid, gd = out[0].cpu().numpy(), out[1].cpu().numpy()

    cpu = parity = recall = None
    if args.cpu_queries > 0:
        import oracle
        ns = min(args.cpu_queries, nq, 2000)
        threads = oracle.lib.orc_max_threads()

        def cpu_search(qq):
            oprobe, _ = oracle.coarse(qq, cent, nprobe)
            otid, _, otc, _, _ = oracle.search_two_phase(qq, cent, cb, offs, ids, codes, oprobe, p1, limit_k, coeff,
                                                         rerank_m)
            return oracle.rerank(qq, x, otid, otc, k, mb, eps, beta)

        cpu_s, (oid, od, _) = cpu_timed(lambda: cpu_search(q[:ns]), warm=lambda: cpu_search(q[:100]))
        cpu = {"value": round(ns / cpu_s, 1), "unit": "queries/s", "cores": threads, "kind": "port",
               "cpu_model": cpu_model(),
               "sample": f"first {ns} of the {nq} queries, same index: coarse + two-phase scan + rerank; median "
                         f"of 3 runs after a warm-up, {cpu_s:.2f}s each, {threads} OpenMP threads"}
        parity = {"queries": ns, "ids_equal": bool(np.array_equal(gid[:ns], oid)),
                  "dists_bit_equal": bool(np.array_equal(gd[:ns].view(np.uint32), od.view(np.uint32)))}
        log(f"cpu baseline {cpu['value']} QPS on {threads} threads; parity {parity}")
    # recall@k against exact ground truth for every query (fgpu_knn_exact, A18), checked on a sample
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    gt_ids, gt_d = fg.knn_exact(dq, dx, k)
    torch.cuda.synchronize()
    gt_s = time.perf_counter() - t0
    gt = gt_ids.cpu().numpy()
    recall = float(np.mean([len(set(gid[i]) & set(gt[i])) / k for i in range(nq)]))
    gt_parity = None
    if args.cpu_queries > 0:
        ng = 50
        ogt, ogd = oracle.knn_exact(q[:ng], x, k)
        gt_parity = bool(np.array_equal(gt[:ng], ogt) and
                         np.array_equal(gt_d.cpu().numpy()[:ng].view(np.uint32), ogd.view(np.uint32)))
    log(f"exact kNN ground truth on GPU: {nq} x {n} in {gt_s:.2f}s; recall@{k} {recall:.4f}; "
        f"ground truth equals the oracle on 50 queries: {gt_parity}")

    res = {
        "metric": "QPS, 10M x 96 IVF-PQ (4096 lists, M=48), nprobe=64, two-phase top-1000 + exact rerank to k=100 "
                  "(1 GPU)",
        "value": round(qps, 1), "unit": "queries/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded Gaussian mixture; index built in-run by this framework's GPU build path",
        "config": {"workload": "BASELINE config 3: 10M x 96 fp32, 4096 lists, PQ M=48, 10k queries, nprobe=64, "
                               "p1_lists 12, limit_k 50, threshold_coeff 1.0, top-1000 -> exact rerank k=100",
                   "n": n, "dim": dim, "nlist": nlist, "pq_m": m, "nq": nq, "nprobe": nprobe, "k": k},
        "roofline": {"bound": "mfma", "kernel": f"screen_kernel<96,48,{rnd}> (phase-1 screen round {rnd})",
                     "achieved": round(scr_tflops, 2), "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(scr_tflops / BF16_MFMA_PEAK_TFLOPS, 4),
                     "traffic": read_traffic(TRAFFIC_FILE_C3, f"traffic_bytes_per_launch_round{rnd}"),
                     "avg_launch_ms": round(scr_ms, 4), "flop_per_launch": scr_flop,
                     "mfma_tile_flop_per_launch": scr_exec_flop,
                     "mfma_tile_frac": round(scr_exec_flop / (scr_ms * 1e-3) / 1e12 / BF16_MFMA_PEAK_TFLOPS, 4),
                     "bytes_read_per_launch": scr_bytes, "hbm_gbs": round(scr_bytes / (scr_ms * 1e-3) / 1e9, 1),
                     "note": "the two-phase call's longest kernel: phase 1 (each phase-1 list's top-50 and cutoff) "
                             "as one single-probe screen query per (query, phase-1 probe); achieved = 2 (dim + 16) "
                             "flops per (query, vector) pair screened / its event-timed duration, against the "
                             "dense bf16 peak; traffic = copy-calibrated FETCH_SIZE + WRITE_SIZE per launch "
                             "(profiles/two_phase_c3_traffic.txt)"},
        "two_phase": {"ms": round(tp_ms, 4), "stages_ms": {kk: round(v, 4) for kk, v in tp_stage.items()},
                      "work_equivalent_adc_bytes": adc_bytes, "work_equivalent_gbs": round(adc_gbs, 1),
                      "note": "work-equivalent: code bytes of every probed list once per (query, list), over the "
                              "two-phase time; phase 2 skips lists whose bound exceeds the threshold",
                      **tstats},
        "stages_ms": {"coarse": round(coarse_ms, 4), "two_phase": round(tp_ms, 4), "rerank": round(rr_ms, 4),
                      "rerank_rows": visited, "rerank_gbs": round(rr_bytes / (rr_ms * 1e-3) / 1e9, 1),
                      "rerank_frac_of_measured_row_rate": round(rr_bytes / (rr_ms * 1e-3) / 1e9 / rows_peak, 4),
                      "candidates_per_query": round(tc.float().mean().item(), 1)},
        "measured_read_gbs": {"random_rows": round(rows_peak, 1), "random_rows_one_lane": round(rows_one_lane, 1),
                              "streaming": round(read_peak, 1),
                              "note": f"random rows: {visited} whole {dim * 4}-byte rows of the base at seeded random "
                                      "ids, eight lanes a row (fgpu_row_gather; the rerank's pattern) and one lane a "
                                      "row (fgpu_row_gather_lanes 1); streaming: fgpu_stream_read over 4 GiB"},
        "cpu_baseline": cpu, "parity": parity, "recall_at_k": recall,
        "ground_truth": {"seconds": round(gt_s, 3), "oracle_parity_50": gt_parity},
    }
    print(json.dumps(res), flush=True)


def knee(lists, sse):
    """Kneedle on a decreasing curve: normalised (log2 L, SSE); largest gap below the chord; first on ties."""
    x = np.log2(np.asarray(lists, np.float64))
    y = np.asarray(sse, np.float64)
    xn = (x - x[0]) / (x[-1] - x[0])
    yn = (y - y[-1]) / (y[0] - y[-1]) if y[0] != y[-1] else np.zeros_like(y)
    return int(lists[int(np.argmax((1.0 - xn) - yn))])


def run_c4(args, torch, fg, dev):
    """the index build, phase by phase, plus the elbow sweep."""
    dim, nlist, m, train = 128, 4096, 32, 1_000_000
    n = args.n if args.n != 1_000_000 else 10_000_000
    t0 = time.time()
    x = fg.gen_gmm(n, dim, 1024, seed=2027, set=0, sig_lo=0.05, sig_hi=0.15)
    log(f"generated {n}x{dim} in {time.time() - t0:.1f}s")
    dx = torch.from_numpy(x).to(dev)
    rows = torch.from_numpy((np.arange(train, dtype=np.int64) * n) // train).to(dev)
    dtr = dx[rows].contiguous()
    torch.cuda.synchronize()

    def timed(fn):
        torch.cuda.synchronize()
        t = time.perf_counter()
        r = fn()
        torch.cuda.synchronize()
        return r, time.perf_counter() - t

    (cent, _), t_km = timed(lambda: fg.kmeans_fit(dtr, nlist, 20, init_mode=1, seed=42, want_assign=False))
    (asg, dist), t_as = timed(lambda: fg.l2_topk(dx, cent, 1))
    asg = asg[:, 0].contiguous()
    cb, t_pq = timed(lambda: fg.pq_train(dx, asg, cent, m, sample_size=50000, iters=15))
    codes, t_en = timed(lambda: fg.pq_encode(dx, asg, cent, cb))
    total = t_km + t_as + t_pq + t_en
    # one Lloyd assignment pass on the sample: the MFMA GEMM + exact re-score
    _, t_lloyd = timed(lambda: fg.l2_topk(dtr, cent, 1))
    gemm_flop = 2.0 * n * nlist * dim
    lloyd_flop = 2.0 * train * nlist * dim
    log(f"build: k-means (k-means++ + 20 iterations on {train} rows) {t_km:.2f}s, assign {n} rows {t_as:.2f}s "
        f"({gemm_flop / t_as / 1e12:.1f} TFLOP/s), PQ train {t_pq:.2f}s, encode {t_en:.2f}s; total {total:.2f}s; "
        f"one Lloyd assignment {t_lloyd * 1e3:.1f} ms ({lloyd_flop / t_lloyd / 1e12:.1f} TFLOP/s)")
    # elbow sweep
    t0 = time.perf_counter()
    sse = {}
    for L in (1024, 2048, 4096):
        c = cent if L == nlist else fg.kmeans_fit(dtr, L, 20, init_mode=1, seed=42, want_assign=False)[0]
        _, d = fg.l2_topk(dtr, c, 1)
        sse[L] = float(d.to(torch.float64).sum().item())
    t_elbow = time.perf_counter() - t0
    chosen = knee(list(sse), list(sse.values()))
    log(f"elbow sweep {t_elbow:.2f}s: SSE {sse}; knee at {chosen} lists")
    cpu = parity = None
    if args.cpu_queries > 0:
        import oracle
        ns = min(args.cpu_queries, 20000)
        threads = oracle.lib.orc_max_threads()
        hcent = cent.cpu().numpy()
        cpu_s, oa = cpu_timed(lambda: oracle.kmeans_assign(x[:ns], hcent),
                              warm=lambda: oracle.kmeans_assign(x[:1000], hcent))
        cpu = {"value": round(ns / cpu_s, 1), "unit": "rows assigned/s", "cores": threads, "kind": "port",
               "cpu_model": cpu_model(),
               "sample": f"exact assignment of the first {ns} rows to the 4096 centroids; median of 3 runs after a "
                         f"warm-up, {cpu_s:.2f}s each, {threads} OpenMP threads"}
        parity = {"rows": ns, "assignment_equal": bool(np.array_equal(asg[:ns].cpu().numpy(), oa)),
                  "codes_equal": bool(np.array_equal(codes[:2000].cpu().numpy(),
                                                     oracle.pq_encode(x[:2000], oa[:2000], hcent, cb.cpu().numpy(),
                                                                      fma_mode=1)))}
        log(f"cpu baseline {cpu['value']} rows/s on {threads} threads; parity {parity}")
    res = {
        "metric": "index build rows/s: 10M x 128, 4096 lists (k-means on a 1M sample), PQ M=32 (1 GPU)",
        "value": round(n / total, 1), "unit": "rows/s", "n_gpus": 1, "steps": 1, "warmup": 0,
        "ms_per_step": round(total * 1e3, 1), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic: seeded 1024-component Gaussian mixture",
        "config": {"workload": "BASELINE config 4: 10M x 128, k-means++ + 20 Lloyd iterations of 4096 centroids on "
                               "a 1M sample, PQ M=32 x 256 (15 iterations), encode 10M, elbow 1024/2048/4096",
                   "n": n, "dim": dim, "nlist": nlist, "pq_m": m, "train_rows": train},
        "roofline": {"bound": "mfma", "kernel": "gemm_est_split_kernel + select_exact_kernel (assignment of all "
                               "rows; FLOP counted as the fp32-equivalent 2 n k D, the split issues three bf16 "
                               "products each)",
                     "achieved": round(gemm_flop / t_as / 1e12, 2), "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_flop / t_as / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4), "traffic": None},
        "phases_s": {"kmeans": round(t_km, 3), "assign": round(t_as, 3), "pq_train": round(t_pq, 3),
                     "encode": round(t_en, 3), "elbow_sweep": round(t_elbow, 3),
                     "lloyd_assignment_ms": round(t_lloyd * 1e3, 2)},
        "elbow": {"sse": sse, "knee": chosen},
        "cpu_baseline": cpu, "parity": parity,
    }
    print(json.dumps(res), flush=True)


def run_c5(args, torch, fg, dev):
    """graph search, itopk 64, width 4, <= 64 steps, k=10."""
    dim, degree, itopk, width, max_iter, k = 128, 32, 64, 4, 64, 10
    n = args.n if args.n != 1_000_000 else 5_000_000
    nq = args.nq
    t0 = time.time()
    ncomp, nrand = args.c5_components, args.c5_random_edges
    x = fg.gen_gmm(n, dim, ncomp, seed=2026, set=0, sig_lo=0.05, sig_hi=0.15)
    q = fg.gen_gmm(nq, dim, ncomp, seed=2026, set=1, sig_lo=0.05, sig_hi=0.15)
    log(f"generated {n}x{dim} base + {nq} queries in {time.time() - t0:.1f}s")
    t0 = time.time()
    dx = torch.from_numpy(x).to(dev)
    # forward candidates by IVF-PQ search + exact rerank, CAGRA's reverse-edge step, seeded long-range edges
    from fusiongpu_amd import workloads as W
    graph = W.knn_graph(dx, degree, nrand, reverse=not args.c5_no_reverse)
    torch.cuda.synchronize()
    log(f"index + degree-{degree} graph built on GPU in {time.time() - t0:.1f}s")
    dq = torch.from_numpy(q).to(dev)
    out = (torch.empty((nq, k), dtype=torch.int32, device=dev), torch.empty((nq, k), dtype=torch.float32, device=dev))
    stream = torch.cuda.current_stream()

    def step():
        fg.graph_search(dq, dx, graph, k, itopk, width, max_iter, seed=1, out=out)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = 1e3 * wall / args.steps
    qps = nq / (wall / args.steps)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record(stream)
    step()
    ev[1].record(stream)
    torch.cuda.synchronize()
    kern_ms = ev[0].elapsed_time(ev[1])
    gid_t, gd_t, it_t, evals = fg.graph_search(dq, dx, graph, k, itopk, width, max_iter, seed=1, want_evals=True)
    assert torch.equal(gid_t, out[0]) and torch.equal(gd_t, out[1]), "instrumented search differs"
    n_evals = int(evals.to(torch.int64).sum().item())
    n_steps = int(it_t.to(torch.int64).sum().item())
    gather_bytes = n_evals * dim * 4 + n_steps * width * degree * 4
    gbs = gather_bytes / (kern_ms * 1e-3) / 1e9
    log(f"graph search: {ms_per_step:.3f} ms/step, {qps:,.0f} QPS; kernel {kern_ms:.3f} ms; {n_steps / nq:.1f} steps "
        f"and {n_evals / nq:.0f} distance evaluations per query -> {gather_bytes / 1e9:.2f} GB = {gbs:.0f} GB/s")
    rows_peak = row_gather_peak(torch, fg, dx, n_evals)
    rows_one_lane = row_gather_peak(torch, fg, dx, n_evals, lanes_per_row=1)
    log(f"measured read rate for random {dim * 4}-byte rows of the base: {rows_peak:.0f} GB/s ({n_evals} rows, "
        f"eight lanes a row; {rows_one_lane:.0f} GB/s one lane a row)")
    gid, gd = out[0].cpu().numpy(), out[1].cpu().numpy()
    gt, _ = fg.knn_exact(dq, dx, k)
    gt = gt.cpu().numpy()
    rec = np.array([len(set(gid[i]) & set(gt[i])) / k for i in range(nq)])
    recall = float(rec.mean())
    # a walk that ends in the query's own mixture component finds a nearest distance within 2x of the
    # true one (components lie about 9 apart, their points about 1.5 from each other)
    gtd = fg.knn_exact(dq, dx, 1)[1][:, 0].cpu().numpy()
    own = gd[:, 0] <= 2.0 * gtd
    log(f"recall@{k} {recall:.4f} against exact kNN; {own.mean():.3f} of the walks end in the query's component, "
        f"recall {rec[own].mean():.4f} there")

    cpu = parity = None
    if args.cpu_queries > 0:
        import oracle
        ns = min(args.cpu_queries, nq, 1000)
        threads = oracle.lib.orc_max_threads()
        hgraph = graph.cpu().numpy()
        cpu_s, (oid, od, _) = cpu_timed(
            lambda: oracle.graph_search(q[:ns], x, hgraph, k, itopk, width, max_iter, seed=1),
            warm=lambda: oracle.graph_search(q[:50], x, hgraph, k, itopk, width, max_iter, seed=1))
        cpu = {"value": round(ns / cpu_s, 1), "unit": "queries/s", "cores": threads, "kind": "port",
               "cpu_model": cpu_model(),
               "sample": f"first {ns} of the {nq} queries, same graph; median of 3 runs after a warm-up, "
                         f"{cpu_s:.2f}s each, {threads} OpenMP threads"}
        parity = {"queries": ns, "ids_equal": bool(np.array_equal(gid[:ns], oid)),
                  "dists_bit_equal": bool(np.array_equal(gd[:ns].view(np.uint32), od.view(np.uint32)))}
        log(f"cpu baseline {cpu['value']} QPS on {threads} threads; parity {parity}")
    res = {
        "metric": "QPS, graph search over 5M x 128 (degree 32, itopk 64, width 4, <= 64 steps), k=10 (1 GPU)",
        "value": round(qps, 1), "unit": "queries/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32",
        "data": f"synthetic: seeded {ncomp}-component Gaussian mixture; graph = forward candidates by this "
                f"framework's IVF-PQ search (ADC top-64, exact rerank)"
                f"{'' if args.c5_no_reverse else ' with CAGRA reverse edges'}, last {nrand} slots seeded random "
                f"long-range edges",
        "config": {"workload": "BASELINE config 5: 5M x 128 fp32, out-degree-32 graph, 10k queries, itopk 64, "
                               "width 4, max 64 steps, k=10",
                   "n": n, "dim": dim, "degree": degree, "nq": nq, "itopk": itopk, "width": width,
                   "max_iter": max_iter, "k": k},
        "roofline": {"bound": "hbm", "kernel": "graph_search_kernel<128>", "achieved": round(gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": gather_bytes, "avg_launch_ms": round(kern_ms, 4),
                     "distance_evaluations": n_evals, "steps": n_steps,
                     "measured_row_gather_gbs": round(rows_peak, 1),
                     "measured_row_gather_one_lane_gbs": round(rows_one_lane, 1),
                     "frac_of_measured_row_rate": round(gbs / rows_peak, 4),
                     "note": "achieved = distance rows + adjacency rows read / kernel time; the measured row rate is "
                             "fgpu_row_gather over as many random whole rows of the base, eight lanes a row"},
        "cpu_baseline": cpu, "parity": parity, "recall_at_k": recall,
        "walks_in_query_component": round(float(own.mean()), 4),
        "recall_in_query_component": round(float(rec[own].mean()), 4),
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
