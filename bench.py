#!/usr/bin/env python3
"""Headline benchmark: queries/sec at recall@100 >= 0.95 on the C2 workload.

C2: 1M base x 128-d integer-valued Gaussian mixture
(1024 components), 10k queries from the same mixture, degree-32 graph with
RaBitQ 1-bit codes, K = 100, beam sweep 100..1024 (the reference README's
Figure 13 list: 100, 128, 256, 384, 512, 640, 768, 896, 1024).  A step is one
search-kernel launch over the whole 10k-query batch, with the codebook and the
queries already resident in HBM.  The reported beam is the smallest one whose
recall@100 reaches 0.95.

Also reported, on the same JSON line:
  roofline     algorithmic HBM bytes of one launch (per query:
               4*d + 4*ids_read + estimates*(B/8 + 12) + exact*4*d, summed from
               the kernel's own work counters) / HIP-event launch duration,
               against the MI355X 8 TB/s peak;
  cpu_baseline the CPU oracle (a restatement of the same search) timed on the
               host cores over a bounded query sample at the same beam, with
               its ids compared to the GPU's.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0

# BASELINE.json configurations (generator, shape, default K, beams).  C2 is
# the headline; the others run with --config for coverage measurements.
CONFIGS = {
    "c1": dict(n=100_000, nq=1000, dim=128, components=64, degree=32, K=10, beams="64",
               gen="integer_mixture", cfg=1),
    "c2": dict(n=1_000_000, nq=10_000, dim=128, components=1024, degree=32, K=100,
               beams="100,128,256,384,512,640,768,896,1024", gen="integer_mixture", cfg=2),
    "c3": dict(n=1_000_000, nq=10_000, dim=96, components=1024, degree=32, K=100,
               beams="16,32,64,96,128,256,384,512", gen="normalized_mixture", cfg=3),
    "c4": dict(n=1_000_000, nq=1000, dim=960, components=256, degree=32, K=100,
               beams="128,256,384,512,640,768,896,1024", gen="unit_box_mixture", cfg=4),
    "c5": dict(n=10_000_000, nq=10_000, dim=1536, components=4096, degree=32, K=100,
               beams="128,256,384,512,640,768,896,1024", gen="anisotropic_unit_mixture", cfg=5),
}


def log(msg: str) -> None:
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=str, default="c2", choices=sorted(CONFIGS),
                    help="BASELINE configuration (c2 = the headline; the others for coverage)")
    ap.add_argument("--metric", type=str, default="l2", choices=("l2", "ip"),
                    help="distance (ip: inner product, the reference's Text2Image path; codes, graph and "
                         "ground truth built for it)")
    ap.add_argument("--n", type=int, default=0, help="base points (default: the configuration's)")
    ap.add_argument("--nq", type=int, default=0)
    ap.add_argument("--components", type=int, default=0)
    ap.add_argument("--degree", type=int, default=0)
    ap.add_argument("--K", type=int, default=0)
    ap.add_argument("--beams", type=str, default="")
    ap.add_argument("--target-recall", type=float, default=0.95)
    ap.add_argument("--beam", type=int, default=0, help="skip the sweep and use this beam")
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="CPU-oracle work budget")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle (baseline and id checks)")
    ap.add_argument("--stop-at-target", action="store_true",
                    help="end the beam sweep at the first beam that reaches the target recall (default: sweep every "
                         "beam of --beams for recall, QPS and oracle parity; the headline is the first beam that "
                         "reaches the target either way)")
    ap.add_argument("--full-sweep", action="store_true", help="(the default; kept for old command lines)")
    ap.add_argument("--graph", type=str, default="mixed", choices=("mixed", "rng", "connected"),
                    help="mixed: RNG-pruned k-NN edges plus degree/4 seeded random long links, empty slots to "
                         "random targets (the default); rng: RNG-pruned k-NN edges only, empty slots backfilled "
                         "from the k-NN candidates; connected: rng plus the links that make every node reachable "
                         "from the entry point (NSG-style repair, in backfilled or empty slots)")
    ap.add_argument("--alpha", type=float, default=1.0,
                    help="RNG prune slack: drop a candidate v when a kept w has alpha^2 d(w,v) < d(u,v)")
    ap.add_argument("--random-links", type=int, default=-1,
                    help="seeded random long links per node (default: degree/4; the rng graph has none)")
    ap.add_argument("--candidates", type=int, default=0, help="k-NN candidates per node before the prune "
                    "(default: 2*degree)")
    ap.add_argument("--no-rng-graph", action="store_true",
                    help="skip the side measurements on the RNG-only and connected graphs (default: C2 with the "
                         "mixed graph also sweeps them and reports them in config.rng_graph and "
                         "config.connected_graph)")
    ap.add_argument("--parity-sample", type=int, default=500,
                    help="queries per swept beam whose GPU ids are compared with the CPU oracle's")
    ap.add_argument("--traffic", type=str, default=os.path.join(ROOT, "profiles", "search_c2_traffic.json"))
    ap.add_argument("--cache", type=str, default="", help="directory to reuse the built index and ground truth")
    ap.add_argument("--serve-batches", type=int, default=8,
                    help="batches of nq queries in the serving measurement (0 = skip)")
    ap.add_argument("--large", type=str, default="auto", choices=("auto", "on", "off"),
                    help="draw the data on the GPU and build the graph from a partitioned k-NN search "
                         "(auto: when n x dim exceeds 2^31 floats, i.e. C5 at 10M)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a 1 GiB device copy, a 1 GiB elementwise kernel and a 512 MiB random-row "
                         "gather, each of known traffic (counter calibration for profiling)")
    args = ap.parse_args()
    conf = CONFIGS[args.config]
    for key in ("n", "nq", "components", "degree", "K", "beams"):
        if not getattr(args, key):
            setattr(args, key, conf[key])

    if args.gpus != 1:
        print(f"bench.py: this search runs on one GPU only (queries are independent; a multi-GPU "
              f"run would replicate the index and split the queries); --gpus {args.gpus} is not supported",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import flashgann_amd as fg
    from flashgann_amd import builder, datasets
    from flashgann_amd.codebook import padded_dim_for

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    dim = conf["dim"]
    B = padded_dim_for(dim)

    from flashgann_amd.codebook import read_codebook

    # Sets too large to draw and hold on the host (C5: 10M x 1536 = 61 GB)
    # are drawn on the GPU and get the partitioned k-NN graph; the codebook
    # rows still land in host memory, where the CPU oracle reads them.
    large = args.n * dim > (1 << 31) if args.large == "auto" else args.large == "on"
    t0 = time.time()
    if large:
        gen_dev = getattr(datasets, conf["gen"] + "_device", None)
        if gen_dev is None:
            print(f"bench.py: {args.config} has no device-side generator for a set of {args.n} x {dim}",
                  file=sys.stderr)
            return 2
        base, queries_t = gen_dev(args.n, args.nq, dim, args.components, config=conf["cfg"], device=dev)
        queries = queries_t.cpu().numpy()
        del queries_t
    else:
        base, queries = getattr(datasets, conf["gen"])(args.n, args.nq, dim, args.components, config=conf["cfg"])
    signs = datasets.signs_for(B, conf["cfg"])
    log(f"data {args.n}x{dim} + {args.nq} queries in {time.time() - t0:.1f}s"
        + (" (drawn on the GPU)" if large else ""))
    if large:
        graph_kw_large = dict(knn_method="partitioned", verbose=True)
    else:
        graph_kw_large = {}
    use_ip = args.metric == "ip"
    tag = (f"{args.config}_{args.n}_{args.nq}_{args.components}_{args.degree}_{args.K}" + ("_ip" if use_ip else "")
           + {"mixed": "", "rng": "_rng", "connected": "_conn"}[args.graph])
    build_stats = {}
    graph_kw = (dict(random_links=0, fill_random=False) if args.graph == "rng" else
                dict(random_links=0, fill_random=False, connect=True, stats=build_stats)
                if args.graph == "connected" else {})
    if args.random_links >= 0 and args.graph == "mixed":
        graph_kw["random_links"] = args.random_links
    graph_kw["alpha"] = args.alpha
    if args.candidates:
        graph_kw["candidates"] = args.candidates
    if args.alpha != 1.0 or args.random_links >= 0 or args.candidates:
        tag += f"_a{args.alpha}_r{args.random_links}_c{args.candidates}"
    cb_path = os.path.join(args.cache, tag + ".index") if args.cache else ""
    gt_path = os.path.join(args.cache, tag + ".gt.npy") if args.cache else ""
    if cb_path and os.path.exists(cb_path) and os.path.exists(gt_path):
        cb = read_codebook(cb_path, args.n, dim, args.degree)
        gt = np.load(gt_path)
        log(f"codebook and ground truth loaded from {args.cache}")
    else:
        t0 = time.time()
        cb = builder.build_codebook(base, args.degree, signs, use_ip=use_ip, device=dev, **graph_kw,
                                    **graph_kw_large)
        log(f"codebook built on GPU in {time.time() - t0:.1f}s (entry {cb.entry})")
        t0 = time.time()
        gt = builder.ground_truth(base, queries, args.K, device=dev, use_ip=use_ip)
        bad = builder.check_ground_truth(base, queries, gt, sample=32, use_ip=use_ip, device=dev)
        log(f"ground truth in {time.time() - t0:.1f}s (32 sampled queries rechecked one at a time: {bad} wrong)")
        if bad:
            print(f"bench.py: the ground truth failed its recheck on {bad} of 32 sampled queries", file=sys.stderr)
            return 3
        if large:
            base = None  # the device copy; the codebook rows hold the vectors
        if cb_path:
            os.makedirs(args.cache, exist_ok=True)
            cb.save(cb_path)
            np.save(gt_path, gt)
    torch.cuda.empty_cache()
    if args.copy_probe:
        src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log("copy probe: 1 GiB read + 1 GiB written by one device copy")
        torch.mul(src, 2.0, out=dst)
        torch.cuda.synchronize()
        log("copy probe: 1 GiB read + 1 GiB written by one elementwise kernel")
        # random 512-byte rows, the search's exact-distance access pattern:
        # 2^20 of the 2^21 rows gathered (512 MiB read, 512 MiB written, plus
        # the 8 MiB index)
        perm = torch.randperm(1 << 21, device=dev)[: 1 << 20]
        torch.cuda.synchronize()
        g = src.view(-1, 128).index_select(0, perm)
        torch.cuda.synchronize()
        log("copy probe: 512 MiB of random 512-byte rows gathered by one index_select")
        del src, dst, perm, g

    index = fg.Index.from_codebook(cb, metric=fg.METRIC_IP if use_ip else fg.METRIC_L2)
    dq = torch.as_tensor(queries, device=dev)
    dres = torch.empty((args.nq, args.K), dtype=torch.int32, device=dev)
    dcnt = torch.empty((args.nq, fg.FG_COUNTERS_PER_QUERY), dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream()

    def launch(beam: int, counters: bool = False) -> None:
        index.search_device(dq.data_ptr(), args.nq, args.K, beam, dres.data_ptr(),
                            dcnt.data_ptr() if counters else 0, stream.cuda_stream)

    def recall_of(ids: np.ndarray) -> float:
        hit = 0
        for i in range(ids.shape[0]):
            hit += np.isin(ids[i], gt[i, : args.K]).sum()
        return hit / float(ids.size)

    # Oracle handle for the per-beam id checks (bounded samples) and the CPU
    # baseline; built once.
    oix = None
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    # the host's CPU share for this GPU: the affinity set, bounded by the
    # thread count the host configures for its jobs (OMP_NUM_THREADS)
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = max(1, min(affinity, share) if share > 0 else affinity)
    cpu_model = ""
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                cpu_model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    if not args.no_cpu:
        from oracle import oracle as O
        oix = O.OracleIndex.from_codebook(cb, use_ip=use_ip)

    # Beam sweep (the reference README's QPS-recall list): per beam one
    # counting launch, then timed launches (HIP events), recall@K against the
    # ground truth, and the GPU ids compared with the CPU oracle's on the first
    # `--parity-sample` queries.
    sweep = []
    beams = [args.beam] if args.beam else [int(b) for b in args.beams.split(",")]
    chosen = None
    # The oracle checks leave the GPU idle for up to a second between beams,
    # and a search right after an idle spell runs 5-15% slower while the
    # clocks come back up, so each beam's timing follows three untimed
    # searches and takes the median of five.
    for beam in beams:
        launch(beam, counters=True)
        for _ in range(3):
            launch(beam)
        torch.cuda.synchronize()
        ms = []
        for _ in range(5):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            launch(beam)
            e1.record(stream)
            torch.cuda.synchronize()
            ms.append(e0.elapsed_time(e1))
        kms = float(np.median(ms))
        ids = dres.cpu().numpy().view(np.uint32)
        r = recall_of(ids)
        row = {"beam": beam, "recall": round(float(r), 5), "qps": round(args.nq / (kms / 1e3), 1),
               "kernel_ms": round(kms, 4)}
        if oix is not None and args.parity_sample > 0:
            m = min(args.nq, args.parity_sample)
            pids, _ = oix.search(queries[:m], args.K, beam, threads=threads)
            row["oracle_ids_identical"] = float((pids == ids[:m]).all(1).mean())
            row["oracle_sample"] = m
        sweep.append(row)
        log(f"beam {beam}: recall@{args.K} {r:.4f}, {row['qps']:.0f} QPS ({kms:.3f} ms)"
            + (f", ids identical to the oracle on {row['oracle_ids_identical'] * 100:.2f}% of {row['oracle_sample']}"
               if "oracle_sample" in row else ""))
        if chosen is None and r >= args.target_recall:
            chosen = beam
            if args.stop_at_target:
                break
    if chosen is None:
        chosen = beams[-1]
        log(f"no beam reached recall {args.target_recall}; reporting beam {chosen}")

    # per-query work counters at the chosen beam -> algorithmic bytes per launch
    launch(chosen, counters=True)
    torch.cuda.synchronize()
    ids = dres.cpu().numpy().view(np.uint32).copy()
    cnt = dcnt.cpu().numpy().view(np.uint32).astype(np.int64)
    recall = recall_of(ids)
    ids_read, estimates, exact = cnt[:, 2].sum(), cnt[:, 3].sum(), cnt[:, 4].sum()
    alg_bytes = int(args.nq * 4 * dim + 4 * ids_read + estimates * (B // 8 + 12) + exact * 4 * dim)
    work = {k: round(float(cnt[:, i].mean()), 2) for i, k in
            enumerate(("iterations", "expansions", "ids_read", "estimates", "exact"))}
    log(f"beam {chosen}: per query {work}")

    # timed region: K launches bracketed by synchronisation
    for _ in range(args.warmup):
        launch(chosen)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_start = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        launch(chosen)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    kernel_ms = ev0.elapsed_time(ev1) / args.steps
    ms_per_step = wall * 1e3 / args.steps
    qps = args.nq / (ms_per_step / 1e3)
    achieved = alg_bytes / (kernel_ms / 1e3) / 1e9
    log(f"beam {chosen}: {ms_per_step:.3f} ms/step (kernel {kernel_ms:.3f} ms), {qps:.0f} QPS, "
        f"{achieved:.1f} GB/s algorithmic")

    # The reference's timing contract for one call: the host clock around one
    # search launch and the device synchronisation (gpu_search_adaptive.cu:98-107),
    # QPS = nq / elapsed (main.cu:85-86).  Eleven single synchronous searches
    # right after the timed region (a warm GPU); the median is reported.
    single = []
    for _ in range(11):
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        launch(chosen)
        torch.cuda.synchronize()
        single.append((time.perf_counter() - t1) * 1e3)
    single_ms = float(np.median(single))
    log(f"beam {chosen}: one synchronous search {single_ms:.3f} ms (median of 11; {args.nq / single_ms * 1e3:.0f} QPS)")

    # The device's measured copy bandwidth, the second yardstick for the
    # roofline fraction: ten 1 GiB device-to-device copies (1 GiB read and
    # 1 GiB written each) timed with events on torch's stream.
    src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    cstream = torch.cuda.current_stream()
    c0.record(cstream)
    for _ in range(10):
        dst.copy_(src)
    c1.record(cstream)
    torch.cuda.synchronize()
    copy_gbs = 10 * 2 * src.numel() * 4 / (c0.elapsed_time(c1) / 1e3) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    log(f"device copy: {copy_gbs:.1f} GB/s (read + write); the search's algorithmic rate is "
        f"{achieved / copy_gbs:.3f} of it")

    # the same search through the host-buffer entry point (queries copied in,
    # ids copied out, PCIe included) -- reported beside, never as, `value`
    host_q = np.ascontiguousarray(queries, dtype=np.float32)
    index.search(host_q, args.K, chosen)
    t_host = time.perf_counter()
    for _ in range(3):
        index.search(host_q, args.K, chosen)
    host_qps = 3 * args.nq / (time.perf_counter() - t_host)
    log(f"beam {chosen}: {host_qps:.0f} QPS through fg_search (host buffers, PCIe included)")

    # Serving measurement (reported beside `value`, never as it): R batches of
    # the nq queries back to back, (a) one launch per batch on one stream (the
    # reference's one-launch-per-call pattern), (b) fg_search_stream with the
    # batches spread over two streams, (c) one launch over all R*nq queries.
    serving = None
    if args.serve_batches > 0:
        R = args.serve_batches
        dqr = dq.repeat(R, 1).contiguous()
        drr = torch.empty((R * args.nq, args.K), dtype=torch.int32, device=dev)

        def timed(fn, reps=3):
            fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(reps):
                fn()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) / reps

        def serial():
            for r in range(R):
                index.search_device(dqr[r * args.nq].data_ptr(), args.nq, args.K, chosen,
                                    drr[r * args.nq].data_ptr(), 0, stream.cuda_stream)

        def streamed():
            index.search_stream(dqr.data_ptr(), R * args.nq, args.K, chosen, drr.data_ptr(), args.nq, 2,
                                stream.cuda_stream)

        def single():
            index.search_device(dqr.data_ptr(), R * args.nq, args.K, chosen, drr.data_ptr(), 0, stream.cuda_stream)

        t_serial, t_stream, t_single = timed(serial), timed(streamed), timed(single)
        same = bool((drr[: args.nq].cpu().numpy().view(np.uint32) == ids).all())
        serving = {"batches": R, "batch": args.nq, "serial_qps": round(R * args.nq / t_serial, 1),
                   "two_stream_qps": round(R * args.nq / t_stream, 1),
                   "one_launch_qps": round(R * args.nq / t_single, 1), "ids_identical": same}
        log(f"serving {R} x {args.nq} queries at beam {chosen}: one stream {serving['serial_qps']:.0f} QPS, "
            f"two streams {serving['two_stream_qps']:.0f} QPS, one launch {serving['one_launch_qps']:.0f} QPS")
        del dqr, drr

    traffic = None
    traffic_source = None
    if os.path.exists(args.traffic):
        try:
            t = json.load(open(args.traffic))
            if (t.get("config", "c2") == args.config and t.get("n") == args.n and t.get("nq") == args.nq
                    and t.get("beam") == chosen):
                traffic = t.get("hbm_bytes_per_launch")
                traffic_source = (os.path.relpath(args.traffic, ROOT) + " (DRAM read and write bytes of a committed "
                                  "rocprofv3 --pmc run of this workload and beam; not measured in this run)")
        except Exception:
            traffic = None

    cpu = None
    if oix is not None:
        probe = min(args.nq, max(threads * 4, 64))
        t1 = time.perf_counter()
        pids, _ = oix.search(queries[:probe], args.K, chosen, threads=threads)
        per_q_cpu = (time.perf_counter() - t1) * threads / probe
        sample = int(min(args.nq, max(probe, args.cpu_seconds / max(per_q_cpu, 1e-6))))
        t1 = time.perf_counter()
        cids, _ = oix.search(queries[:sample], args.K, chosen, threads=threads)
        cpu_s = time.perf_counter() - t1
        same = float((cids == ids[:sample]).all(1).mean())
        # one host thread over a proportionally smaller sample (about 2 s)
        one = int(min(sample, max(8, 2.0 / max(per_q_cpu, 1e-6))))
        t1 = time.perf_counter()
        oix.search(queries[:one], args.K, chosen, threads=1)
        one_qps = one / (time.perf_counter() - t1)
        cpu = {"value": round(sample / cpu_s, 1), "unit": "queries/s", "cores": threads, "kind": "port",
               "sample": f"first {sample} of the {args.nq} {args.config.upper()} queries at beam {chosen}, "
                         f"{threads} host threads, {cpu_s:.1f} s wall",
               "ids_identical_to_gpu": same, "single_thread_value": round(one_qps, 1),
               "cpu_model": cpu_model, "affinity_cpus": affinity, "os_cpu_count": os.cpu_count(),
               "omp_num_threads": share or None}
        log(f"cpu oracle: {sample / cpu_s:.0f} QPS on {threads} threads; ids identical on {same * 100:.2f}% "
            f"of the sample")

    # Side measurements (never `value`): the same data and queries on the
    # RNG-only graph (RNG-pruned k-NN edges, no random long links) and on the
    # connected graph (the same edges plus the links that make every node
    # reachable from the entry point), swept over the same beams.
    side = {}
    if args.config == "c2" and args.graph == "mixed" and not args.no_rng_graph and not use_ip:
        for sname, skw, sdesc in (
                ("rng_graph", dict(random_links=0, fill_random=False),
                 "RNG-pruned k-NN edges only (random_links=0, empty slots backfilled from the k-NN candidates)"),
                ("connected_graph", dict(random_links=0, fill_random=False, connect=True),
                 "RNG-pruned k-NN edges, empty slots backfilled from the k-NN candidates, then the links that make "
                 "every node reachable from the entry point (the unreached node nearest the entry linked from its "
                 "nearest reached node, into a backfilled or empty slot, repeated)")):
            t0 = time.time()
            sst = {}
            cb_r = builder.build_codebook(base, args.degree, signs, device=dev, stats=sst, **skw)
            log(f"{sname} built in {time.time() - t0:.1f}s" +
                (f" ({sst['connect_links']} links added)" if "connect_links" in sst else ""))
            ix_r = fg.Index.from_codebook(cb_r)
            oix_r = O.OracleIndex.from_codebook(cb_r) if oix is not None else None
            rows = []
            for beam in beams:
                for _ in range(4):
                    ix_r.search_device(dq.data_ptr(), args.nq, args.K, beam, dres.data_ptr(), 0, stream.cuda_stream)
                torch.cuda.synchronize()
                ms = []
                for _ in range(5):
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                    ix_r.search_device(dq.data_ptr(), args.nq, args.K, beam, dres.data_ptr(), 0, stream.cuda_stream)
                    e1.record(stream)
                    torch.cuda.synchronize()
                    ms.append(e0.elapsed_time(e1))
                rids = dres.cpu().numpy().view(np.uint32)
                row = {"beam": beam, "recall": round(float(recall_of(rids)), 5),
                       "qps": round(args.nq / (float(np.median(ms)) / 1e3), 1), "kernel_ms": round(float(np.median(ms)), 4)}
                if oix_r is not None and args.parity_sample > 0:
                    m = min(args.nq, args.parity_sample)
                    pids, _ = oix_r.search(queries[:m], args.K, beam, threads=threads)
                    row["oracle_ids_identical"] = float((pids == rids[:m]).all(1).mean())
                    row["oracle_sample"] = m
                rows.append(row)
                log(f"{sname}, beam {beam}: recall@{args.K} {row['recall']:.4f}, {row['qps']:.0f} QPS"
                    + (f", ids identical to the oracle on {row['oracle_ids_identical'] * 100:.2f}% of "
                       f"{row['oracle_sample']}" if "oracle_sample" in row else ""))
            first = next((r["beam"] for r in rows if r["recall"] >= args.target_recall), None)
            side[sname] = {"graph": sdesc, "beam_sweep": rows, "first_beam_reaching_target": first}
            if "connect_links" in sst:
                side[sname]["links_added"] = sst["connect_links"]
            ix_r.close()
            del cb_r, oix_r

    knn_desc = ("k-NN candidates searched in the 2 nearest of ~n/2500 k-means cells" if large
                else "exact k-NN candidates")
    graph_desc = (f"RNG-pruned k-NN edges only ({knn_desc}), empty slots backfilled from the candidates"
                  if args.graph == "rng" else
                  f"RNG-pruned k-NN edges ({knn_desc}), empty slots backfilled from the candidates, plus "
                  f"{build_stats.get('connect_links')} links that make every node reachable from the entry point"
                  if args.graph == "connected"
                  else f"RNG-pruned k-NN edges ({knn_desc}, {args.candidates or 2 * args.degree} per node"
                       + (f", alpha {args.alpha}" if args.alpha != 1.0 else "")
                       + f") plus {args.random_links if args.random_links >= 0 else args.degree // 4} seeded "
                       "random long links per node, empty slots to random targets")
    line = {
        "metric":("queries/sec at recall@100>=0.95 (1M x 128 fp32, deg 32)" if args.config == "c2" and not use_ip
                   else f"queries/sec at recall@{args.K}>={args.target_recall} ({args.n} x {dim} fp32, deg {args.degree}"
                        f"{', inner product' if use_ip else ''})"),
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
        "data": f"synthetic: seeded {conf['gen'].replace('_', ' ')} ({args.components} components"
                + (", drawn on the GPU" if large else "") + "), graph and codes built in-run",
        "config": {"workload": f"{args.config.upper()} {args.n}x{dim} deg {args.degree}, K={args.K}, nq={args.nq}, "
                               f"beam={chosen}" + (", inner product" if use_ip else ""),
                   "beam": chosen, "recall": round(float(recall), 5), "beam_sweep": sweep,
                   "single_search_ms": round(single_ms, 4), "single_search_qps": round(args.nq / single_ms * 1e3, 1),
                   "host_buffers_qps": round(host_qps, 1), "work_per_query": work, "serving": serving,
                   "lds_bytes": fg.lds_bytes(dim, chosen, args.degree),
                   "waves_per_query": index.search_waves(args.nq, args.K, chosen),
                   "launches_per_search": index.search_launches(args.nq, args.K, chosen), "graph": graph_desc,
                   "rng_graph": side.get("rng_graph"), "connected_graph": side.get("connected_graph")},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_source,
                     "measured_copy_gbs": round(copy_gbs, 1), "frac_of_measured_copy": round(achieved / copy_gbs, 4),
                     "kernel": "fg_search_kernel", "kernel_ms": round(kernel_ms, 4),
                     "algorithmic_bytes_per_launch": alg_bytes},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    index.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
