"""Throughput of the HIP openTSNE-style t-SNE gradient loop on one MI355X.

Workload: 1,000,000 x 50 float32 Gaussian mixture
(50 components, means ~ N(0, 6^2 I), unit std), exact KNN with k = 90
(computed on the GPU by the library's exact search, fastembedr_hip_knn_exact,
and handed to the P build in device memory; --config 4 runs the
4,000,000-row, 200-component case), perplexity 30, PCA
initialisation, and the reference schedule: 250 early-exaggeration
iterations (exaggeration 12, momentum 0.5) then 500 (momentum 0.8), learning
rate n / 12.  Repulsion (--repulsion): by default the FIt-SNE interpolation
grid with the configs' FFT settings (3 interpolation points per interval, at
least 50 intervals, one interval per unit of span: the late-phase layout
drives it to hundreds of intervals per axis); --repulsion grid runs the
reference's bilinear grid with its CPU policy (256 nodes per axis at this n).

A step is one gradient iteration (repulsion + attraction + update +
centring).  Inputs (P, layout, optimiser state) are resident in HBM before
the timed region; the P construction is timed separately.  After W untimed
warm-up iterations the state is reset to the initialisation and the timed
region runs the first K iterations of the schedule (K = 750 is the whole
run).  In the timed region the library runs the attraction and the kernel
spectrum on side streams beside the rest of each iteration.  The dominant
kernel's duration comes from HIP events recorded on the stream it runs on,
around each of its launches in the timed region; the other kernels run
without events.  A separate, untimed pass of the same K iterations runs the
kernels in sequence and brackets every one with events for the breakdown
(ms_per_repulsion_step sums the repulsion kernels of that pass).

Prints one JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=750)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--n", type=int, default=0, help="override the number of points (smaller smoke runs)")
    ap.add_argument("--grid", type=int, default=0, help="bilinear grid nodes per axis; 0 = reference CPU policy")
    ap.add_argument("--repulsion", choices=["interp", "grid"], default="interp",
                    help="interp: FIt-SNE interpolation grid with the configs' FFT settings (3 points per "
                         "interval, >= 50 intervals, one interval per unit); grid: the reference's bilinear grid")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--host-boundary", action="store_true",
                    help="also time the one-shot C-ABI call from host KNN buffers (PCIe and P build included)")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="run one device-to-device copy of this size first (counter calibration under rocprofv3)")
    return ap.parse_args()


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the t-SNE path is built and measured on a single MI355X "
              "(multi-GPU sharding is a design note, not part of this build).", file=sys.stderr)
        return 2

    import torch

    import fastembedr_amd as fe
    from fastembedr_amd import synthetic

    if not fe.available():
        log("no gfx950 device visible to the HIP backend")
        return 1
    if args.calibrate_copy_mib > 0:
        # A plain copy kernel of known size: its FETCH_SIZE / WRITE_SIZE under
        # rocprofv3 give the factor between counter units and bytes.
        src = torch.ones(args.calibrate_copy_mib * (1 << 18), dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: {src.numel() * 4} bytes read, {dst.numel() * 4} bytes written")
        del src, dst
    if args.config == 3:
        return bench_transform(args, torch, fe, synthetic)
    sched = synthetic.SCHEDULE
    spec = synthetic.CONFIGS[args.config]
    n = args.n or spec.n
    k = sched["k"]
    t0 = time.perf_counter()
    x, _ = synthetic.gaussian_mixture(spec, seed=1, n=n)
    log(f"data {x.shape} in {time.perf_counter() - t0:.1f}s")
    # exact KNN on the GPU with the library's own search; the result stays
    # in device memory and P is built from it there
    knn = fe.exact_knn(np.ascontiguousarray(x, dtype=np.float32), k, keep_device=True)
    log(f"exact KNN k={k} in {knn.elapsed_sec:.3f}s (fastembedr_hip_knn_exact, host input; {knn.stats})")
    y0 = synthetic.pca_init(x)

    sess = fe.TsneSession(perplexity=sched["perplexity"], index_offset=1, grid_size=args.grid, n=n, k=k,
                          device_pointers=(knn.indices_ptr, knn.distances_ptr))
    p_build_ms = sess.p_build_ms
    nnz = sess.nnz
    g = sess.grid_size
    interp = args.repulsion == "interp"
    if interp:
        from fastembedr_amd import _lib

        sess.set_repulsion(_lib.REPULSION_LAGRANGE, sched["interpolation_points"], sched["min_intervals"],
                           sched["ints_in_interval"])
    log(f"P build {p_build_ms:.1f} ms, nnz={nnz}, repulsion={args.repulsion}"
        + ("" if interp else f", grid={g}"))

    ee = sched["early_exaggeration_iter"]
    lr = n / 12.0

    def schedule_run(count: int) -> None:
        early = min(count, ee)
        if early:
            sess.run(early, sched["early_exaggeration"], sched["initial_momentum"], lr, sched["min_gain"],
                     sched["max_step_norm"])
        if count - early:
            sess.run(count - early, sched["exaggeration"], sched["final_momentum"], lr, sched["min_gain"],
                     sched["max_step_norm"])

    # warm-up (untimed), then reset to the initialisation
    sess.set_state(y0)
    sess.center()
    schedule_run(args.warmup)
    sess.sync()
    sess.set_state(y0)
    sess.center()
    sess.sync()

    # Breakdown pass (untimed): HIP events around every kernel give the
    # per-kernel durations and pick the dominant kernel.  In this pass the
    # library runs the iteration's kernels in sequence (no side streams), so
    # each duration is the kernel's alone; the timed pass below overlaps the
    # attraction and the kernel spectrum with the rest of the iteration.
    sess.set_timing(True)
    schedule_run(args.steps)
    sess.sync()
    breakdown = sess.timing()
    sess.set_timing(False)
    per_kernel = {name: (tot / cnt if cnt else 0.0) for name, (cnt, tot) in breakdown.items() if cnt}
    # The repulsion step: every kernel from the binning of the points to the
    # potentials on the grid (the read-back is fused into the update).
    rep_kernels = [kname for kname in per_kernel if kname.startswith("interp_")] if interp else \
        ["bin_count", "bin_plan", "bin_scatter", "spread", "kernel_rows", "kernel_cols", "charge_rows",
         "conv_cols", "inverse_rows"]
    rep_ms = sum(per_kernel[kname] for kname in rep_kernels)
    geo_end = sess.interp_info() if interp else None
    dom = max(breakdown, key=lambda kname: breakdown[kname][1])  # largest total time
    sess.set_state(y0)
    sess.center()
    sess.sync()

    # Timed region: events only around the dominant kernel, so that the other
    # launches run back to back as in an uninstrumented run.
    sess.set_timing(True, only=dom)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    schedule_run(args.steps)
    sess.sync()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    timing = sess.timing()
    sess.set_timing(False)
    y_final = sess.y
    if not np.all(np.isfinite(y_final)):
        log("non-finite layout after the timed region")
        return 1
    its = args.steps / wall
    ms_per_step = 1000.0 * wall / args.steps
    cnt, tot = timing[dom]
    dom_ms = tot / cnt if cnt else 0.0
    # Algorithmic bytes per launch.  attract: P streamed once (a 16-bit slot
    # word and the fp32 value per stored entry, 6 nnz), y_i read and the row
    # sum written (16 n); the neighbour positions y_j are counted as
    # cache-resident, as the grid reads are; bridge and padding slots are
    # overhead, not algorithmic bytes.  update: y_i, attraction, gains,
    # update read (32 n) and y, gains, update written (24 n).
    layout = sess.attraction_info()
    alg_bytes = {"attract": 6.0 * nnz + 16.0 * n, "update": 56.0 * n}
    dom_bytes = alg_bytes.get(dom, 0.0)
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9 if dom_ms > 0 else 0.0
    traffic = measured_traffic(dom, n, nnz, g, args.repulsion)
    log(f"{its:.1f} it/s, {ms_per_step:.3f} ms/step, repulsion {rep_ms:.3f} ms, {dom} {dom_ms:.3f} ms "
        f"({achieved:.0f} GB/s)")
    log("per-kernel ms (breakdown pass, every kernel bracketed by events): "
        + ", ".join(f"{kk}={v:.4f}" for kk, v in per_kernel.items()))

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(sess, y0, n, lr, sched, args.cpu_seconds, interp)
    sess.close()
    host_boundary = None
    if args.host_boundary:
        host_knn = knn.to_host()
        host_boundary = one_shot_from_host(np.asfortranarray(host_knn.indices), np.asfortranarray(host_knn.distances),
                                           y0, sched, lr)

    line = {
        "metric": "t-SNE gradient iterations/sec at N=1M (2D); ms per FFT repulsion step; % HBM peak",
        "value": round(its, 3),
        "unit": "iterations/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"config{args.config}: {n} x 50 Gaussian mixture ({spec.components} components), "
                        f"exact KNN k={k}, perplexity 30, 250 early-exaggeration + 500 iterations, "
                        f"PCA init, "
                        + ("FIt-SNE interpolation grid (3 points per interval, >= 50 intervals, "
                           "1 interval per unit of span)" if interp else
                           f"bilinear grid {g}x{g} ({'reference CPU policy' if args.grid == 0 else 'explicit'})"),
            "n": n,
            "knn": {"engine": "fastembedr_hip_knn_exact (exact, certified)", "seconds": round(knn.elapsed_sec, 4),
                    "tiles_computed_per_32_queries": round(knn.stats["tiles_computed"] / ((n + 31) // 32), 1),
                    "tiles": (n + 63) // 64},
            "k": k,
            "nnz": nnz,
            "attraction_layout": {"runs": layout["tiles"], "slots": layout["slots"],
                                  "slots_per_entry": round(layout["slots"] / max(nnz, 1), 4)},
            "repulsion": args.repulsion,
            "timed_iterations": f"first {args.steps} of the 750-iteration schedule",
        },
        "ms_per_repulsion_step": round(rep_ms, 4),
        "repulsion_kernels": rep_kernels,
        "p_build_ms": round(p_build_ms, 2),
        "per_kernel_ms": {kk: round(v, 5) for kk, v in per_kernel.items()},
        "roofline": {
            "kernel": dom,
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "algorithmic_bytes": int(dom_bytes),
            "traffic_source": TRAFFIC_FILES[args.repulsion].name if traffic is not None else None,
        },
        "cpu_baseline": cpu,
        "host_boundary": host_boundary,
    }
    if interp:
        line["config"]["interp_grid_at_end"] = {"boxes_per_axis": geo_end["boxes"],
                                                "nodes_per_axis": geo_end["nodes"],
                                                "fft_len": geo_end["fft_len"]}
    else:
        line["config"]["grid_nodes_per_axis"] = g
    print(json.dumps(line), flush=True)
    return 0


def bench_transform(args, torch, fe, synthetic) -> int:
    """Config 3: fixed-reference transform.  Reference: the config-1 mixture
    (70,000 x 50) embedded on the GPU with the full schedule; queries:
    100,000 new points of the same mixture with exact k = 30 neighbours in
    the reference; transform_tsne defaults except exaggeration 1 (perplexity
    5, 250 iterations, learning rate 0.1, momentum 0.8, gradient clip 0.25,
    median initialisation, 256 sampled negatives per query and iteration).
    The per-iteration rate is taken from two calls (all iterations, and one)
    so that upload, P and initialisation drop out."""
    import ctypes as C

    from fastembedr_amd import _lib

    spec = synthetic.CONFIGS[1]
    n_ref = args.n or spec.n
    nq = 100_000 if not args.n else max(1, args.n // 2)
    x, _ = synthetic.gaussian_mixture(spec, seed=1, n=n_ref + nq)
    xr, xq = x[:n_ref], x[n_ref:]
    sched = synthetic.SCHEDULE
    ref_knn = fe.exact_knn(np.ascontiguousarray(xr, dtype=np.float32), sched["k"], keep_device=True)
    with fe.TsneSession(perplexity=sched["perplexity"], index_offset=1, n=n_ref, k=sched["k"],
                        device_pointers=(ref_knn.indices_ptr, ref_knn.distances_ptr)) as sess:
        sess.set_state(synthetic.pca_init(xr))
        sess.center()
        lr = n_ref / 12.0
        sess.run(sched["early_exaggeration_iter"], sched["early_exaggeration"], sched["initial_momentum"], lr,
                 sched["min_gain"], sched["max_step_norm"])
        sess.run(sched["n_iter"], sched["exaggeration"], sched["final_momentum"], lr, sched["min_gain"],
                 sched["max_step_norm"])
        ref_layout = np.asarray(sess.y, np.float64)
    del ref_knn
    qknn = fe.exact_query_knn(np.ascontiguousarray(xr, dtype=np.float32), np.ascontiguousarray(xq, dtype=np.float32),
                              30)
    log(f"reference layout {ref_layout.shape}, query KNN {qknn.indices.shape} in {qknn.elapsed_sec:.3f}s "
        f"(fastembedr_hip_knn_query)")
    lib = _lib.load()
    ref_cm = np.asfortranarray(ref_layout)
    qi = np.asfortranarray(qknn.indices, dtype=np.int32)
    qd = np.asfortranarray(qknn.distances, dtype=np.float64)
    out = np.empty((nq, 2), np.float64, order="F")
    params = dict(perplexity=5.0, early_iter=0, lr=0.1, early_ex=4.0, ex=1.0, m0=0.8, m1=0.8, gmax=0.25,
                  smax=float("inf"), n_neg=256, thr=4096, seed=4)

    def call(iters: int) -> float:
        exact = C.c_int(0)
        t0 = time.perf_counter()
        rc = lib.fastembedr_hip_transform_tsne(
            ref_cm.ctypes.data_as(C.c_void_p), n_ref, qi.ctypes.data_as(C.c_void_p), qd.ctypes.data_as(C.c_void_p),
            nq, 30, None, 0, params["perplexity"], iters, params["early_iter"], params["lr"], params["early_ex"],
            params["ex"], params["m0"], params["m1"], params["gmax"], params["smax"], params["n_neg"],
            params["thr"], params["seed"], out.ctypes.data_as(C.c_void_p), C.byref(exact))
        _lib.check(rc, "transform")
        return time.perf_counter() - t0

    call(2)  # warm-up
    iters = args.steps if args.steps != 750 else 250
    t_all = call(iters)
    t_one = call(1)
    per_iter = (t_all - t_one) / max(1, iters - 1)
    its = 1.0 / per_iter
    log(f"transform: {iters} iterations in {t_all:.3f}s, 1 in {t_one:.3f}s -> {its:.1f} it/s "
        f"({per_iter * 1e3:.3f} ms per iteration over {nq} queries)")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle

        threads = min(16, os.cpu_count() or 1)
        sample_q = min(nq, 20_000)
        t0 = time.perf_counter()
        oracle.transform_run(ref_layout, qi[:sample_q], qd[:sample_q], n_iter=1, perplexity=5.0, exaggeration=1.0,
                             n_negatives=256, exact_threshold=4096, seed=4, threads=threads)
        t1 = time.perf_counter() - t0
        cpu_iters = 10
        t0 = time.perf_counter()
        oracle.transform_run(ref_layout, qi[:sample_q], qd[:sample_q], n_iter=cpu_iters + 1, perplexity=5.0,
                             exaggeration=1.0, n_negatives=256, exact_threshold=4096, seed=4, threads=threads)
        t_cpu = (time.perf_counter() - t0 - t1) / cpu_iters * (nq / sample_q)
        cpu = {"value": round(1.0 / t_cpu, 3), "unit": "iterations/s", "cores": threads, "kind": "port",
               "sample": f"{cpu_iters} iterations over {sample_q} of the {nq} queries, scaled to all queries"}
        log(f"CPU oracle transform: {1.0 / t_cpu:.2f} it/s (scaled) on {threads} threads")
    line = {
        "metric": "t-SNE transform iterations/sec (config 3: 100K queries against a fixed 70K reference)",
        "value": round(its, 3), "unit": "iterations/s", "n_gpus": 1, "steps": iters, "warmup": 2,
        "ms_per_step": round(per_iter * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f64", "data": "synthetic",
        "config": {"workload": f"config3: {nq} queries, reference {n_ref} (config-1 mixture embedded on the GPU), "
                               f"k=30, perplexity 5, 256 sampled negatives, lr 0.1, exaggeration 1",
                   "n_reference": n_ref, "n_query": nq, "k": 30},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def one_shot_from_host(idx_r, dist_r, y0, sched, lr):
    """The reference-shaped one-shot call (fastembedr_hip_opentsne_fft_from_knn_float)
    on host column-major KNN and a host initialisation: upload, P build, the
    whole 750-iteration schedule and the download of the layout, timed from
    the host.  Reported beside `value`, never as it."""
    import ctypes as C

    from fastembedr_amd import _lib

    lib = _lib.load()
    n, k = idx_r.shape
    init = np.ascontiguousarray(y0, np.float32)
    out = np.empty((n, 2), np.float32)
    args = (idx_r.ctypes.data_as(C.c_void_p), dist_r.ctypes.data_as(C.c_void_p), init.ctypes.data_as(C.c_void_p),
            1, n, k, 2, sched["perplexity"], sched["early_exaggeration_iter"], sched["n_iter"],
            sched["early_exaggeration"], sched["exaggeration"], lr, 0, sched["initial_momentum"],
            sched["final_momentum"], sched["min_gain"], sched["max_step_norm"], 1, 1,
            out.ctypes.data_as(C.c_void_p))
    t0 = time.perf_counter()
    _lib.check(lib.fastembedr_hip_opentsne_fft_from_knn_float(*args), "one-shot call")
    dt = time.perf_counter() - t0
    total = sched["early_exaggeration_iter"] + sched["n_iter"]
    log(f"one-shot from host buffers: {dt:.3f}s for {total} iterations ({total / dt:.1f} it/s incl. upload + P)")
    return {"seconds": round(dt, 4), "iterations": total, "iterations_per_s": round(total / dt, 3),
            "includes": "host->device KNN copy, P build, 750 iterations, device->host layout copy"}


TRAFFIC_FILES = {"grid": ROOT / "profiles" / "tsne_loop_config2_traffic.json",
                 "interp": ROOT / "profiles" / "tsne_loop_config2_interp_traffic.json"}


def measured_traffic(kernel: str, n: int, nnz: int, g: int, repulsion: str):
    """HBM bytes per launch of `kernel` (FETCH_SIZE + WRITE_SIZE, calibrated
    against a copy of known size) from the committed rocprofv3 digest, when
    that digest was taken on this same workload; None otherwise."""
    try:
        rec = json.loads(TRAFFIC_FILES[repulsion].read_text())
    except (OSError, ValueError):
        return None
    if (rec.get("n"), rec.get("nnz"), rec.get("repulsion")) != (n, nnz, repulsion):
        return None
    if repulsion == "grid" and rec.get("grid") != g:
        return None
    # the timer's name is the kernel symbol's stem: "attract" is k_attract or
    # the tiled k_attract_tiles_seg<NT>, "update" k_update<mode, grid>
    for name, t in rec.get("kernels", {}).items():
        if name.split("<")[0].startswith("k_" + kernel):
            return int(t["fetch_bytes"] + t["write_bytes"])
    return None


def cpu_baseline(sess, y0, n, lr, sched, budget_s, interp):
    """The CPU oracle (a restatement of the reference CPU path) on the same P
    and initialisation, timed on this host's cores for a bounded number of
    early-exaggeration iterations (gradient + update + centring), with the
    same repulsion as the timed GPU run."""
    from oracle import oracle

    threads = min(16, os.cpu_count() or 1)
    method = oracle.METHOD_LAGRANGE if interp else oracle.METHOD_GRID
    P = oracle.OracleP.wrap(*sess.csr())
    y = np.array(y0, np.float32, copy=True)
    oracle.zero_mean(y)
    t0 = time.perf_counter()
    y, _, _ = P.optimize(y, 1, 0, sched["early_exaggeration"], 1.0, lr, False, sched["initial_momentum"],
                         sched["final_momentum"], method=method, threads=threads)
    one = time.perf_counter() - t0
    iters = max(1, min(400, int(budget_s / max(one, 1e-3))))
    t0 = time.perf_counter()
    P.optimize(y, iters, 0, sched["early_exaggeration"], 1.0, lr, False, sched["initial_momentum"],
               sched["final_momentum"], method=method, threads=threads)
    dt = time.perf_counter() - t0
    log(f"CPU oracle: {iters} iterations in {dt:.1f}s on {threads} threads")
    rep = ("FIt-SNE interpolation grid (fp64 restatement: 3 points per interval, >= 50 intervals)" if interp
           else "reference CPU grid policy")
    return {
        "value": round(iters / dt, 4),
        "unit": "iterations/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{iters} early-exaggeration iterations (after 1 untimed) of the same n={n} problem, "
                  f"same P and initialisation, {rep}",
    }


if __name__ == "__main__":
    sys.exit(main())
