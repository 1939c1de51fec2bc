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
the timed region; the P construction is timed separately.  With --steps K
the timed region is the LAST K iterations of the 750-iteration schedule
(the late phase, where the layout's span and so the interpolation grid are
largest): the first 750 - K iterations run untimed before it; K = 750 times
the whole schedule.  Passes, in order (so that the last dispatches of every
kernel belong to the timed window, which rocprof digests rely on):
  1. W untimed warm-up iterations, then a reset to the initialisation;
  2. the whole schedule timed from the host without events
     (full_schedule: its mean rate);
  3. the window with HIP events around every kernel, which runs the
     kernels in sequence (the per-kernel breakdown);
  4. the window run in sequence again with one pair of events around the
     repulsion step's kernels only (ms_per_repulsion_step: the step alone,
     without the per-kernel events' overhead);
  5. the window timed (value), with events only around the dominant kernel,
     on the stream it runs on, on every DOM_EVERY-th iteration (an event's
     marker delays the launch behind it); the library runs the attraction
     and the kernel spectrum on side streams beside the rest of each
     iteration.
The CPU baseline runs the oracle, a restatement of the reference's CPU
algorithm (bilinear grid, CPU grid policy), from the layout at the start of
the window.

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
# The timed window brackets the dominant kernel with HIP events on every
# DOM_EVERY-th iteration only (with a 20-step window: 5 launches timed).
DOM_EVERY = 4


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
    ap.add_argument("--host-boundary", action=argparse.BooleanOptionalAction, default=True,
                    help="also time the one-shot C-ABI call from host KNN buffers (PCIe and P build included; "
                         "on by default, reported beside `value`)")
    ap.add_argument("--fft-sweep", action="store_true",
                    help="instead of the bench line: the interpolation grid's repulsion kernels at FFT lengths "
                         "768 ... 4096, the converged config-2 layout scaled until it needs them (one JSON line)")
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

    total = sched["early_exaggeration_iter"] + sched["n_iter"]
    steps = max(1, min(args.steps, total))
    head = total - steps  # untimed iterations before the timed window
    ee = sched["early_exaggeration_iter"]
    lr = n / 12.0

    def schedule_run(start: int, end: int) -> None:
        """Iterations [start, end) of the two-phase schedule."""
        early = max(0, min(end, ee) - start)
        if early:
            sess.run(early, sched["early_exaggeration"], sched["initial_momentum"], lr, sched["min_gain"],
                     sched["max_step_norm"])
        late = end - max(start, ee)
        if late > 0:
            sess.run(late, sched["exaggeration"], sched["final_momentum"], lr, sched["min_gain"],
                     sched["max_step_norm"])

    def reset() -> None:
        sess.set_state(y0)
        sess.center()
        sess.sync()

    # 1. warm-up (untimed), then reset to the initialisation
    reset()
    schedule_run(0, args.warmup)
    sess.sync()

    # 2. the whole schedule, timed from the host (no events)
    reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    schedule_run(0, total)
    sess.sync()
    torch.cuda.synchronize()
    full_wall = time.perf_counter() - t0
    log(f"whole schedule: {total} iterations in {full_wall:.3f}s = {total / full_wall:.1f} it/s")

    if args.fft_sweep:
        return fft_sweep(sess, n, nnz, sched, lr, log)

    # 3. breakdown pass over the window: HIP events around every kernel give
    # the per-kernel durations and pick the dominant kernel.  In this pass
    # the library runs the iteration's kernels in sequence (no side streams),
    # so each duration is the kernel's alone.
    reset()
    schedule_run(0, head)
    sess.sync()
    y_window = sess.y  # the layout at the start of the window (CPU baseline input)
    sess.set_timing(True)
    schedule_run(head, total)
    sess.sync()
    breakdown = sess.timing()
    sess.set_timing(False)
    # milliseconds per iteration of the window: a kernel launched every
    # iteration counts its average duration, one launched every few
    # iterations (the interpolation grid's spread order) its share
    per_kernel = {name: tot / steps for name, (cnt, tot) in breakdown.items() if cnt}
    # The repulsion step: every kernel from the binning of the points to the
    # potentials on the grid (the read-back is fused into the update).
    rep_kernels = [kname for kname in per_kernel if kname.startswith("interp_")] if interp else \
        [kname for kname in ("bin_count", "bin_plan", "bin_scatter", "spread", "kernel_rows", "kernel_cols",
                             "charge_rows", "conv_cols", "inverse_rows") if kname in per_kernel]
    rep_sum_ms = sum(per_kernel[kname] for kname in rep_kernels)
    dom = max(breakdown, key=lambda kname: breakdown[kname][1])  # largest total time

    # 3b. the repulsion step's span: the window in sequence again, with one
    # pair of events around the step's kernels (kernel spectrum to
    # potentials) instead of a pair around each of them
    reset()
    schedule_run(0, head)
    sess.sync()
    sess.set_timing(True, only="repulsion")
    schedule_run(head, total)
    sess.sync()
    span_cnt, span_tot = sess.timing()["repulsion"]
    sess.set_timing(False)
    rep_ms = span_tot / span_cnt if span_cnt else rep_sum_ms

    # 4. the timed window: events only around the dominant kernel, and only
    # on every DOM_EVERY-th iteration (an event's marker delays the launch
    # behind it by ~5 us), so that the other launches run back to back as in
    # an uninstrumented run; the kernel's duration is the mean over the
    # bracketed launches.
    reset()
    schedule_run(0, head)
    sess.sync()
    sess.set_timing(True, only=dom, every=DOM_EVERY)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    schedule_run(head, total)
    sess.sync()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    timing = sess.timing()
    sess.set_timing(False)
    geo_end = sess.interp_info() if interp else None
    y_final = sess.y
    if not np.all(np.isfinite(y_final)):
        log("non-finite layout after the timed region")
        return 1
    its = steps / wall
    ms_per_step = 1000.0 * wall / steps
    cnt, tot = timing[dom]
    dom_ms = tot / cnt if cnt else 0.0
    layout = sess.attraction_info()
    # Algorithmic bytes per launch (the CSR basis).  attract: col int32 +
    # val fp32 streamed once per stored entry and the row pointers,
    # 8 nnz + 4 (n + 1); the neighbour positions y_j are counted as
    # cache-resident.  The kernel's own slot format moves 6 bytes per entry
    # (a 16-bit slot word + the fp32 value) plus 16 n (y_i read, row sum
    # written): reported beside it.  update: y_i, attraction, gains, update
    # read (32 n) and y, gains, update written (24 n).
    alg_bytes = {"attract": 8.0 * nnz + 4.0 * (n + 1), "update": 56.0 * n}
    dom_bytes = alg_bytes.get(dom, 0.0)
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9 if dom_ms > 0 else 0.0
    slot_bytes = 6.0 * nnz + 16.0 * n
    traffic = measured_traffic(dom, n, nnz, g, args.repulsion)
    digest = _digest(n, nnz, g, args.repulsion)
    traffic_source = digest["_file"] if traffic is not None and digest is not None else None
    # The repulsion step's roofline: B_rep = 16 n + 8 n
    # + 28 G^2 + 288 F^2 with G the grid nodes per axis and F the FFT length
    # at the end of the window, over the repulsion step's span in sequence
    # (pass 3b); traffic: the rocprof digest's bytes of the same kernels
    # per iteration.
    if interp:
        # the shortest FFT length the grid can use (2^a or 3 * 2^a, at least
        # 64, zero padding to >= 2 nodes); the run may use a longer one,
        # chosen from a lagged bound
        g_nodes = geo_end["nodes"]
        f_len = 64
        while f_len < 2 * g_nodes:
            f_len = f_len // 2 * 3 if f_len & (f_len - 1) == 0 else f_len // 3 * 4
    else:
        g_nodes, f_len = g, 2 * g
    rep_bytes = 24.0 * n + 28.0 * g_nodes ** 2 + 288.0 * f_len ** 2
    rep_alg = rep_bytes / (rep_ms * 1e-3) / 1e9 if rep_ms > 0 else 0.0
    rep_traffic = repulsion_traffic(n, nnz, g, args.repulsion)
    # measured: the digest's HBM bytes (FETCH_SIZE + WRITE_SIZE) over the
    # same time; null without a digest of this workload
    rep_measured = rep_traffic / (rep_ms * 1e-3) / 1e9 if rep_traffic and rep_ms > 0 else None
    dom_measured = traffic / (dom_ms * 1e-3) / 1e9 if traffic and dom_ms > 0 else None
    log(f"{its:.1f} it/s over iterations {head}-{total - 1}, {ms_per_step:.3f} ms/step, repulsion {rep_ms:.3f} ms "
        f"({rep_alg:.0f} GB/s on B_rep"
        + (f", {rep_measured:.0f} GB/s measured" if rep_measured else "")
        + f"), {dom} {dom_ms:.3f} ms ({achieved:.0f} GB/s"
        + (f", {dom_measured:.0f} GB/s measured" if dom_measured else "") + ")")
    log("per-kernel ms per iteration (breakdown pass, every kernel bracketed by events): "
        + ", ".join(f"{kk}={v:.4f}" for kk, v in per_kernel.items()))

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(sess, y_window, n, lr, sched, args.cpu_seconds, head)
    sess.close()
    host_boundary = None
    if args.host_boundary:
        host_knn = knn.to_host()
        host_boundary = one_shot_from_host(np.asfortranarray(host_knn.indices), np.asfortranarray(host_knn.distances),
                                           y0, sched, lr)

    window = (f"last {steps} of the {total}-iteration schedule (iterations {head}-{total - 1}; the first {head} "
              f"run untimed before the timed region)" if head else f"the whole {total}-iteration schedule")
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
            "timed_iterations": window,
        },
        "full_schedule": {"iterations": total, "iterations_per_s": round(total / full_wall, 3),
                          "ms_per_step": round(1000.0 * full_wall / total, 4),
                          "note": "whole 750-iteration schedule timed from the host, no events"},
        "ms_per_repulsion_step": round(rep_ms, 4),
        "repulsion_step_basis": "the step's kernels run in sequence, one pair of HIP events around them all, "
                                "mean over the window's iterations",
        "repulsion_kernels_summed_ms": round(rep_sum_ms, 4),
        "repulsion_kernels": rep_kernels,
        "repulsion_roofline": {
            "bound": "hbm",
            "achieved": round(rep_measured, 1) if rep_measured else None,
            "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(rep_measured / HBM_PEAK_GBS, 4) if rep_measured else None,
            "traffic": rep_traffic,
            "basis": "measured: the traffic digest's FETCH_SIZE + WRITE_SIZE bytes of the repulsion kernels per "
                     "iteration over ms_per_repulsion_step (the repulsion step in sequence)",
            "algorithmic": {
                "bytes": int(rep_bytes), "achieved": round(rep_alg, 1), "frac": round(rep_alg / HBM_PEAK_GBS, 4),
                "basis": f"B_rep = 24 n + 28 G^2 + 288 F^2 with G = {g_nodes} nodes per axis, F = {f_len}; it "
                         f"counts every FFT pass as an HBM round trip, which the LDS transforms avoid"}},
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
            "basis": "attract: 8 nnz + 4 (n + 1) (col int32 + val fp32 + row_ptr) over the kernel's mean "
                     "event-timed duration in the timed window" if dom == "attract" else "see per-kernel bytes",
            "launches_timed": int(cnt),
            "timed_every": DOM_EVERY,
            "slot_basis": {"bytes": int(slot_bytes), "achieved": round(slot_bytes / (dom_ms * 1e-3) / 1e9, 1)
                           if dom_ms > 0 else 0.0,
                           "note": "the tiled kernel's own format: 6 bytes per stored entry + 16 n"}
            if dom == "attract" else None,
            "kernel_ms": round(dom_ms, 5),
            "traffic_source": traffic_source,
            # the same duration over the measured traffic
            "measured_achieved": round(dom_measured, 1) if dom_measured else None,
            "measured_frac": round(dom_measured / HBM_PEAK_GBS, 4) if dom_measured else None,
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


def fft_sweep(sess, n, nnz, sched, lr, log) -> int:
    """The repulsion kernels at large FFT lengths on a real 1M-point layout:
    the converged layout (the schedule just run) scaled by s, so that its
    span needs s times the boxes.  Per scale, 20 iterations at learning rate
    0 (the layout does not move) with every kernel timed alone by events,
    then 20 more with one pair of events around the repulsion step's kernels
    (ms_per_repulsion_step, as in the main line); the step clip is off, so
    the host sizes each iteration's FFT from that iteration's own box count
    (the shortest length that holds the grid)."""
    y_end = np.asarray(sess.y, np.float64)
    y_end -= y_end.mean(axis=0)
    cases = []
    for scale in (1.0, 2.8, 4.2, 5.6):
        sess.set_state((y_end * scale).astype(np.float32))
        sess.center()
        sess.sync()
        sess.set_timing(True)
        sess.run(20, sched["exaggeration"], sched["final_momentum"], 0.0, sched["min_gain"], 0.0)
        sess.sync()
        br = sess.timing()
        sess.set_timing(False)
        info = sess.interp_info()
        per = {name: tot / 20 for name, (cnt, tot) in br.items() if cnt and name.startswith("interp_")}
        rep_sum = sum(per.values())
        sess.set_timing(True, only="repulsion")
        sess.run(20, sched["exaggeration"], sched["final_momentum"], 0.0, sched["min_gain"], 0.0)
        sess.sync()
        span_cnt, span_tot = sess.timing()["repulsion"]
        sess.set_timing(False)
        rep = span_tot / span_cnt if span_cnt else rep_sum
        cases.append({"scale": scale, "boxes_per_axis": info["boxes"], "nodes_per_axis": info["nodes"],
                      "fft_len": info["fft_len"], "ms_per_repulsion_step": round(rep, 4),
                      "repulsion_kernels_summed_ms": round(rep_sum, 4),
                      "per_kernel_ms": {kk: round(v, 5) for kk, v in per.items()}})
        log(f"scale {scale}: {info['boxes']} boxes, {info['nodes']} nodes, FFT {info['fft_len']}: repulsion "
            f"{rep:.3f} ms in sequence ({rep_sum:.3f} one by one: "
            f"{', '.join(f'{kk}={v:.4f}' for kk, v in per.items())})")
    print(json.dumps({"metric": "interpolation-grid repulsion step at large FFT lengths (ms, kernels in sequence)",
                      "n": n, "nnz": nnz, "data": "synthetic (config 2, converged layout scaled)",
                      "cases": cases}), flush=True)
    return 0


def bench_transform(args, torch, fe, synthetic) -> int:
    """Config 3: fixed-reference transform.  Reference: the config-1 data
    (70,000 x 50) embedded on the GPU with the full schedule (FIt-SNE grid);
    queries: 100,000 new points of the same mixture
    (synthetic.mixture_queries) with exact k = 30 neighbours in the
    reference; transform_tsne defaults except exaggeration 1 (perplexity 5,
    250 iterations, learning rate 0.1, momentum 0.8, gradient clip 0.25,
    median initialisation).  Repulsion: the reference's transform_tsne_cpp
    mode, 256 sampled negatives per query and iteration.
    The per-iteration rate is taken from two calls (all iterations, and one)
    so that upload, P and initialisation drop out."""
    import ctypes as C

    from fastembedr_amd import _lib

    spec = synthetic.CONFIGS[1]
    n_ref = args.n or spec.n
    nq = 100_000 if not args.n else max(1, args.n // 2)
    xr, _ = synthetic.gaussian_mixture(spec, seed=1, n=n_ref)
    xq = synthetic.mixture_queries(spec, nq)
    sched = synthetic.SCHEDULE
    ref_knn = fe.exact_knn(np.ascontiguousarray(xr, dtype=np.float32), sched["k"], keep_device=True)
    with fe.TsneSession(perplexity=sched["perplexity"], index_offset=1, n=n_ref, k=sched["k"],
                        device_pointers=(ref_knn.indices_ptr, ref_knn.distances_ptr)) as sess:
        from fastembedr_amd import _lib as lib_

        sess.set_repulsion(lib_.REPULSION_LAGRANGE, sched["interpolation_points"], sched["min_intervals"],
                           sched["ints_in_interval"])
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
    grid_settings = (3, 50, 0.5)  # points per box, min boxes, box width (the grid transform's defaults)
    grid_stats = (C.c_longlong * 3)()

    def call(iters: int, mode: str) -> float:
        t0 = time.perf_counter()
        if mode == "grid":
            rc = lib.fastembedr_hip_transform_tsne_grid(
                ref_cm.ctypes.data_as(C.c_void_p), n_ref, qi.ctypes.data_as(C.c_void_p),
                qd.ctypes.data_as(C.c_void_p), nq, 30, None, 0, params["perplexity"], iters, params["early_iter"],
                params["lr"], params["early_ex"], params["ex"], params["m0"], params["m1"], params["gmax"],
                params["smax"], params["seed"], *grid_settings, out.ctypes.data_as(C.c_void_p), grid_stats)
        else:
            exact = C.c_int(0)
            rc = lib.fastembedr_hip_transform_tsne(
                ref_cm.ctypes.data_as(C.c_void_p), n_ref, qi.ctypes.data_as(C.c_void_p),
                qd.ctypes.data_as(C.c_void_p), nq, 30, None, 0, params["perplexity"], iters, params["early_iter"],
                params["lr"], params["early_ex"], params["ex"], params["m0"], params["m1"], params["gmax"],
                params["smax"], params["n_neg"], params["thr"], params["seed"], out.ctypes.data_as(C.c_void_p),
                C.byref(exact))
        _lib.check(rc, f"transform ({mode})")
        return time.perf_counter() - t0

    iters = args.steps if args.steps != 750 else 250
    exact_full = []  # query-iterations that took the exact sums, per full grid call

    def rate(mode: str) -> tuple[float, float, float]:
        """Per-iteration time from calls of `iters` and of 1 iteration (upload,
        P, initialisation and, for the grid, the node fields drop out); the
        median of 5 pairs."""
        call(2, mode)  # warm-up
        diffs, t_alls = [], []
        for _ in range(5):
            t_all = call(iters, mode)
            if mode == "grid":
                exact_full.append(int(grid_stats[2]))
            t_one = call(1, mode)
            diffs.append((t_all - t_one) / max(1, iters - 1))
            t_alls.append(t_all)
        per_iter = float(np.median(diffs))
        log(f"transform ({mode}): {iters} iterations in {np.median(t_alls):.4f}s (whole call) -> "
            f"{1.0 / per_iter:.1f} it/s ({per_iter * 1e3:.4f} ms per iteration over {nq} queries)")
        return per_iter, float(np.median(t_alls)), 1.0 / per_iter

    per_iter, t_call, its = rate("grid")
    geo = [int(v) for v in grid_stats]
    geo[2] = max(exact_full) if exact_full else geo[2]
    per_iter_s, t_call_s, its_s = rate("sampled")
    # fp64 flops per query and iteration of the fused run kernel (grid mode):
    # attraction 13 per neighbour (2 sub, 2 mul + 2 add, 1 div, 2 mul, 2 x
    # (mul + add)); interpolation 88 (box location 4, weights 18, 9 nodes x 7,
    # quotient 3); update 25.
    flops_q = 13 * 30 + 88 + 25
    tflops = flops_q * nq / per_iter / 1e12
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle

        threads = cpu_share()
        sample_q = min(nq, 20_000)

        def cpu_rate(run, label):
            t0 = time.perf_counter()
            run(1)
            t1 = time.perf_counter() - t0
            cpu_iters = 10
            t0 = time.perf_counter()
            run(cpu_iters + 1)
            t_cpu = (time.perf_counter() - t0 - t1) / cpu_iters * (nq / sample_q)
            log(f"CPU oracle transform ({label}): {1.0 / t_cpu:.2f} it/s (scaled) on {threads} threads")
            return round(1.0 / t_cpu, 3), cpu_iters

        v_s, n_s = cpu_rate(lambda it: oracle.transform_run(
            ref_layout, qi[:sample_q], qd[:sample_q], n_iter=it, perplexity=5.0, exaggeration=1.0, n_negatives=256,
            exact_threshold=4096, seed=4, threads=threads), "sampled, the reference's algorithm")
        cpu = {"value": v_s, "unit": "iterations/s", "cores": threads, "kind": "port",
               "sample": f"{n_s} iterations over {sample_q} of the {nq} queries, scaled to all queries; the "
                         f"reference's CPU transform (transform_tsne_cpp, 256 sampled negatives) restated by the "
                         f"oracle",
               "cpu_model": cpu_model(), "host_cpus_visible": os.cpu_count()}
    line = {
        "metric": "t-SNE transform iterations/sec (config 3: 100K queries against a fixed 70K reference)",
        "value": round(its, 3), "unit": "iterations/s", "n_gpus": 1, "steps": iters, "warmup": 2,
        "ms_per_step": round(per_iter * 1e3, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f64", "data": "synthetic",
        "config": {"workload": f"config3: {nq} queries, reference {n_ref} (config-1 mixture embedded on the GPU), "
                               f"k=30, perplexity 5, lr 0.1, exaggeration 1, {iters} iterations",
                   "n_reference": n_ref, "n_query": nq, "k": 30,
                   "repulsion": f"reference grid: the reference's repulsion fields summed once at {geo[1]} x "
                                f"{geo[1]} nodes ({geo[0]} boxes per axis, 3 points per box, 2 boxes per unit) and "
                                f"interpolated at each query; at most {geo[2]} query-iterations of a {iters}-iteration call took the exact sums"},
        "whole_call_seconds": round(t_call, 4),
        # the whole call (upload, device checks, P, initialisation, node
        # fields, every iteration, download) per iteration
        "whole_call_iterations_per_s": round(iters / t_call, 1),
        "roofline": {"kernel": "k_transform_run<grid>", "bound": "fp64 VALU", "achieved": round(tflops, 3),
                     "peak": 78.6, "unit": "TFLOP/s", "frac": round(tflops / 78.6, 4), "traffic": None,
                     "algorithmic_flops_per_query_iteration": flops_q},
        "sampled_mode": {"iterations_per_s": round(its_s, 3), "ms_per_step": round(per_iter_s * 1e3, 5),
                         "whole_call_seconds": round(t_call_s, 4),
                         "repulsion": "256 reference points sampled per query and iteration (transform_tsne_cpp's "
                                      "mode for n_reference > 4096)"},
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


# Committed traffic digests per repulsion; the one taken on the workload being
# measured (same n, nnz and grid) is used.
TRAFFIC_FILES = {"grid": [ROOT / "profiles" / "tsne_loop_config2_grid_traffic.json"],
                 "interp": [ROOT / "profiles" / "tsne_loop_config2_interp_traffic.json",
                            ROOT / "profiles" / "tsne_loop_config4_interp_traffic.json"]}

# Kernels of the repulsion step.  Every one runs once per iteration except the
# interpolation grid's spread order (k_lg_order_keys and the rocPRIM radix
# sort behind it, the only rocPRIM launches of the timed window), which runs
# every few iterations: its bytes count per iteration from its dispatches in
# the digest's window.
REPULSION_SYMBOLS = {
    "interp": ("k_lg_order_keys", "rocprim:", "k_lg_spread", "k_lg_kernel_rows", "k_lg_kernel_cols",
               "k_lg_box_chunks", "k_lg_charge_rows", "k_lg_conv_cols", "k_lg_inverse_rows", "k_lg_finalize_z"),
    "grid": ("k_bin_count", "k_bin_plan", "k_bin_scatter", "k_spread_tiles", "k_kernel_rows", "k_kernel_cols",
             "k_charge_rows", "k_conv_cols", "k_inverse_rows", "k_finalize_sumq"),
}
# kernels that need not occur in a window (run every few iterations)
OCCASIONAL = ("k_lg_order_keys", "rocprim:")


def _digest(n: int, nnz: int, g: int, repulsion: str):
    """The committed rocprofv3 traffic digest (FETCH_SIZE + WRITE_SIZE per
    dispatch, calibrated against a copy of known size), when it was taken on
    this same workload; None otherwise."""
    for path in TRAFFIC_FILES[repulsion]:
        try:
            rec = json.loads(path.read_text())
        except (OSError, ValueError):
            continue
        if (rec.get("n"), rec.get("nnz"), rec.get("repulsion")) != (n, nnz, repulsion):
            continue
        if repulsion == "grid" and rec.get("grid") != g:
            continue
        rec["_file"] = path.name
        return rec
    return None


def measured_traffic(kernel: str, n: int, nnz: int, g: int, repulsion: str):
    """HBM bytes per launch of the timer `kernel` from the digest."""
    rec = _digest(n, nnz, g, repulsion)
    if rec is None:
        return None
    # the timer's name is the kernel symbol's stem: "attract" is k_attract or
    # the tiled k_attract_tiles_seg<...>, "update" k_update<mode, grid>.  The
    # shared attraction is a pair of launches per iteration (the primary and
    # the helper that joins it on the main stream, HELPER = true): their
    # bytes per dispatch add up to the iteration's.
    hits = [t for name, t in rec.get("kernels", {}).items() if name.split("<")[0].startswith("k_" + kernel)]
    if not hits:
        return None
    return int(sum(t["fetch_bytes"] + t["write_bytes"] for t in hits))


def repulsion_traffic(n: int, nnz: int, g: int, repulsion: str):
    """HBM bytes per iteration of the repulsion kernels, from the digest:
    each kernel's bytes per dispatch times its dispatches in the digest's
    window of iterations."""
    rec = _digest(n, nnz, g, repulsion)
    if rec is None or "window_iterations" not in rec:
        return None
    total = 0.0
    kernels = rec.get("kernels", {})
    for sym in REPULSION_SYMBOLS[repulsion]:
        hits = [t for name, t in kernels.items()
                if (name.startswith(sym) if sym.endswith(":") else name.split("<")[0] == sym)]
        if not hits and sym not in OCCASIONAL:
            return None
        total += sum((t["fetch_bytes"] + t["write_bytes"]) * t["dispatches"] for t in hits)
    return int(total / rec["window_iterations"])


def cpu_share() -> int:
    """Threads for the CPU baseline: the CPUs this process may run on, at
    most 16 (one GPU's share of a GPU box's host)."""
    try:
        visible = len(os.sched_getaffinity(0))
    except AttributeError:
        visible = os.cpu_count() or 1
    return max(1, min(16, visible))


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(sess, y_start, n, lr, sched, budget_s, start_iter):
    """The reference's CPU algorithm, restated by the oracle
    (src/tsne_neighbors.cpp:1076-1256: fp32 bilinear FFT grid with the CPU
    grid policy, CSR attraction, gains/momentum update, fp64 centring), on
    the same P, from the layout at the start of the timed window, in that
    window's phase: at this host's thread share and at 4 threads (the
    reference's published CPU figures use 4 cores).  The oracle's fp64
    FIt-SNE restatement (no counterpart in the reference) is timed as an
    extra figure."""
    from oracle import oracle

    P = oracle.OracleP.wrap(*sess.csr())
    early = start_iter < sched["early_exaggeration_iter"]
    phase = "early-exaggeration" if early else "normal-phase"

    def rate(threads: int, method: int, budget: float):
        def run(count):
            y = np.array(y_start, np.float32, copy=True)
            if early:
                P.optimize(y, count, 0, sched["early_exaggeration"], 1.0, lr, False, sched["initial_momentum"],
                           sched["final_momentum"], method=method, threads=threads)
            else:
                P.optimize(y, 0, count, sched["early_exaggeration"], sched["exaggeration"], lr, False,
                           sched["initial_momentum"], sched["final_momentum"], method=method, threads=threads)

        t0 = time.perf_counter()
        run(1)
        one = time.perf_counter() - t0
        iters = max(2, min(400, int(budget / max(one, 1e-3))))
        t0 = time.perf_counter()
        run(iters)
        dt = time.perf_counter() - t0
        log(f"CPU oracle ({'bilinear' if method == oracle.METHOD_GRID else 'FIt-SNE fp64'}): {iters} {phase} "
            f"iterations in {dt:.1f}s on {threads} threads")
        return iters, dt

    share = cpu_share()
    it_all, dt_all = rate(share, oracle.METHOD_GRID, 0.55 * budget_s)
    it_4, dt_4 = rate(4, oracle.METHOD_GRID, 0.3 * budget_s)
    it_lg, dt_lg = rate(share, oracle.METHOD_LAGRANGE, 0.15 * budget_s)
    return {
        "value": round(it_all / dt_all, 4),
        "unit": "iterations/s",
        "cores": share,
        "kind": "port",
        "sample": f"{it_all} {phase} iterations of the same n={n} problem from the layout at iteration "
                  f"{start_iter}, same P; the reference's CPU algorithm (bilinear grid, CPU policy "
                  f"{oracle.policy_grid_size(n)} nodes per axis) restated by the oracle",
        "cpu_model": cpu_model(),
        "host_cpus_visible": os.cpu_count(),
        "threads_4": {"value": round(it_4 / dt_4, 4), "cores": 4, "iterations": it_4},
        "fitsne_fp64_oracle": {"value": round(it_lg / dt_lg, 4), "cores": share, "iterations": it_lg,
                               "note": "the oracle's fp64 FIt-SNE interpolation grid (no counterpart in the "
                                       "reference)"},
    }


if __name__ == "__main__":
    sys.exit(main())
