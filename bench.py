#!/usr/bin/env python3
"""Benchmark of the DROID-SLAM per-edge update path on one MI355X.

One step = the frontend-window workload the reference's run_update_pass
(cuda_slam/main.cu:2171-2405) drives through this path:
  * batched correlation volume + 4-level pyramid + radius-3 lookup for the
    48 edges of a 12-frame window of 128x48x64 fp32 features
    (batch_build_and_sample_correlation, main.cu:1555-1613), then
  * 3 Gauss-Newton bundle-adjustment iterations on the same window
    (BundleAdjustment::iterate, ba.cuh:476-803; Schur over depths, 10 free
    poses).
Inputs are synthetic (workloads.py), already resident in HBM when the timed
region starts.

Printed: one JSON line. `value` is edges/s of the full step (48 edges per
step); corr-only edges/s and BA-only iterations/s are timed separately in the
same run. `roofline` is for the dominant kernel (the correlation GEMM with its
pyramid epilogue), its average launch duration measured with hipEvents on the
launch stream. `cpu_baseline` times the path's PyTorch-CPU equivalents
(oracle/torch_baseline.py, in a child process on the host's cores) on a
bounded sample of the same workload, with the C oracle beside it.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

`--highres` times the same step on the high-resolution window instead (16
frames of 128x54x96 features, 64 edges in one launch, 3 BA iterations over
14 free poses) and prints one JSON line for it.

`--update` times the update operator (UpdateModule::forward with its
ConvGRU on the 48-edge window, then compute_eta of the 12 keyframes,
main.cu:385-667) and prints one JSON line for it.

`--encode` times the front of the pipe for one 384x512 frame: the NV12
1920x1080 -> 512x384 BGR conversion (main.cu:947-985) and encode_frame
(fnet + cnet fp16 encoders, main.cu:1465-1497), and prints one JSON line.

`--glue` times the update-pass glue around the path (motion/target kernels,
hidden-state gathers and scatters, the keyframe scatter-mean, the BA edge
set) for one 48-edge batch and prints one JSON line for it.

`--graph` times the backend's proximity-factor selection (frame distances of
all pairs of a 200-keyframe graph in one launch, then the reference's
selection) and prints one JSON line for it.

`--backend` instead times the backend configuration (200 keyframes, 2000
edges: correlation + lookup of every edge in 48-edge launches, then 5 BA
iterations over 198 free poses with the dense 1188x1188 Schur system) and
prints one JSON line for it; the headline line above is unaffected.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "slam-hands_amd"))

import numpy as np  # noqa: E402

METRIC = "corr edges/sec + BA iters/sec (48-edge window, 1 MI355X); % roofline"
PEAK_FP32_TFLOPS = 157.3  # MI355X dense fp32 (matrix and vector)
PEAK_F16_TFLOPS = 2500.0  # MI355X dense fp16 / bf16 MFMA
# HBM bytes per corr_window launch (48 edges): rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE passes of this script, scaled by a 256 MiB device copy
# (profiles/corr_window48_pmc_traffic.md)
TRAFFIC_BYTES = 381435721
# HBM bytes of the glue's 48-row copy (gather of 48 distinct 128x3072-float
# rows): the same passes over bench.py --glue (profiles/glue48_kernel_stats.md)
GLUE_ROWS_TRAFFIC_BYTES = 151029965
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=30,
                    help="untimed steps first (the clock settles over the first few dozen)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="after the run, one device-to-device copy of MIB MiB (the plain "
                         "copy kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--backend", action="store_true",
                    help="time the 200-keyframe backend configuration instead")
    ap.add_argument("--graph", action="store_true",
                    help="time the backend proximity-factor selection (200 keyframes) instead")
    ap.add_argument("--highres", action="store_true",
                    help="time the high-resolution window (16 frames of 128x54x96, 64 edges, "
                         "3 BA iterations) instead")
    ap.add_argument("--update", action="store_true",
                    help="time the update operator (UpdateModule forward of the 48-edge "
                         "window + compute_eta of its 12 keyframes) instead")
    ap.add_argument("--encode", action="store_true",
                    help="time the decode conversion + encode_frame of one 384x512 frame instead")
    ap.add_argument("--glue", action="store_true",
                    help="time the update-pass glue of one 48-edge batch instead")
    ap.add_argument("--cpu-edges", type=int, default=48,
                    help="edges of the window the CPU baseline runs (bounded sample)")
    ap.add_argument("--fp16-fmaps", action="store_true",
                    help="the window with fp16 feature maps (the reference's fmap storage)")
    ap.add_argument("--no-extras", action="store_true",
                    help="the headline line without the extra keys of configs 4 and 5 and of "
                         "the fp16-fmap window")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py: this build runs on one GPU only (asked for {args.gpus}); the path "
              "would shard by edge across GPUs, each holding the frames its edges touch, "
              "but no multi-GPU run is "
              "implemented.", file=sys.stderr)
        sys.exit(2)
    import slk
    import workloads as wl

    H = slk.hip()
    if H.device_count() < 1:
        raise SystemExit("bench.py: no GPU visible")
    slk.lib()  # fails loudly if libslk.so is missing
    if args.backend:
        return backend(args, slk, wl, H)
    if args.glue:
        return glue(args, slk, wl, H)
    if args.update:
        return update(args, slk, wl, H)
    if args.encode:
        return encode(args, slk, wl, H)
    if args.graph:
        return graph(args, slk, wl, H)

    if args.highres or args.fp16_fmaps:
        out = window(args, slk, wl, H, "highres" if args.highres else "corr_window",
                     fp16=args.fp16_fmaps)
        print(json.dumps(out), flush=True)
        return
    out = window(args, slk, wl, H, "corr_window")
    if not args.no_extras:
        out["extra"] = extras(args, slk, wl, H)
    print(json.dumps(out), flush=True)
    calibrate_copy(args, H)


def calibrate_copy(args, H):
    """One device-to-device copy of --calibrate-copy MiB, after the measured
    work: the known-size dispatch that scales rocprofv3's FETCH_SIZE and
    WRITE_SIZE to bytes."""
    if args.calibrate_copy > 0:
        nbytes = args.calibrate_copy << 20
        src, dst = H.malloc(nbytes), H.malloc(nbytes)
        H.memset(src, 1, nbytes)
        H.sync()
        H.dtod(dst, src, nbytes)
        H.sync()
        H.free(src)
        H.free(dst)
        print(f"bench.py: copy calibration {nbytes} bytes device-to-device", file=sys.stderr,
              flush=True)


def extras(args, slk, wl, H):
    """Summaries of the other configurations, measured in the same run: the
    high-resolution window (config 5), the 200-keyframe backend (config 4),
    and the headline window with the reference's fp16 fmaps."""
    sub = argparse.Namespace(**vars(args))
    sub.no_cpu_baseline = True
    out = {}
    hr = window(sub, slk, wl, H, "highres")
    out["config5_highres"] = {
        "workload": hr["config"]["workload"], "edges_per_s": hr["value"],
        "ms_per_step": hr["ms_per_step"], "corr_edges_per_s": hr["corr_edges_per_s"],
        "ba_iter_ms": hr["ba_iter_ms"], "corr_window_us": hr["kernels_us"]["corr_window"],
        "corr_window_frac": hr["roofline"]["frac"], "kernels_us": hr["kernels_us"]}
    f16 = window(sub, slk, wl, H, "corr_window", fp16=True)
    out["config2_fp16_fmaps"] = {
        "workload": f16["config"]["workload"] + " (fp16 fmaps)", "edges_per_s": f16["value"],
        "ms_per_step": f16["ms_per_step"], "corr_edges_per_s": f16["corr_edges_per_s"],
        "corr_window_us": f16["kernels_us"]["corr_window"],
        "corr_window_frac": f16["roofline"]["frac"], "kernels_us": f16["kernels_us"]}
    be = backend(sub, slk, wl, H, emit=False)
    out["config4_backend"] = {k: be[k] for k in (
        "value", "unit", "corr_ms_all_edges", "corr_edges_per_s", "ba_iter_ms",
        "ba_iters_per_s")}
    out["config4_backend"]["workload"] = be["config"]["workload"]
    return out


# the two window workloads: the headline (48 edges of a 12-frame 48x64 window)
# and the high-resolution window (64 edges of a 16-frame 54x96 window), each
# with 3 BA iterations on the same frames (poses 0 and 1 fixed)
WINDOWS = {
    "corr_window": dict(h=48, w=64, n=12, B=48, traffic=TRAFFIC_BYTES,
                        workload="corr_window + 3x ba_window"),
    "highres": dict(h=54, w=96, n=16, B=64, traffic=None,
                    workload="highres: corr of 64 edges at 54x96 + 3x ba"),
}


def window(args, slk, wl, H, name, fp16=False):
    """One window workload (fp16: the feature maps stored as fp16, the
    reference's fmap storage); returns the JSON dict."""
    cfg = WINDOWS[name]
    h, w, n, B = cfg["h"], cfg["w"], cfg["n"], cfg["B"]
    C = 128
    HW = h * w
    iters = 3
    lm, ep = 1e-4, 0.1
    fm = wl.frames(n, C, h, w, seed=0)
    if fp16:
        fm = fm.astype(np.float16)
    fdt = slk.SLK_F16 if fp16 else slk.SLK_F32
    ii, jj = wl.cyclic_edges(n)
    assert len(ii) == B
    coords = wl.flow_coords(B, h, w, seed=1)
    p = wl.ba_problem(n=n, h=h, w=w, ii=ii, jj=jj, seed=3)

    ctx = slk.Context(h, w, C=C, max_batch=B, corr_scale=wl.CORR_ALPHA_REF)
    D = slk.DeviceArray.from_host
    d_f, d_c = D(fm), D(coords)
    d_out = slk.DeviceArray((B, 196, HW))
    dp = {k: D(p[k]) for k in ("poses", "disps", "intr", "target", "weight", "eta", "ii", "jj")}
    stream = H.stream()

    def corr():
        ctx.batch_build_and_sample_correlation(d_f, ii, jj, d_c, d_out, dtype=fdt,
                                               stream=stream)

    def ba():
        # the step's BA iterations on the window's edge set, as the loop of
        # run_update_pass (main.cu:2371-2389): one slk_ba_iterate_n call
        ctx.ba_iterate_n(dp["poses"], dp["disps"], dp["intr"], dp["target"], dp["weight"],
                         dp["eta"], dp["ii"], dp["jj"], ii, jj, p["t0"], p["t1"], lm, ep,
                         iters, stream=stream)

    def step():
        corr()
        ba()

    def timed(fn, k):
        H.sync()
        e0, e1 = H.event(), H.event()
        H.record(e0, stream)
        for _ in range(k):
            fn()
        H.record(e1, stream)
        ms = H.elapsed_ms(e0, e1)
        H.sync()
        return ms

    for _ in range(args.warmup):
        step()
    H.sync()
    if ctx.ba_status(stream) != slk.SLK_OK:
        raise SystemExit("bench.py: BA system not positive definite during warmup")
    t0 = time.perf_counter()
    total_ms = timed(step, args.steps)
    wall = time.perf_counter() - t0
    ms_step = total_ms / args.steps
    value = B * args.steps / (total_ms / 1e3)

    corr_ms = timed(corr, args.steps) / args.steps
    ba_ms = timed(ba, args.steps) / (args.steps * iters)

    # per-kernel durations (events on the launch stream around each kernel),
    # over as many back-to-back steps as the timed region. The first pass
    # creates the events; the measured pass reuses them, so the host enqueues
    # as fast as in the timed region and the GPU runs the kernels back to
    # back, at the clock it holds under sustained load (a host that falls
    # behind leaves gaps in which the part recovers clock, which shortens the
    # kernels measured after them).
    ctx.profile_enable(True)
    for _ in range(args.steps):
        step()
    H.sync()
    ctx.profile()
    ctx.profile_enable(True)
    prof_ms_step = timed(step, args.steps) / args.steps
    prof = ctx.profile()
    ctx.profile_enable(False)
    kern = {k: {"avg_us": 1e3 * v[0] / v[1], "launches": v[1]} for k, v in prof.items()}

    # dominant kernel: corr_window, the correlation GEMM of the batched path
    # (every pyramid level as alpha * f_i . pool_l(f_j), only the 8x8 lookup
    # windows stored). `achieved` is the reference's algorithmic work, 2*HW^2*C
    # flops per edge (the volume GEMM of main.cu:1573-1581), over the average
    # launch duration, against the dense MFMA peak of the datapath the kernel
    # runs on (fp16 for the default 3-pass scaled hi/lo split, bf16 for the
    # bf16 split: both 2.5 PFLOP/s dense; fp32 for SLK_PREC_FP32). The split
    # issues 3 MFMA passes per product of fp32 features and each source tile
    # multiplies only the targets of its windows' boxes: `mfma_issued_*` is the
    # MFMA work it actually issued (listed 128x256 tiles x C x 2 x 3) in the
    # same time,
    # and `frac_ceiling_of_method` = algorithmic / issued flops is the highest
    # `frac` this method reaches with the MFMA pipes always busy.
    flop = 2.0 * HW * HW * C * B
    gemm_s = kern["corr_window"]["avg_us"] * 1e-6
    achieved = flop / gemm_s / 1e12
    split = ctx.corr_precision in (slk.SLK_PREC_F16X3, slk.SLK_PREC_BF16X3)
    f16 = ctx.corr_precision == slk.SLK_PREC_F16X3
    peak = PEAK_F16_TFLOPS if split else PEAK_FP32_TFLOPS
    roof = {
        "kernel": (f"corr_window ({'scaled fp16' if f16 else 'bf16'} hi/lo split, 3 MFMA "
                   f"passes: all-pairs volume at every pyramid level, lookup windows stored; "
                   f"{B} edges)" if split else
                   f"corr_window (fp32 MFMA all-pairs GEMM + pyramid epilogue, {B} edges)"),
        "bound": "mfma",
        "achieved": round(achieved, 2),
        "peak": peak,
        "unit": "TFLOP/s",
        "frac": round(achieved / peak, 4),
        "traffic": cfg["traffic"],
        "algorithmic_flop_per_launch": flop,
        "avg_launch_us": round(gemm_s * 1e6, 2),
    }
    if split:
        active, total = split_tiles_active(coords, h, w)
        exe = active * 128 * 256 * C * 2.0 * 3
        roof.update({"listed_tiles": int(active), "all_pairs_tiles": int(total),
                     "mfma_issued_flop_per_launch": exe,
                     "mfma_issued_TFLOPs": round(exe / gemm_s / 1e12, 2),
                     "mfma_issued_frac": round(exe / gemm_s / 1e12 / PEAK_F16_TFLOPS, 4),
                     "frac_ceiling_of_method": round(flop / exe, 4)})
    # lookup: coords + four 8x8 windows read, 196 channels written per pixel
    look_bytes = B * HW * (2 * 4 + 4 * 64 * 4 + 196 * 4)
    look_s = kern["corr_lookup_win"]["avg_us"] * 1e-6

    out = {
        "metric": METRIC if name == "corr_window" else
        "corr edges/sec + BA iters/sec (64-edge 54x96 window, 1 MI355X); % roofline",
        "value": round(value, 1),
        "unit": "edges/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("f32 (correlation: f32 features as a 3-pass scaled fp16 hi/lo MFMA split, "
                  "22 significant bits, f32 accumulation) / f64 (BA arithmetic and storage)"),
        "data": "synthetic (seeded N(0,1) features, U(-8,8) flow, BA window of workloads.py)",
        "config": {"workload": cfg["workload"], "frames": n, "edges": B, "h": h,
                   "w": w, "C": C, "levels": 4, "radius": 3, "ba_iters_per_step": iters,
                   "free_poses": p["t1"] - p["t0"], "lm": lm, "ep": ep,
                   "corr_scale": wl.CORR_ALPHA_REF, "parallelism": "single GPU"},
        "corr_edges_per_s": round(B / (corr_ms / 1e3), 1),
        "ba_iters_per_s": round(1e3 / ba_ms, 1),
        "corr_ms": round(corr_ms, 4),
        "ba_iter_ms": round(ba_ms, 4),
        "roofline": roof,
        "lookup_hbm": {"achieved_GBs": round(look_bytes / look_s / 1e9, 1), "peak": PEAK_HBM_GBS,
                       "frac": round(look_bytes / look_s / 1e9 / PEAK_HBM_GBS, 4)},
        "kernels_us": {k: round(v["avg_us"], 2) for k, v in kern.items()},
        "kernels_pass_ms_per_step": round(prof_ms_step, 4),
        "wall_s_timed": round(wall, 3),
    }
    if not args.no_cpu_baseline and not fp16:
        out["cpu_baseline"] = cpu_baseline(fm, ii, jj, coords, p, iters, lm, ep,
                                           min(args.cpu_edges, B))
    ctx.close()
    return out


def backend(args, slk, wl, H, emit=True):
    """The backend configuration (200 keyframes, ~2000 edges): correlation + lookup
    of all 2000 edges of a 200-keyframe graph in 48-edge launches (every
    keyframe's operands split once per pass, slk_corr_prepare_frames; the
    per-call preparation is timed beside it), then 5 BA
    iterations over 198 free poses (dense 1188x1188 Schur system, blocked
    multi-workgroup Cholesky). One JSON line; synthetic inputs resident in HBM."""
    h, w, C, n, B = 48, 64, 128, 200, 48
    HW = h * w
    iters = 5
    lm, ep = 1e-5, 1e-2
    ii, jj = wl.backend_edges(n, 2000)
    M = len(ii)
    fm = wl.frames(n, C, h, w, seed=0)
    coords = wl.flow_coords(B, h, w, seed=1)
    p = wl.ba_problem(n=n, h=h, w=w, ii=ii, jj=jj, seed=21)
    ctx = slk.Context(h, w, C=C, max_batch=B, corr_scale=wl.CORR_ALPHA_REF)
    D = slk.DeviceArray.from_host
    d_f, d_c = D(fm), D(coords)
    d_out = slk.DeviceArray((B, 196, HW))
    dp = {k: D(p[k]) for k in ("poses", "disps", "intr", "target", "weight", "eta", "ii", "jj")}
    stream = H.stream()
    nb = (M + B - 1) // B
    batches = [(ii[b * B:(b + 1) * B], jj[b * B:(b + 1) * B]) for b in range(nb)]

    def corr():
        # one pass: every keyframe split once, then the 42 batches over them
        ctx.prepare_frames(d_f, n, stream=stream)
        for bi, bj in batches:
            ctx.batch_build_and_sample_prepared(bi, bj, d_c, d_out, stream=stream)

    def corr_per_call():
        for bi, bj in batches:
            ctx.batch_build_and_sample_correlation(d_f, bi, bj, d_c, d_out, stream=stream)

    def ba():
        ctx.ba_iterate_n(dp["poses"], dp["disps"], dp["intr"], dp["target"], dp["weight"],
                         dp["eta"], dp["ii"], dp["jj"], ii, jj, p["t0"], p["t1"], lm, ep,
                         iters, stream=stream)

    def timed(fn, k):
        H.sync()
        e0, e1 = H.event(), H.event()
        H.record(e0, stream)
        for _ in range(k):
            fn()
        H.record(e1, stream)
        ms = H.elapsed_ms(e0, e1)
        H.sync()
        return ms

    corr()
    ba()
    H.sync()
    if ctx.ba_status(stream) != slk.SLK_OK:
        raise SystemExit("bench.py: backend BA system not positive definite")
    steps = max(1, min(args.steps, 5))
    corr_ms = timed(corr, steps) / steps
    corr_per_call()
    corr_pc_ms = timed(corr_per_call, steps) / steps
    ba_ms = timed(ba, steps) / (steps * iters)
    ctx.profile_enable(True)
    ba()
    H.sync()
    prof = ctx.profile()
    ctx.profile_enable(False)
    out = {
        "metric": "backend: corr edges/s + BA iters/s (200 keyframes, 2000 edges, 1 MI355X)",
        "value": round(M / (corr_ms / 1e3 + iters * ba_ms / 1e3), 1),
        "unit": "edges/s",
        "n_gpus": 1,
        "steps": steps,
        "higher_is_better": True,
        "dtype": "f32 correlation (scaled fp16 hi/lo split, 3 MFMA passes) / f64 BA",
        "data": "synthetic (workloads.py backend graph)",
        "config": {"workload": "backend corr + 5x ba", "frames": n, "edges": M, "h": h, "w": w,
                   "C": C, "free_poses": p["t1"] - p["t0"], "system": 6 * (p["t1"] - p["t0"]),
                   "ba_iters": iters, "lm": lm, "ep": ep},
        "corr_ms_all_edges": round(corr_ms, 3),
        "corr_ms_all_edges_per_call_preparation": round(corr_pc_ms, 3),
        "corr_edges_per_s": round(M / (corr_ms / 1e3), 1),
        "ba_iter_ms": round(ba_ms, 4),
        "ba_iters_per_s": round(1e3 / ba_ms, 1),
        "ba_kernels_us": {k: round(1e3 * v[0] / v[1], 1) for k, v in prof.items()},
    }
    ctx.close()
    if emit:
        print(json.dumps(out), flush=True)
    return out


def update_flops(h, w, B, K):
    """Algorithmic flops of UpdateModule::forward on B edges and compute_eta
    on K keyframes of h x w maps: 2 * Co * Ci * k^2 per output pixel and
    convolution (main.cu:552-603 shapes), plus the three 1x1 global terms."""
    from oracle import update_oracle as uo
    hw = h * w
    fwd = {n: 2.0 * co * ci * k * k * hw * B for n, co, ci, k in uo.LAYERS}
    for n in ("update_gru_convz_glo", "update_gru_convr_glo", "update_gru_convq_glo"):
        fwd[n] = 2.0 * 128 * 128 * B
    eta = {n: 2.0 * co * ci * k * k * hw * K for n, co, ci, k in uo.LAYERS
           if n in ("update_agg_conv2", "update_agg_eta_0")}
    for n in eta:
        fwd.pop(n)
    return fwd, eta


def encoder_flops(H_, W_, out_dim):
    """Algorithmic flops of one HalfBasicEncoder forward on an H x W frame:
    2 * Co * Ci * k^2 per output pixel of every convolution (main.cu:316-353
    shapes)."""
    from oracle import encoder_oracle as eo
    total, h, w = 0.0, H_, W_
    for suffix, co, ci, k, s in eo.LAYERS:
        co = out_dim if co is None else co
        if suffix in ("conv1", "layer2_0_conv1", "layer3_0_conv1"):
            h, w = h // 2, w // 2
        total += 2.0 * co * ci * k * k * h * w
    return total


def encode(args, slk, wl, H):
    """The front of the pipe for one frame: NV12 1920x1080 -> BGR 512x384
    (bilinear, BT.709) and encode_frame (fnet 128 with instance norm, cnet
    256) on seeded weights of the reference's shapes. One JSON line: frames/s
    of encode_frame, its achieved fp16 MFMA TFLOP/s against the 2.5 PFLOP/s
    dense peak, and the decode conversion's time and HBM rate."""
    sys.path.insert(0, ROOT)
    from oracle import encoder_oracle as eo
    Hf, Wf, sw, sh = 384, 512, 1920, 1080
    Pf = eo.seeded_weights("fnet", 128, seed=0)
    Pc = eo.seeded_weights("cnet", 256, seed=1)
    fnet = slk.Encoder(Hf, Wf, 128, True)
    cnet = slk.Encoder(Hf, Wf, 256, False)
    fnet.set_weights(Pf, "fnet")
    cnet.set_weights(Pc, "cnet")
    bgr = eo.seeded_frame(Hf, Wf, seed=2)
    rng = np.random.default_rng(3)
    D = slk.DeviceArray.from_host
    d_bgr = D(bgr)
    d_y = D(rng.integers(0, 256, (sh, sw), dtype=np.uint8))
    d_uv = D(rng.integers(0, 256, (sh // 2, sw), dtype=np.uint8))
    d_out = slk.DeviceArray((Hf, Wf, 3))
    fmap = slk.DeviceArray((128, Hf // 8, Wf // 8), np.float16)
    net = slk.DeviceArray((128, Hf // 8, Wf // 8))
    inp = slk.DeviceArray((128, Hf // 8, Wf // 8))
    stream = H.stream()

    def enc():
        slk.encode_frame(fnet, cnet, d_bgr, fmap, net, inp, stream=stream)

    def dec():
        slk.nv12_to_bgr(d_y, d_uv, d_out, sw, sh, sw, sw, Wf, Hf, stream=stream)

    def timed(fn, k):
        H.sync()
        e0, e1 = H.event(), H.event()
        H.record(e0, stream)
        for _ in range(k):
            fn()
        H.record(e1, stream)
        ms = H.elapsed_ms(e0, e1)
        H.sync()
        return ms / k

    for _ in range(max(3, args.warmup)):
        dec()
        enc()
    H.sync()
    k = max(5, min(args.steps, 50))
    t0w = time.perf_counter()
    e_ms = timed(enc, k)
    wall = time.perf_counter() - t0w
    d_ms = timed(dec, k)
    fl = encoder_flops(Hf, Wf, 128) + encoder_flops(Hf, Wf, 256)
    peak = PEAK_F16_TFLOPS
    # decode bytes: the 2x2 Y neighbourhoods and UV samples come through
    # the caches; algorithmic = Y plane + UV plane read once, BGR written
    dec_bytes = sw * sh * 1.5 + Hf * Wf * 12
    tc = time.perf_counter()
    eo.encode_frame(bgr, Pf, Pc)
    cpu_s = time.perf_counter() - tc
    out = {
        "metric": "front of the pipe: encode_frame (fnet + cnet) of a 384x512 frame, 1 MI355X",
        "value": round(1e3 / e_ms, 1),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": k,
        "higher_is_better": True,
        "dtype": "f16 activations and MFMA operands, f32 accumulation (the reference's fp16 "
                 "cuDNN convolutions)",
        "data": "synthetic (seeded weights of the reference's shapes, a structured BGR frame)",
        "config": {"workload": "encode_frame", "H": Hf, "W": Wf},
        "encode_frame_ms": round(e_ms, 4),
        "roofline": {"kernel": "encode_frame (every convolution of fnet and cnet)",
                     "bound": "mfma", "achieved": round(fl / (e_ms * 1e-3) / 1e12, 2),
                     "peak": peak, "unit": "TFLOP/s",
                     "frac": round(fl / (e_ms * 1e-3) / 1e12 / peak, 4), "traffic": None,
                     "algorithmic_flop": fl},
        "nv12_to_bgr_ms": round(d_ms, 4),
        "nv12_to_bgr_GBs": round(dec_bytes / (d_ms * 1e-3) / 1e9, 1),
        "cpu_baseline": {"value": round(1.0 / cpu_s, 3), "unit": "frames/s", "cores": 1,
                         "kind": "port",
                         "sample": "one frame through the numpy oracle (float64 sums)"},
        "wall_s_timed": round(wall, 3),
    }
    print(json.dumps(out), flush=True)
    fnet.close()
    cnet.close()


def update(args, slk, wl, H):
    """UpdateModule::forward on the 48-edge 48x64 window (corr lookup, motion,
    hidden states, context) and compute_eta on its 12 keyframes, seeded
    weights of the reference's shapes. One JSON line: forward and eta times,
    achieved fp16 MFMA TFLOP/s against the 2.5 PFLOP/s dense peak, and the
    PyTorch-free CPU oracle (float64 numpy) on one edge as the CPU figure."""
    sys.path.insert(0, ROOT)
    from oracle import update_oracle as uo
    h, w, B, K = 48, 64, 48, 12
    P = uo.seeded_weights(0)
    corr, motion, net, inp = uo.seeded_inputs(B, h, w, seed=1)
    agg = np.random.default_rng(2).uniform(0, 2, (K, 128, h, w)).astype(np.float32)
    um = slk.UpdateModule(B, h, w)
    um.set_weights(P)
    D = slk.DeviceArray.from_host
    dc, dm, dn, di, dk = D(corr), D(motion), D(net), D(inp), D(agg)
    dd, dw = slk.DeviceArray((B, 3, h, w)), slk.DeviceArray((B, 3, h, w))
    da, de = slk.DeviceArray((B, 128, h, w)), slk.DeviceArray((K, 1, h, w))
    stream = H.stream()

    def fwd():
        um.forward(dc, dm, dn, di, dd, dw, da, B, stream=stream)

    def eta():
        um.compute_eta(dk, de, K, stream=stream)

    def timed(fn, k):
        H.sync()
        e0, e1 = H.event(), H.event()
        H.record(e0, stream)
        for _ in range(k):
            fn()
        H.record(e1, stream)
        ms = H.elapsed_ms(e0, e1)
        H.sync()
        return ms / k

    for _ in range(max(3, args.warmup)):
        fwd()
        eta()
    H.sync()
    k = max(5, min(args.steps, 50))
    t0w = time.perf_counter()
    f_ms = timed(fwd, k)
    wall = time.perf_counter() - t0w
    e_ms = timed(eta, k)
    ff, fe = update_flops(h, w, B, K)
    f_fl, e_fl = sum(ff.values()), sum(fe.values())
    peak = PEAK_F16_TFLOPS
    zr_fl = ff["update_gru_convz"] + ff["update_gru_convr"]
    tc = time.perf_counter()
    uo.update_forward(P, corr[:1], motion[:1], net[:1], inp[:1])
    cpu_s = time.perf_counter() - tc
    out = {
        "metric": "update operator: UpdateModule forward, 48-edge 48x64 window, 1 MI355X",
        "value": round(B / (f_ms * 1e-3), 1),
        "unit": "edges/s",
        "n_gpus": 1,
        "steps": k,
        "higher_is_better": True,
        "dtype": "f16 MFMA operands, f32 accumulation (the reference's tensor-op convolutions "
                 "round operands to the same 10-bit mantissa); fp16 activations",
        "data": "synthetic (seeded weights of the reference's shapes, N(0,1) lookup, "
                "U(-8,8) motion, U(-1,1) state, N(0,1) context)",
        "config": {"workload": "update operator", "edges": B, "keyframes": K, "h": h, "w": w},
        "forward_ms": round(f_ms, 4),
        "compute_eta_ms": round(e_ms, 4),
        "forward_TFLOPs": round(f_fl / (f_ms * 1e-3) / 1e12, 1),
        "roofline": {"kernel": "UpdateModule::forward (all convolutions, 48 edges)",
                     "bound": "mfma", "achieved": round(f_fl / (f_ms * 1e-3) / 1e12, 2),
                     "peak": peak, "unit": "TFLOP/s",
                     "frac": round(f_fl / (f_ms * 1e-3) / 1e12 / peak, 4), "traffic": None,
                     "algorithmic_flop": f_fl, "convz_convr_flop": zr_fl},
        "compute_eta_TFLOPs": round(e_fl / (e_ms * 1e-3) / 1e12, 1),
        "cpu_baseline": {"value": round(1.0 / cpu_s, 3), "unit": "edges/s", "cores": 1,
                         "kind": "port",
                         "sample": "one edge through the float64 numpy oracle"},
        "wall_s_timed": round(wall, 3),
    }
    um.close()
    print(json.dumps(out), flush=True)


def glue(args, slk, wl, H):
    """The update-pass glue of one 48-edge batch of run_update_pass
    (cuda_slam/main.cu:2186-2390) around correlation and BA, on the 48x64
    window with 128-channel hidden states: motion features, hidden-state and
    inps loads, target/weight, hidden-state and conv1 saves, the keyframe
    scatter-mean and eta write-back, and the BA edge set with 24 inactive
    edges. One JSON line: the whole glue per batch, each call, the dominant
    row-copy kernel against HBM peak, the same copies issued the reference's
    way (one copy per edge and array), and the CPU oracle on the same data."""
    import ctypes

    h, w, B, nkf, ninac = 48, 64, 48, 12, 24
    HW = h * w
    row = 128 * HW
    L = slk.lib()
    rng = np.random.default_rng(0)
    ii, jj = wl.cyclic_edges(nkf)
    ii_in = rng.integers(0, nkf, ninac).astype(np.int32)
    jj_in = rng.integers(0, nkf, ninac).astype(np.int32)
    host = {
        "coords1": wl.flow_coords(B, h, w, seed=1),
        "target": wl.flow_coords(B, h, w, seed=2),
        "nets": rng.normal(size=(B, row)).astype(np.float32),
        "inps": rng.normal(size=(nkf, row)).astype(np.float32),
        "agg1": rng.normal(size=(B, row)).astype(np.float32),
        "delta": rng.normal(size=(B, 3, HW)).astype(np.float32),
        "wt": rng.random((B, 3, HW)).astype(np.float32),
        "kf_eta": rng.random((nkf, HW)).astype(np.float32),
        "target_inac": rng.normal(size=(ninac, 2, HW)).astype(np.float32),
        "weight_inac": rng.random((ninac, 2, HW)).astype(np.float32),
    }
    ctx = slk.Context(h, w, C=128, max_batch=B)
    D = slk.DeviceArray.from_host
    d = {k: D(v) for k, v in host.items()}
    d["ii"] = D(ii.astype(np.int32))
    for k, shape in [("motion", (B, 4, HW)), ("batch_nets", (B, row)), ("batch_inps", (B, row)),
                     ("tgt", (B, 2, HW)), ("wgt", (B, 2, HW)), ("all_agg1", (B, row)),
                     ("kf_agg", (nkf, row)), ("damping", (nkf, HW)),
                     ("ba_target", (B + ninac, 2, HW)), ("ba_weight", (B + ninac, 2, HW))]:
        d[k] = slk.DeviceArray(shape)
    d["act"] = slk.DeviceArray((B,), np.int32)
    d["ba_ii"] = slk.DeviceArray((B + ninac,), np.int32)
    d["ba_jj"] = slk.DeviceArray((B + ninac,), np.int32)
    ii_h, jj_h = np.ascontiguousarray(ii, np.int32), np.ascontiguousarray(jj, np.int32)
    bi_h, bj_h = np.zeros(B + ninac, np.int32), np.zeros(B + ninac, np.int32)
    na, cnt, t0 = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
    stream = H.stream()
    ck = slk.check

    calls = {
        "compute_motion": lambda: ck(L.slk_compute_motion(
            d["motion"].ptr, d["coords1"].ptr, None, d["target"].ptr, B, h, w, stream)),
        "gather_nets": lambda: ck(L.slk_gather_rows(
            d["batch_nets"].ptr, d["nets"].ptr, None, B, row, stream)),
        "gather_inps": lambda: ck(L.slk_gather_rows(
            d["batch_inps"].ptr, d["inps"].ptr, d["ii"].ptr, B, row, stream)),
        "compute_target": lambda: ck(L.slk_compute_target(
            d["tgt"].ptr, d["wgt"].ptr, d["coords1"].ptr, d["delta"].ptr, d["wt"].ptr, B, HW,
            stream)),
        "scatter_nets": lambda: ck(L.slk_scatter_rows(
            d["nets"].ptr, d["batch_nets"].ptr, None, B, row, stream)),
        "scatter_agg1": lambda: ck(L.slk_scatter_rows(
            d["all_agg1"].ptr, d["agg1"].ptr, None, B, row, stream)),
        "scatter_mean": lambda: ck(L.slk_scatter_mean(
            ctx.ptr, d["kf_agg"].ptr, d["all_agg1"].ptr, ii_h.ctypes.data, B, row, d["act"].ptr,
            None, ctypes.byref(na), stream)),
        "scatter_eta": lambda: ck(L.slk_scatter_rows(
            d["damping"].ptr, d["kf_eta"].ptr, d["act"].ptr, nkf, HW, stream)),
        "ba_edge_set": lambda: ck(L.slk_ba_edge_set(
            ctx.ptr, ii_h.ctypes.data, jj_h.ctypes.data, B, ii_in.ctypes.data,
            jj_in.ctypes.data, ninac, d["tgt"].ptr, d["wgt"].ptr, d["target_inac"].ptr,
            d["weight_inac"].ptr, HW, nkf, -1, 1, bi_h.ctypes.data, bj_h.ctypes.data,
            d["ba_ii"].ptr, d["ba_jj"].ptr, d["ba_target"].ptr, d["ba_weight"].ptr,
            ctypes.byref(cnt), ctypes.byref(t0), stream)),
    }

    def step():
        for fn in calls.values():
            fn()

    def reference_copies():
        # the reference's per-edge cudaMemcpy loops of one batch
        # (main.cu:2216-2224, 2245-2252, 2305-2309) as async device copies
        rb = row * 4
        for e in range(B):
            H.dtod_async(d["batch_nets"].ptr + e * rb, d["nets"].ptr + e * rb, rb, stream)
            H.dtod_async(d["batch_inps"].ptr + e * rb, d["inps"].ptr + int(ii[e]) * rb, rb,
                         stream)
        for e in range(B):
            H.dtod_async(d["nets"].ptr + e * rb, d["batch_nets"].ptr + e * rb, rb, stream)
            H.dtod_async(d["all_agg1"].ptr + e * rb, d["agg1"].ptr + e * rb, rb, stream)
        for a in range(nkf):
            H.dtod_async(d["damping"].ptr + a * HW * 4, d["kf_eta"].ptr + a * HW * 4, HW * 4,
                         stream)

    def timed(fn, k):
        H.sync()
        e0, e1 = H.event(), H.event()
        H.record(e0, stream)
        for _ in range(k):
            fn()
        H.record(e1, stream)
        ms = H.elapsed_ms(e0, e1)
        H.sync()
        return ms / k

    for _ in range(max(1, args.warmup)):
        step()
        reference_copies()
    H.sync()
    k = max(5, min(args.steps, 50))
    t0w = time.perf_counter()
    step_ms = timed(step, k)
    wall = time.perf_counter() - t0w
    per_call = {name: round(timed(fn, k) * 1e3, 2) for name, fn in calls.items()}
    copies_ms = timed(lambda: [calls[c]() for c in ("gather_nets", "gather_inps", "scatter_nets",
                                                     "scatter_agg1", "scatter_eta")], k)
    ref_ms = timed(reference_copies, max(2, k // 5))

    # algorithmic HBM bytes of each call (read once + written once)
    f4 = 4
    nbytes = {
        "compute_motion": B * HW * f4 * (2 + 2 + 4),
        "gather_nets": 2 * B * row * f4, "gather_inps": 2 * B * row * f4,
        "compute_target": B * HW * f4 * (2 + 2 + 2 + 2 + 2),
        "scatter_nets": 2 * B * row * f4, "scatter_agg1": 2 * B * row * f4,
        "scatter_mean": (B + nkf) * row * f4, "scatter_eta": 2 * nkf * HW * f4,
        "ba_edge_set": 2 * 2 * cnt.value * 2 * HW * f4,
    }
    total_bytes = sum(nbytes.values())
    copy_bytes = sum(nbytes[c] for c in ("gather_nets", "gather_inps", "scatter_nets",
                                         "scatter_agg1", "scatter_eta"))
    # gather_nets: 48 distinct rows read once and written once (gather_inps
    # reads 12 rows four times each, partly from cache)
    dom = "gather_nets"
    dom_gbs = nbytes[dom] / (per_call[dom] * 1e-6) / 1e9

    # CPU oracle on the same arrays (one batch; memcpy loops, a sequential mean)
    from oracle import oracle as orc
    orc.build()
    t = time.perf_counter()
    orc.compute_motion(host["coords1"], host["target"], h, w)
    orc.gather_rows(host["nets"], None, n=B)
    orc.gather_rows(host["inps"], ii)
    orc.compute_target(host["coords1"], host["delta"], host["wt"])
    orc.scatter_rows(host["nets"], host["nets"], None)
    orc.scatter_rows(host["agg1"], host["agg1"], None)
    orc.scatter_mean(host["agg1"], ii)
    orc.ba_edge_set(ii, jj, ii_in, jj_in, host["target"], host["target"],
                    host["target_inac"], host["weight_inac"], nkf)
    cpu_ms = (time.perf_counter() - t) * 1e3

    out = {
        "metric": "update-pass glue of one 48-edge batch (48x64, 128-channel rows), 1 MI355X",
        "value": round(step_ms * 1e3, 2),
        "unit": "us per batch",
        "n_gpus": 1,
        "steps": k,
        "higher_is_better": False,
        "dtype": "f32 (copies; scatter-mean sums in f32 with one fused multiply-add)",
        "data": "synthetic (seeded N(0,1) rows, U(-8,8) flow)",
        "config": {"workload": "update-pass glue", "edges": B, "keyframes": nkf,
                   "inactive_edges": ninac, "h": h, "w": w, "row_floats": row},
        "algorithmic_bytes": total_bytes,
        "achieved_GBs": round(total_bytes / (step_ms * 1e-3) / 1e9, 1),
        "calls_us": per_call,
        "roofline": {"kernel": f"k_rows ({dom}: 48 rows of 128x3072 floats)",
                     "bound": "hbm", "achieved": round(dom_gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(dom_gbs / PEAK_HBM_GBS, 4),
                     "traffic": GLUE_ROWS_TRAFFIC_BYTES,
                     "algorithmic_bytes_per_launch": nbytes[dom]},
        "row_copies": {"one_launch_per_array_us": round(copies_ms * 1e3, 2),
                       "per_edge_async_copies_us": round(ref_ms * 1e3, 2),
                       "copies": 4 * B + nkf, "bytes": copy_bytes},
        "cpu_baseline": {"value": round(cpu_ms * 1e3, 1), "unit": "us per batch", "cores": 1,
                         "kind": "port", "sample": "the same batch through the C oracle"},
        "wall_s_timed": round(wall, 3),
    }
    print(json.dumps(out), flush=True)


def graph(args, slk, wl, H):
    """The backend's add_proximity_factors(0, 0, radius 2, nms 3, thresh 20)
    (cuda_slam/main.cu:2462-2471, 1679-1779) over a 200-keyframe graph with
    its 2000 active edges: frame distances of all 40000 pairs plus the
    selection, through slk_proximity_factors (one launch, one read-back).
    Beside it: the same distances fetched the reference's way
    (compute_frame_distances_batch, main.cu:1655-1676: 1024 pairs per
    upload + launch + synchronise + read-back), and the CPU oracle's
    distances and selection on the same inputs."""
    import ctypes

    h, w, t, rad, nms, thresh, beta = 48, 64, 200, 2, 3, 20.0, 0.3
    HW = h * w
    L = slk.lib()
    rng = np.random.default_rng(0)
    poses = np.zeros((t, 7), np.float32)
    poses[:, 0] = 0.02 * np.arange(t) + rng.normal(0, 0.01, t)
    poses[:, 1:3] = rng.normal(0, 0.01, (t, 2))
    poses[:, 3:] = wl.quat_from_rotvec(rng.normal(0, 0.02, (t, 3)))
    disps = rng.uniform(0.2, 2.0, (t, h, w)).astype(np.float32)
    intr = np.array([60.0, 60.0, 32.0, 24.0], np.float32)
    ii, jj = wl.backend_edges(t, 2000)
    ii, jj = np.ascontiguousarray(ii, np.int32), np.ascontiguousarray(jj, np.int32)
    ctx = slk.Context(h, w, C=128, max_batch=1)
    D = slk.DeviceArray.from_host
    dp, dd, di = D(poses), D(disps), D(intr)
    stream = H.stream()
    npairs = t * t
    cap = 2 * t * (t + rad + 1)
    ni, nj = np.zeros(cap, np.int32), np.zeros(cap, np.int32)
    dist = np.zeros(npairs, np.float32)
    n_new, n_es = ctypes.c_int(0), ctypes.c_int(0)

    def ours():
        slk.check(L.slk_proximity_factors(
            ctx.ptr, dp.ptr, dd.ptr, di.ptr, t, 0, 0, rad, nms, thresh, beta, ii.ctypes.data,
            jj.ctypes.data, len(ii), None, None, 0, 0, ni.ctypes.data, nj.ctypes.data, cap,
            ctypes.byref(n_new), ctypes.byref(n_es), dist.ctypes.data, stream))

    pi = np.repeat(np.arange(t), t).astype(np.int32)
    pj = np.tile(np.arange(t), t).astype(np.int32)
    bi, bj = slk.DeviceArray((1024,), np.int32), slk.DeviceArray((1024,), np.int32)
    bd = slk.DeviceArray((1024,))
    ref_d = np.zeros(npairs, np.float32)

    def reference_batches():
        for off in range(0, npairs, 1024):
            b = min(1024, npairs - off)
            H.htod(bi.ptr, pi[off:off + b])
            H.htod(bj.ptr, pj[off:off + b])
            slk.check(L.slk_frame_distance(dp.ptr, dd.ptr, di.ptr, bi.ptr, bj.ptr, bd.ptr, b, h,
                                           w, beta, None))
            H.sync()
            H.dtoh(ref_d[off:off + b], bd.ptr)

    ours()
    reference_batches()
    k = max(3, min(args.steps, 20))
    t0w = time.perf_counter()
    for _ in range(k):
        ours()
    ours_ms = (time.perf_counter() - t0w) * 1e3 / k
    t0w = time.perf_counter()
    for _ in range(max(2, k // 4)):
        reference_batches()
    ref_ms = (time.perf_counter() - t0w) * 1e3 / max(2, k // 4)
    # distance kernel alone (hipEvents on the stream)
    dpi, dpj = D(pi), D(pj)
    dall = slk.DeviceArray((npairs,))
    H.sync()
    e0, e1 = H.event(), H.event()
    H.record(e0, stream)
    for _ in range(k):
        slk.check(L.slk_frame_distance(dp.ptr, dd.ptr, di.ptr, dpi.ptr, dpj.ptr, dall.ptr, npairs,
                                       h, w, beta, stream))
    H.record(e1, stream)
    kern_ms = H.elapsed_ms(e0, e1) / k
    H.sync()
    assert np.array_equal(ref_d, dist), "batched and one-launch distances differ"
    # ~80 flops per pixel-pair (two projections; divisions and square roots
    # counted as one flop each)
    flops = 80.0 * npairs * HW
    gflops = flops / (kern_ms * 1e-3) / 1e9

    # edge-state update of a 48-edge frontend window (main.cu:1757-1796): the
    # 8 oldest edges stored as inactive and the other 40 closed up, hidden
    # states (128 x 48 x 64 floats), targets and weights moving with them;
    # against the reference's pattern, one device copy per row and array
    ne, eh, ew = 48, 48, 64
    ehw = eh * ew
    rng = np.random.default_rng(21)
    e_age = rng.integers(0, 30, ne).astype(np.int32)
    e_mask = np.zeros(ne, np.uint8)
    L.slk_oldest_edges_mask(e_age.ctypes.data, ne, 8, e_mask.ctypes.data)
    e_nets = slk.DeviceArray((ne, 128, ehw))
    e_tg, e_wt = slk.DeviceArray((ne, 2, ehw)), slk.DeviceArray((ne, 2, ehw))
    e_tin, e_win = slk.DeviceArray((64, 2, ehw)), slk.DeviceArray((64, 2, ehw))
    ectx = slk.Context(eh, ew, C=128, max_batch=48)
    e_ii = rng.integers(0, 12, ne).astype(np.int32)

    def edge_state():
        hii, hjj, hage = e_ii.copy(), e_ii.copy(), e_age.copy()
        iin, jin = np.zeros(64, np.int32), np.zeros(64, np.int32)
        ni, nk = ctypes.c_int(0), ctypes.c_int(0)
        slk.check(L.slk_store_and_remove_edges(
            ectx.ptr, e_mask.ctypes.data, ne, hii.ctypes.data, hjj.ctypes.data, hage.ctypes.data,
            iin.ctypes.data, jin.ctypes.data, ctypes.byref(ni), 64, e_nets.ptr, 128 * ehw,
            e_tg.ptr, e_wt.ptr, e_tin.ptr, e_win.ptr, 2 * ehw, ctypes.byref(nk), stream))
        H.sync()

    def edge_state_reference():
        kept, ni = 0, 0
        for e in range(ne):
            if e_mask[e]:
                for a, b in ((e_tin, e_tg), (e_win, e_wt)):
                    H.dtod_async(a.ptr + ni * 8 * ehw, b.ptr + e * 8 * ehw, 8 * ehw, stream)
                ni += 1
            else:
                if kept != e:
                    H.dtod_async(e_nets.ptr + kept * 512 * ehw, e_nets.ptr + e * 512 * ehw,
                                 512 * ehw, stream)
                    for a in (e_tg, e_wt):
                        H.dtod_async(a.ptr + kept * 8 * ehw, a.ptr + e * 8 * ehw, 8 * ehw,
                                     stream)
                kept += 1
        H.sync()

    edge_state()
    edge_state_reference()
    t0w = time.perf_counter()
    for _ in range(k):
        edge_state()
    es_ms = (time.perf_counter() - t0w) * 1e3 / k
    t0w = time.perf_counter()
    for _ in range(k):
        edge_state_reference()
    es_ref_ms = (time.perf_counter() - t0w) * 1e3 / k
    ectx.close()

    from oracle import oracle as orc
    orc.build()
    sample = 4000  # bounded CPU sample: the first 4000 pairs' distances
    tc = time.perf_counter()
    orc.frame_distance(poses, disps, intr, pi[:sample], pj[:sample], h, w, beta)
    cpu_dist_ms = (time.perf_counter() - tc) * 1e3 * npairs / sample
    tc = time.perf_counter()
    orc.proximity_select(dist, t, 0, 0, rad, nms, thresh, ii, jj)
    cpu_sel_ms = (time.perf_counter() - tc) * 1e3
    out = {
        "metric": "backend proximity factors (200 keyframes, 40000 pairs, 2000 edges), 1 MI355X",
        "value": round(ours_ms, 3),
        "unit": "ms per call",
        "n_gpus": 1,
        "steps": k,
        "higher_is_better": False,
        "dtype": "f32",
        "data": "synthetic (200-keyframe trajectory, backend edge graph of workloads.py)",
        "config": {"workload": "proximity factors", "keyframes": t, "pairs": npairs,
                   "edges": len(ii), "rad": rad, "nms": nms, "thresh": thresh, "h": h, "w": w},
        "new_edges": n_new.value,
        "greedy_edges": n_es.value,
        "frame_distance_kernel_ms": round(kern_ms, 4),
        "roofline": {"kernel": "k_frame_distance (40000 pairs x 3072 pixels)", "bound": "valu",
                     "achieved": round(gflops / 1e3, 2), "peak": PEAK_FP32_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(gflops / 1e3 / PEAK_FP32_TFLOPS, 4),
                     "traffic": None, "flop_per_pixel_pair": 80},
        "reference_pattern_ms": round(ref_ms, 3),
        "edge_state_update": {"workload": "48 active edges, the 8 oldest stored as inactive, "
                                          "40 closed up (hidden states 128x48x64)",
                              "ms": round(es_ms, 3), "reference_pattern_ms": round(es_ref_ms, 3)},
        "cpu_baseline": {"value": round(cpu_dist_ms + cpu_sel_ms, 1), "unit": "ms per call",
                         "cores": orc.lib().orc_num_threads(), "kind": "port",
                         "sample": f"oracle distances of {sample} pairs scaled to {npairs}, "
                                   "plus the selection"},
    }
    print(json.dumps(out), flush=True)


def split_tiles_active(coords, h, w, levels=4, src_tile=128, tgt_tile=256, band=16,
                       max_keys=8192):
    """(listed, all-pairs) 128-source x 256-target tiles of the batched
    correlation, restating the order pass of the GPU (order_and_boxes) in
    numpy: sources sorted by (band of 16 rows of the clamped floored y,
    snaking column of the clamped floored x); a source tile is a run of 128
    sorted sources, its level-l target box the windows' extent over the
    tile's bucket range, clipped to the level; the boxes' cells concatenated
    are cut into runs of 256 targets, each one listed tile. `all-pairs` is
    the number of tiles of the full volume (every source tile x every
    256-target run of the concatenated levels)."""
    B, HW = coords.shape[0], h * w
    hl = [h >> l for l in range(levels)]
    wl = [w >> l for l in range(levels)]
    ttot = sum(a * b for a, b in zip(hl, wl))
    mtiles = -(-HW // src_tile)
    lim = float(1 << 20)
    f = np.clip(np.floor(np.nan_to_num(coords, nan=-lim)), -lim, lim).astype(np.int64)
    fx, fy = f[:, 0, :], f[:, 1, :]
    kx, nb = w + 9, -(-(h + 9) // band)
    sx, nxb = 0, kx
    while nb * nxb > max_keys and sx < 20:
        sx += 1
        nxb = (kx + (1 << sx) - 1) >> sx
    bnd = (np.clip(fy, -8, h) + 8) // band
    xb = (np.clip(fx, -8, w) + 8) >> sx
    key = np.sort(bnd * nxb + np.where(bnd & 1, nxb - 1 - xb, xb), axis=1)
    first = np.arange(mtiles) * src_tile
    last = np.minimum(first + src_tile, HW) - 1
    b0, b1 = key[:, first], key[:, last]
    band0, band1 = b0 // nxb, b1 // nxb

    def col(b):
        s_ = b % nxb
        return np.where((b // nxb) & 1, nxb - 1 - s_, s_)

    c0, c1 = col(b0), col(b1)
    same, next_ = band0 == band1, band1 == band0 + 1
    xlo = np.where(same, np.minimum(c0, c1),
                   np.where(next_ & (band0 % 2 == 0), np.minimum(c0, c1), 0))
    xhi = np.where(same, np.maximum(c0, c1),
                   np.where(next_ & (band0 % 2 == 1), np.maximum(c0, c1), nxb - 1))
    fx0, fx1 = (xlo << sx) - 8, ((xhi + 1) << sx) - 9
    fy0, fy1 = band0 * band - 8, band1 * band + band - 9
    total = np.zeros_like(b0)
    for l in range(levels):
        xa, xe = np.maximum((fx0 >> l) - 3, 0), np.minimum((fx1 >> l) + 4, wl[l] - 1)
        ya, ye = np.maximum((fy0 >> l) - 3, 0), np.minimum((fy1 >> l) + 4, hl[l] - 1)
        total += np.where((xa <= xe) & (ya <= ye), (xe - xa + 1) * (ye - ya + 1), 0)
    listed = int((-(-total // tgt_tile)).sum())
    return listed, B * mtiles * (-(-ttot // tgt_tile))


def cpu_baseline(fm, ii, jj, coords, p, iters, lm, ep, nedges):
    """The CPU baseline: the path's PyTorch-CPU equivalents (oracle/
    torch_baseline.py: torch.bmm fp32 correlation, F.avg_pool2d pyramid, an
    8x8 gather lookup, float64 einsum / index_add_ / Cholesky BA; checked
    against the C oracle by tests/test_torch_baseline.py), timed in a child
    process on this host's cores with CPU tensors only: the median of 5
    repetitions of `nedges` of the window's edges and its BA iterations,
    scaled to edges/s of the step. The C oracle (C + OpenMP, fp64
    accumulation) is timed beside it as a second, labelled figure; it alone is
    reported if the child cannot run torch."""
    import subprocess
    B = len(ii)
    n, C, h, w = fm.shape
    sample = (f"{nedges}/{B} edges (corr + pyramid + lookup, 8 edges per bmm) + {iters} BA "
              f"iterations on the full {n}-frame window, median of 5 after a warm-up, scaled "
              f"to the {B}-edge + {iters}-iteration step")
    oracle_fig = cpu_baseline_oracle(fm, ii, jj, coords, p, iters, lm, ep, min(nedges, 8))
    cmd = [sys.executable, os.path.join(ROOT, "oracle", "torch_baseline.py"), "--frames",
           str(n), "--h", str(h), "--w", str(w), "--edges", str(B), "--sample-edges",
           str(nedges), "--iters", str(iters), "--reps", "5"]
    try:
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=600, check=True)
        t = json.loads(r.stdout.strip().splitlines()[-1])
    except (subprocess.SubprocessError, ValueError, IndexError) as exc:
        out = dict(oracle_fig)
        out["note"] = f"PyTorch-CPU baseline unavailable ({type(exc).__name__}); C oracle only"
        return out
    return {"value": round(t["edges_per_s"], 2), "unit": "edges/s", "cores": t["threads"],
            "kind": "port", "impl": "pytorch-cpu", "torch": t["torch"],
            "os_cpu_count": t["os_cpu_count"], "affinity_cpus": t["affinity_cpus"],
            "sample": sample, "corr_s_per_edge": round(t["corr_s_per_edge"], 5),
            "ba_s_per_iter": round(t["ba_s_per_iter"], 5), "c_oracle": oracle_fig}


def cpu_baseline_oracle(fm, ii, jj, coords, p, iters, lm, ep, nedges):
    """The CPU oracle (oracle/liboracle.so, C + OpenMP, fp64 accumulation)
    on a bounded sample: correlation+lookup of `nedges` edges and the step's
    BA iterations on the full window, scaled to the step's edges/s."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc
    orc.lib()
    B = len(ii)
    t0 = time.perf_counter()
    orc.corr_batch(fm, ii[:nedges], jj[:nedges], coords[:nedges], 1.0 / 16.0)
    t_corr = (time.perf_counter() - t0) / nedges
    t0 = time.perf_counter()
    poses, disps = p["poses"], p["disps"]
    for _ in range(iters):
        r = orc.ba_iterate(poses, disps, p["intr"], p["target"], p["weight"], p["eta"], p["ii"],
                           p["jj"], p["h"], p["w"], p["t0"], p["t1"], lm, ep)
        poses, disps = r["poses"], r["disps"]
    t_ba = (time.perf_counter() - t0) / iters
    step_s = B * t_corr + iters * t_ba
    return {"value": round(B / step_s, 2), "unit": "edges/s", "cores": orc.num_threads(),
            "kind": "port", "impl": "C oracle (OpenMP, fp64 accumulation)",
            "sample": f"oracle corr+pyramid+lookup of {nedges}/{B} edges + {iters} BA "
                      f"iterations (full window), scaled to the {B}-edge + {iters}-iteration "
                      "step",
            "corr_s_per_edge": round(t_corr, 4), "ba_s_per_iter": round(t_ba, 4)}


if __name__ == "__main__":
    main()
