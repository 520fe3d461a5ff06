#!/usr/bin/env python3
"""Benchmark: one forward+backward rasterization step on one MI355X.

Workload: 1,000,000 Gaussians, SH degree 3,
one 1280x720 pinhole camera, gsplat_amd.rasterization() with the API defaults
(packed=True, 16x16 tiles), L1 loss against a random target, backward to all
Gaussian parameters.  Synthetic seeded data (gsplat_amd._helper.make_scene).

Prints ONE JSON line (rank 0).  The metric is the median of the per-step
times of the K timed steps (HIP events between consecutive steps).  Besides
ms/step it reports Mpix/s, a
per-stage breakdown (HIP events around every C-ABI entry point, measured in a
separate pass), the roofline of the dominant kernel (HIP events around that
kernel inside the timed steps) and a CPU baseline: the host oracle pipeline
(oracle/torch_ref.py, float32, autograd) timed on this machine's cores on a
strided sample of the tiles, scaled to the full image.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

# BASELINE.json's metric (config 1) and the same quantity named for the other
# configurations' workloads
METRICS = {
    0: "ms per fwd+bwd step @10k Gaussians 256x256 SH0; Mpix/s; % HBM roofline",
    1: "ms per fwd+bwd step @1M Gaussians 1280x720 SH3; Mpix/s; % HBM roofline",
    2: "ms per fwd+bwd step @500k Gaussians 8x 960x540 SH1 RGB+ED; Mpix/s; % HBM roofline",
    3: "ms per forward render @6M Gaussians 1920x1080 SH3; Mpix/s; % HBM roofline",
    4: ("ms per optimizer step (fwd+bwd, absgrad stats, fused Adam) @2M Gaussians "
        "1600x1040 SH3; Mpix/s; % HBM roofline"),
}
HBM_PEAK_GBS = 8000.0
# MI355X: 256 CUs x 128 B/clk of LDS at 2.4 GHz
LDS_PEAK_GBS = 256 * 128 * 2.4
SIMDS = 1024
F32 = 4


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=1, choices=[0, 1, 2, 3, 4])
    ap.add_argument("--unpacked", action="store_true",
                    help="rasterization(packed=False) (dense [C, N] rows)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-copy-bandwidth", action="store_true",
                    help="skip the device-copy bandwidth measurement (profiling runs)")
    ap.add_argument("--no-extra-ops", action="store_true",
                    help="skip the timing of the ops outside the step (profiling runs)")
    ap.add_argument("--cpu-tile-stride", type=int, default=0,
                    help="rasterize every k-th tile in the CPU baseline (0: auto)")
    ap.add_argument("--stages-only", action="store_true",
                    help="print the per-stage breakdown and exit")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a device-to-device copy of 256 MiB x 10 (the "
                         "reference kernel for scaling rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE counters to bytes)")
    return ap.parse_args()


def _copy_calibration():
    """A plain copy of known size: 256 MiB read + 256 MiB written per launch."""
    import torch

    n = 64 * 1024 * 1024  # float32 elements = 256 MiB
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration": {"bytes_read_per_launch": n * 4,
                                           "bytes_written_per_launch": n * 4,
                                           "launches": 10}}))


def _algorithmic_bytes(name, ctx):
    """Algorithmic HBM bytes of one launch of an entry point (each input read
    once, each output written once) -- the roofline numerator."""
    n_isects, nnz, N = ctx["n_isects"], ctx["nnz"], ctx["N"]
    pix, D, tiles = ctx["pixels"], ctx["D"], ctx["tiles"]
    K = ctx["K"]
    gauss2d = 8 + 12 + 4 + F32 * D  # means2d, conic, opacity, colour
    # the replay forms move the same inputs and outputs; their replay state
    # is scratch between the two launches
    if name in ("gsplat_rasterize_fwd", "gsplat_rasterize_fwd_replay"):
        return n_isects * (4 + gauss2d) + tiles * 4 + pix * (F32 * D + 4 + 4 + 4)
    if name in ("gsplat_rasterize_bwd", "gsplat_rasterize_bwd_replay"):
        return (n_isects * (4 + gauss2d) + tiles * 4 + pix * (4 + 4 + F32 * D + 4)
                + nnz * (8 + 12 + F32 * D + 4))
    if name == "gsplat_projection_packed_fwd":
        return N * 44 + nnz * (24 + 8 + 8 + 4 + 12)
    if name == "gsplat_projection_packed_bwd":
        return N * 44 + nnz * (24 + 12 + 8 + 4 + 12) + N * 40
    if name == "gsplat_sh_fwd":
        return nnz * (12 + 12 * K + 1 + 12)
    if name == "gsplat_sh_bwd":
        return nnz * (12 + 12 * K + 1 + 12) + nnz * (12 * K + 12)
    if name == "gsplat_projection_packed_bwd_rows":
        # row map, geometry of the visible Gaussians, the rows' conics and
        # gradients in; dense v_means / v_quats / v_scales out
        return N * 4 * ctx["C"] + nnz * (44 + 12 + 8 + 4 + 12) + N * 40
    if name == "gsplat_sh_rows_fwd":
        # row map, mean + used coefficients of the visible Gaussians in,
        # one colour row per packed row out
        return N * 4 * ctx["C"] + nnz * (12 + 12 * K) + nnz * 12
    if name == "gsplat_sh_rows_bwd":
        return (N * 4 * ctx["C"] + nnz * (12 + 12 * K + 12)
                + N * (12 * K + 12))
    if name == "gsplat_sh_rows_fwd_isect_count":
        # gsplat_sh_rows_fwd plus the count pass: the rows' 32-byte sweep
        # inputs in; their counts, in-block prefixes and records out
        return (N * 4 * ctx["C"] + nnz * (12 + 12 * K) + nnz * 12
                + nnz * (32 + 4 + 8 + 32))
    if name == "gsplat_isect_row_starts":
        return nnz * 16
    if name == "gsplat_projection_packed_bwd_rows_sh":
        # gsplat_projection_packed_bwd_rows plus the SH backward's
        # coefficients and colour gradients in and dense v_coeffs out (the
        # row map, the means and v_means counted once)
        return (N * 4 * ctx["C"] + nnz * (44 + 12 + 8 + 4 + 12) + N * 40
                + nnz * (12 * K + 12) + N * 12 * K)
    if name in ("gsplat_isect_emit_tiles", "gsplat_isect_emit_tiles_dev"):
        # the rows' 32-byte sweep records and starts in; sorted 64-bit ids,
        # rows and tile offsets out
        return nnz * (32 + 8) + n_isects * (8 + 4) + tiles * 4
    if name == "gsplat_adam_multi":
        return ctx.get("adam_elems", 0) * 28
    return None


def _gpu_bench(args):
    import torch

    import gsplat_amd as gs
    from gsplat_amd import _lib
    from gsplat_amd._helper import make_scene

    dev = "cuda:0"
    scene = make_scene(args.config).to(dev)
    C = scene.viewmats.shape[0]
    kw = dict(scene.kwargs)
    if args.unpacked:
        kw["packed"] = False

    if args.config == 4:
        # full optimizer step: raw parameters, absgrad
        # densification statistics, one fused Adam launch over six tensors
        from gsplat_amd.cuda import _ops
        from gsplat_amd.strategy.stats import accumulate_grad2d_stats, fuse_grad2d_stats
        raw = {
            "means": scene.means, "log_scales": scene.log_scales,
            "quats": scene.quats, "opacity_logits": scene.opacity_logits,
            "sh0": scene.colors[:, :1], "shN": scene.colors[:, 1:],
        }
        params = {k: v.clone().contiguous().requires_grad_() for k, v in raw.items()}
        lrs = {"means": 1.6e-4, "log_scales": 5e-3, "quats": 1e-3,
               "opacity_logits": 5e-2, "sh0": 2.5e-3, "shN": 1.25e-4}
        moments = {k: (torch.zeros_like(v), torch.zeros_like(v)) for k, v in params.items()}
        stats = {"grad2d": None, "count": None}
        kw["absgrad"] = True

        def step():
            for p in params.values():
                p.grad = None
            rc, ra, meta = gs.rasterization(
                params["means"], params["quats"], params["log_scales"].exp(),
                torch.sigmoid(params["opacity_logits"]),
                torch.cat([params["sh0"], params["shN"]], dim=1), scene.viewmats,
                scene.Ks, scene.width, scene.height, sh_degree=scene.sh_degree, **kw)
            # the densification statistics join the projection's backward pass
            stats["grad2d"], stats["count"], fused = fuse_grad2d_stats(
                meta, stats["grad2d"], stats["count"], scene.means.shape[0])
            loss = (rc - scene.target).abs().mean()
            loss.backward()
            if not fused:
                stats["grad2d"], stats["count"] = accumulate_grad2d_stats(
                    meta, stats["grad2d"], stats["count"], scene.means.shape[0],
                    packed=True, absgrad=True)
            with torch.no_grad():
                _ops.adam_multi(
                    [(params[k], params[k].grad, moments[k][0], moments[k][1], None,
                      lrs[k]) for k in params], 0.9, 0.999, 1e-15)
            return meta
    elif args.config == 3:
        # large-scene inference render: forward only
        params = {k: getattr(scene, k).contiguous()
                  for k in ("means", "quats", "scales", "opacities", "colors")}

        def step():
            with torch.no_grad():
                rc, ra, meta = gs.rasterization(
                    params["means"], params["quats"], params["scales"],
                    params["opacities"], params["colors"], scene.viewmats, scene.Ks,
                    scene.width, scene.height, sh_degree=scene.sh_degree, **kw)
            return meta
    else:
        params = {k: getattr(scene, k).clone().requires_grad_()
                  for k in ("means", "quats", "scales", "opacities", "colors")}

        def step():
            for p in params.values():
                p.grad = None
            rc, ra, meta = gs.rasterization(
                params["means"], params["quats"], params["scales"], params["opacities"],
                params["colors"], scene.viewmats, scene.Ks, scene.width, scene.height,
                sh_degree=scene.sh_degree, **kw)
            loss = (rc - scene.target).abs().mean()
            loss.backward()
            return meta

    for _ in range(args.warmup):
        meta = step()
    torch.cuda.synchronize()

    # per-stage breakdown (separate pass, every entry point bracketed)
    stage_timer = _lib.EntryTimer()
    with _lib.timing(stage_timer):
        for _ in range(3):
            meta = step()
    torch.cuda.synchronize()
    stages = {k: sum(v) / 3.0 for k, v in stage_timer.results().items()}
    dominant = max(stages, key=stages.get)

    ctx = {
        "n_isects": int(meta["isect_ids"].numel()),
        "nnz": int(meta["means2d"].shape[0]) if meta["means2d"].dim() == 2 else
        int((meta["radii"] > 0).all(-1).sum()),
        "N": scene.means.shape[0],
        "pixels": C * scene.width * scene.height,
        "D": 3 if kw.get("render_mode", "RGB") == "RGB" else 4,
        "tiles": C * meta["tile_width"] * meta["tile_height"],
        "K": scene.colors.shape[-2] if scene.sh_degree is not None else 0,
        "adam_elems": sum(p.numel() for p in params.values()) if args.config == 4 else 0,
        "C": C,
    }

    # timed region: K steps, an event between consecutive steps (per-step
    # times, their median is the metric) and HIP events around the dominant
    # entry point
    torch.cuda.synchronize()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    dom_timer = _lib.EntryTimer({dominant})
    marks[0].record()
    with _lib.timing(dom_timer):
        for k in range(args.steps):
            step()
            marks[k + 1].record()
    torch.cuda.synchronize()
    step_ms = sorted(marks[k].elapsed_time(marks[k + 1]) for k in range(args.steps))
    mean_ms = marks[0].elapsed_time(marks[-1]) / args.steps
    mid = len(step_ms) // 2
    ms_per_step = (step_ms[mid] if len(step_ms) % 2 else
                   0.5 * (step_ms[mid - 1] + step_ms[mid]))
    dom_ms = dom_timer.results()[dominant]
    dom_avg = sum(dom_ms) / len(dom_ms)
    abytes = _algorithmic_bytes(dominant, ctx)
    roofline = None
    if abytes is not None:
        achieved = abytes / (dom_avg * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 5),
                    "traffic": _measured_traffic(dominant, args.config),
                    "kernel": dominant, "avg_ms": round(dom_avg, 4),
                    "algorithmic_bytes": int(abytes)}
    stage_report = {}
    for k, v in sorted(stages.items(), key=lambda kv: -kv[1]):
        ab = _algorithmic_bytes(k, ctx)
        e = {"ms": round(v, 4)}
        if ab is not None and v > 0:
            e["GBps"] = round(ab / (v * 1e-3) / 1e9, 1)
        stage_report[k] = e
    return {
        "ms_per_step": ms_per_step,
        "mean_ms_per_step": mean_ms,
        "step_ms_min_max": (step_ms[0], step_ms[-1]),
        "roofline": roofline,
        "stages": stage_report,
        "extra_ops": None if args.no_extra_ops else _extra_ops(scene, meta, ctx),
        "ctx": ctx,
        "scene": scene,
    }


def _extra_ops(scene, meta, ctx):
    """Timing of the ops outside the training step, on the same workload
    (after the timed region; not part of the metric): covariance/precision
    fwd+bwd for every Gaussian, rasterize-to-indices over the full range of
    the step's intersections, and the densification statistics over its
    rows.  HIP events around each entry point; average of 10 calls."""
    import torch

    from gsplat_amd import _lib
    from gsplat_amd.cuda import _ops

    if meta["means2d"].dim() != 2 or ctx["C"] != 1:  # packed rows of one image
        return None
    dev = scene.means.device
    N, nnz = ctx["N"], ctx["nnz"]
    quats, scales = scene.quats.contiguous(), scene.scales.contiguous()
    v_c = torch.randn(N, 3, 3, device=dev)
    v_p = torch.randn(N, 3, 3, device=dev)
    m2 = meta["means2d"].detach()[None].contiguous()
    con = meta["conics"].detach()[None].contiguous()
    op = meta["opacities"].detach()[None].contiguous()
    T = torch.ones(1, scene.height, scene.width, device=dev)
    offs = meta["isect_offsets"].reshape(1, meta["tile_height"], meta["tile_width"])
    grads = torch.randn(nnz, 2, device=dev) * 1e-3
    ids = meta["gaussian_ids"]
    g2d = torch.zeros(N, device=dev)
    cnt = torch.zeros(N, device=dev)
    n_pairs = [0]

    def run():
        _ops.quat_scale_to_covar_preci_fwd(quats, scales, True, True, False)
        _ops.quat_scale_to_covar_preci_bwd(quats, scales, False, v_c, v_p)
        gi, _ = _ops.rasterize_to_indices_3dgs(0, 1 << 40, T, m2, con, op, scene.width,
                                               scene.height, 16, offs,
                                               meta["flatten_ids"])
        n_pairs[0] = int(gi.numel())
        _ops.grad2d_stats(grads, ids, None, N, 640.0, 360.0, g2d, cnt)

    run()
    torch.cuda.synchronize()
    timer = _lib.EntryTimer()
    with _lib.timing(timer):
        for _ in range(10):
            run()
    torch.cuda.synchronize()
    ms = {k: sum(v) / len(v) for k, v in timer.results().items()}
    algorithmic = {
        "gsplat_quat_scale_to_covar_preci_fwd": N * (16 + 12 + 36 + 36),
        "gsplat_quat_scale_to_covar_preci_bwd": N * (16 + 12 + 36 + 36 + 16 + 12),
        "gsplat_grad2d_stats": nnz * (8 + 8 + 8),
    }
    out = {}
    for k, v in ms.items():
        e = {"ms": round(v, 4)}
        if k in algorithmic and v > 0:
            e["GBps"] = round(algorithmic[k] / (v * 1e-3) / 1e9, 1)
        out[k] = e
    out["rasterize_to_indices_pairs"] = n_pairs[0]
    return out


def _copy_bandwidth():
    """Measured HBM bandwidth of a plain device copy (256 MiB read + 256 MiB
    written per launch, 10 launches, HIP events), reported beside the 8 TB/s
    specification: the practical ceiling of a streaming kernel on this box."""
    import torch

    n = 64 * 1024 * 1024
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(10):
        dst.copy_(src)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / 10
    return {"GBps": round(2 * n * 4 / (ms * 1e-3) / 1e9, 1), "bytes_per_launch": 2 * n * 4,
            "ms_per_launch": round(ms, 4), "spec_GBps": HBM_PEAK_GBS}


def _raster_counters(config):
    """VALU and LDS figures of the two rasterizer kernels from the committed
    rocprofv3 SQ-counter summary of the same workload
    (profiles/cfg<N>_raster_sq_counters.txt), or None.

    valu_busy = SQ_INSTS_VALU x 4 cycles (a wave64 instruction on a 16-lane
    SIMD) / 1,024 SIMDs / (GRBM_GUI_ACTIVE / 8 XCDs); lds_GBps estimates the
    LDS bytes as SQ_INSTS_LDS x 64 lanes x 4 B over the kernel's time
    (GRBM_GUI_ACTIVE / 8 at 2.4 GHz), against 256 CUs x 128 B/clk."""
    f = ROOT / "profiles" / f"cfg{config}_raster_sq_counters.txt"
    if not f.exists():
        return None
    out, cur = {}, None
    for line in f.read_text().splitlines():
        if line.startswith("void gs::rasterize_"):
            cur = "bwd" if "rasterize_bwd" in line else "fwd"
            out[cur] = {}
        elif cur and line.strip() and line.split()[0].isupper():
            k, v = line.split()[:2]
            out[cur][k] = float(v)
    res = {}
    for k, c in out.items():
        if "GRBM_GUI_ACTIVE" not in c or "SQ_INSTS_VALU" not in c:
            continue
        cycles = c["GRBM_GUI_ACTIVE"] / 8.0
        secs = cycles / 2.4e9
        lds_bytes = c.get("SQ_INSTS_LDS", 0.0) * 64 * 4
        res[k] = {"valu_busy": round(c["SQ_INSTS_VALU"] * 4 / SIMDS / cycles, 3),
                  "lds_GBps": round(lds_bytes / secs / 1e9, 1),
                  "lds_peak_GBps": LDS_PEAK_GBS,
                  "lds_bank_conflicts": int(c.get("SQ_LDS_BANK_CONFLICT", 0)),
                  "source": f.name}
    return res or None


def _measured_traffic(kernel, config):
    """HBM bytes per launch of an entry point's kernel, from the committed
    rocprofv3 PMC summary of the same workload (FETCH_SIZE and WRITE_SIZE
    scaled by a plain copy kernel; profiles/cfg1_step_pmc_traffic.txt), or
    None where no such measurement is committed."""
    f = ROOT / "profiles" / f"cfg{config}_step_pmc_traffic.txt"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        parts = line.split()
        if len(parts) == 3 and parts[0] == "traffic" and parts[1] == kernel:
            return int(parts[2])
    return None


def _cpu_baseline(config, stride, packed=True):
    """Oracle pipeline on the host: full projection / SH / intersection for all
    Gaussians plus rasterization on a strided sample of the tiles, fwd+bwd.

    Two samples are timed (every `stride`-th and every `2*stride`-th tile);
    the per-tile raster cost is their difference over the tile-count
    difference, and the full-image step is the fixed part plus that per-tile
    cost times the number of tiles."""
    import torch

    from gsplat_amd._helper import make_scene
    from oracle import torch_ref

    torch.set_num_threads(os.cpu_count() or 1)
    scene = make_scene(config)
    C = scene.viewmats.shape[0]
    tw = math.ceil(scene.width / 16)
    th = math.ceil(scene.height / 16)
    n_tiles = C * tw * th

    fwd_only = config == 3
    moments = {}

    def run(subset):
        leaves = {k: getattr(scene, k).clone().requires_grad_(not fwd_only)
                  for k in ("means", "quats", "scales", "opacities", "colors")}
        t = time.perf_counter()
        with torch.set_grad_enabled(not fwd_only):
            rc, ra, meta = torch_ref.rasterization_ref(
                leaves["means"], leaves["quats"], leaves["scales"], leaves["opacities"],
                leaves["colors"], scene.viewmats, scene.Ks, scene.width, scene.height,
                sh_degree=scene.sh_degree, dtype=torch.float32, tile_subset=subset,
                packed=packed, **scene.kwargs)
        if fwd_only:
            return time.perf_counter() - t
        loss = (rc - scene.target).abs().mean()
        loss.backward()
        if config == 4:
            # the Adam update over the same parameter elements (118M), in torch
            with torch.no_grad():
                for k, p in leaves.items():
                    m, v = moments.setdefault(k, (torch.zeros_like(p), torch.zeros_like(p)))
                    g = p.grad
                    m.mul_(0.9).add_(g, alpha=0.1)
                    v.mul_(0.999).addcmul_(g, g, value=0.001)
                    p.sub_(1e-3 * m / (v.sqrt() + 1e-15))
        return time.perf_counter() - t

    sample_a = list(range(0, n_tiles, stride))
    sample_b = list(range(0, n_tiles, 2 * stride))
    t_b = run(sample_b)
    t_a = run(sample_a)
    per_tile = max(0.0, (t_a - t_b) / max(1, len(sample_a) - len(sample_b)))
    fixed = max(0.0, t_b - per_tile * len(sample_b))
    est = fixed + per_tile * n_tiles
    return {
        "value": round(est * 1e3, 1),
        "unit": "ms/step",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "method": ("extrapolated: fixed part + per-tile rasterization cost x all tiles, "
                   "from two timed strided tile samples"),
        "sample": (f"config {config}: oracle {'fwd' if fwd_only else 'fwd+bwd'}"
                   f"{' + Adam' if config == 4 else ''} with projection+SH+intersection for all "
                   f"{scene.means.shape[0]} Gaussians and rasterization on {len(sample_b)} "
                   f"then {len(sample_a)} of {n_tiles} tiles (strided); took "
                   f"{t_b:.1f}s / {t_a:.1f}s -> fixed {fixed:.1f}s + "
                   f"{per_tile * 1e3:.1f} ms/tile x {n_tiles} tiles"),
    }


def main():
    args = _parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "bench.py runs on exactly one GPU: this build has no "
                          "multi-GPU path (one-GPU boxes only); run with --gpus 1"}))
        sys.exit(2)
    if args.copy_calibration:
        _copy_calibration()
        return
    res = _gpu_bench(args)
    copy_bw = None if args.no_copy_bandwidth else _copy_bandwidth()
    if args.stages_only:
        print(json.dumps(res["stages"], indent=1))
        return
    scene = res["scene"]
    C = scene.viewmats.shape[0]
    mpix = C * scene.width * scene.height / (res["ms_per_step"] * 1e-3) / 1e6
    cpu = None
    if not args.no_cpu_baseline:
        stride = args.cpu_tile_stride or {0: 1, 1: 12, 2: 48, 3: 30, 4: 20}[args.config]
        cpu = _cpu_baseline(args.config, stride, packed=not args.unpacked)
    workload = {
        0: "cfg0: 10k Gaussians, SH0, 256x256, packed, fwd+bwd L1",
        1: "cfg1: 1M Gaussians, SH3, 1280x720, packed, fwd+bwd L1",
        2: "cfg2: 500k Gaussians, SH1, 8x 960x540, packed, RGB+ED, fwd+bwd L1",
        3: "cfg3: 6M Gaussians, SH3, 1920x1080, forward only",
        4: ("cfg4: 2M Gaussians, SH3, 1600x1040, fwd+bwd L1 with absgrad stats and "
            "fused Adam over 6 tensors"),
    }[args.config]
    if args.unpacked:
        workload = workload.replace("packed,", "unpacked (packed=False),")
    out = {
        "metric": METRICS[args.config],
        "value": round(res["ms_per_step"], 4),
        "unit": "ms/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded, gsplat_amd._helper.make_scene)",
        "config": {"workload": workload, "gaussians": int(scene.means.shape[0]),
                   "width": scene.width, "height": scene.height, "cameras": C,
                   "n_isects": res["ctx"]["n_isects"], "visible_rows": res["ctx"]["nnz"]},
        "mpix_per_s": round(mpix, 2),
        "timing": {"statistic": "median of per-step times (HIP events between steps)",
                   "mean_ms_per_step": round(res["mean_ms_per_step"], 4),
                   "min_ms": round(res["step_ms_min_max"][0], 4),
                   "max_ms": round(res["step_ms_min_max"][1], 4)},
        "roofline": res["roofline"],
        "hbm_copy": copy_bw,
        "raster_counters": _raster_counters(args.config),
        "stages_ms": res["stages"],
        "extra_ops_ms": res["extra_ops"],
        "cpu_baseline": cpu,
    }
    if cpu is not None:
        out["speedup_vs_cpu"] = round(cpu["value"] / res["ms_per_step"], 1)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
