#!/usr/bin/env python3
"""Benchmark of the Gaussian-to-Voxel splatting hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3] [--no-cpu]

One step = one forward + one backward of the G2V splat through the reference's module
(``PyCudaGaussianVoxelizer`` forward, then ``torch.autograd.backward`` with the upstream
gradients; the module's autograd function calls the library through the ``_C`` functions) on the
benchmark configuration (BASELINE config 3 by default: 18k Gaussians x 1024-D features into a
200x200x16 grid, all-ones upstream gradients materialised before timing).  Inputs are resident
in HBM before the timed region; synthetic data from tests/workloads.py.

Prints ONE JSON line with ms/step (the metric), forward/backward ms, achieved HBM GB/s over the
compulsory bytes, the roofline of the dominant kernel (per-kernel HIP events recorded by the
library over K further steps run right after the timed ones; the timed steps carry no
instrumentation) and the CPU baseline (the C oracle on a bounded sample, host cores,
extrapolated to one full step).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "shelfgaussian-cudagaussianvoxelizer_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "G2V fwd+bwd ms/step, 18k Gaussians×1024-D, 200×200×16 grid; achieved HBM GB/s"
HBM_PEAK_GBPS = 8000.0
FP32_PEAK_TFLOPS = 157.3
BF16_PEAK_TFLOPS = 2500.0
PUBLISHED_FWD_BWD_MS = 3200.0   # README Table 13, 1x L40S, 18k Gaussians x 1024-D


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3, help="BASELINE config (1-5)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-sample", type=float, default=1.0,
                    help="fraction of tiles (forward) and Gaussians (backward) the CPU baseline runs")
    ap.add_argument("--no-cosine", action="store_true",
                    help="skip the feature cosine-loss leg (the consumer of grid_feats)")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the covariance-construction and batched-scenes legs")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="also run a plain device copy of this size (PMC scale reference)")
    ap.add_argument("--copy-peak-mib", type=int, default=2048,
                    help="size of the device-to-device copy timed in the same run as the measured HBM peak")
    ap.add_argument("--batched-only", action="store_true",
                    help="run only the batched-scenes leg (the recorded batch) and print its result (profiling)")
    return ap.parse_args()


def algorithmic_bytes(N, C, V, M, T, MR):
    """Compulsory HBM bytes per step (every input read once, every output written once) and, per
    kernel, the bytes its own inputs and outputs take when each is moved once.  The intermediates
    of the feature backward count for the kernels that produce and consume them: the split pair
    weights (256 B per G->T pair) and the partial feature-gradient rows (C floats per
    (region, Gaussian) pair)."""
    fwd = 4 * (13 * N + N * C + V + V * C + (N + 1) + M + 16 * N)
    bwd = 4 * (2 * V + V * C + N * C + 4 * N + 16 * N + (N + 1) + M + 13 * N + N * C)
    params = 4 * 19 * N                      # means, opacity, cov_inv, lb, ub
    # each compulsory byte of the step attributed to the first kernel that moves it (the kernels'
    # own intermediates and second reads count for nothing here)
    compulsory = {
        "k_fwd_feats": 4 * (N * C + V + V * C) + params,
        "k_fwd_density": 4 * V + params,
        "k_bwd_tile": 4 * (V * C + 2 * V + N * C + (N + 1) + M) + params,
        "k_bwd_region": 0,
        "k_bwd_gauss": 4 * (13 * N + N * C),
        "k_bwd_density": 4 * (V + 13 * N) + params,
    }
    per_kernel = {
        "k_fwd_feats": 4 * (N * C + (T + 1) + M + V + V * C) + params,
        "k_fwd_density": 4 * ((T + 1) + M + V) + params,
        "k_bwd_tile": 4 * (V * C + N * C + 2 * V + (N + 1) + (T + 1) + M + 10 * M) + 256 * M + params,
        "k_bwd_region": 4 * (V * C + (T + 1) + M + 2 * MR + MR * C) + 256 * M,
        "k_bwd_gauss": 4 * (10 * M + MR * C + 2 * (N + 1) + 13 * N + N * C),
        "k_bwd_density": 4 * (V + 13 * N) + params,
    }
    return fwd, bwd, per_kernel, compulsory


def region_pairs(lb, ub, tiles_z):
    """Number of (region, Gaussian) pairs of the feature backward (regions of 8x8x(4*min(Tz,4)) voxels)."""
    import numpy as np
    cell = np.array([8, 8, 4 * min(tiles_z, 4)])
    lb = np.asarray(lb, np.int64)
    ub = np.asarray(ub, np.int64)
    ok = (ub >= lb).all(axis=1)
    ext = ub // cell - lb // cell + 1
    return int(np.where(ok, ext.prod(axis=1), 0).sum())


def cpu_baseline(w, host, gpu_out, frac):
    """The C oracle (a port of the reference algorithm, float64) on a bounded sample, extrapolated."""
    import numpy as np
    from oracle import g2v_oracle as O
    from oracle import g2v_oracle_c as OC
    m, o, c, f, gD, gF = host
    vs, vr = np.array(w.voxel_size, np.float32), np.array(w.voxel_range, np.float32)
    threads = OC.max_threads()
    t0 = time.perf_counter()
    b = OC.boxes(m, c, vs, vr)
    (X, Y, Z), tiles = O.grid_dims(vs, vr)
    off, tid, gid, toff, sg = OC.csr(b["tile_lo"], b["tile_hi"], tiles)
    t_csr = time.perf_counter() - t0
    Ainv = b["cov_inv"].astype(np.float64)
    T = len(toff) - 1
    n = m.shape[0]
    # forward: 8 tile ranges spread over the grid, frac of all tiles in total
    per = max(1, int(T * frac / 8))
    t_fwd = 0.0
    done_tiles = 0
    for k in range(8):
        a = min(T - per, (k * T) // 8)
        t0 = time.perf_counter()
        OC.forward(m, o, Ainv, b["lb"], b["ub"], vs, vr, toff, sg, f, (X, Y, Z), tile_range=(a, a + per),
                   nthreads=threads)
        t_fwd += time.perf_counter() - t0
        done_tiles += per
    # backward: a contiguous range of Gaussians (their order is random)
    ng = max(1, int(n * frac))
    dens, grid = gpu_out
    t0 = time.perf_counter()
    OC.backward(m, o, Ainv, b["lb"], b["ub"], vs, vr, off, tid, f, dens, grid, gD, gF, g_range=(0, ng),
                nthreads=threads)
    t_bwd = time.perf_counter() - t0
    full_ms = 1e3 * (t_csr + t_fwd * T / done_tiles + t_bwd * n / ng)
    return {"value": round(full_ms, 1), "unit": "ms", "cores": threads, "kind": "port",
            "sample": (f"C oracle (float64 port of the reference tile-major forward and Gaussian-major "
                       f"backward, OpenMP) on {done_tiles}/{T} tiles and {ng}/{n} Gaussians of the same "
                       f"workload, plus the full box+CSR build; extrapolated to one full step "
                       f"(measured {t_csr + t_fwd + t_bwd:.1f} s)"),
            "fwd_ms": round(1e3 * (t_csr + t_fwd * T / done_tiles), 1),
            "bwd_ms": round(1e3 * t_bwd * n / ng, 1)}


def copy_peak(dev, mib, reps=10):
    """Measured HBM peak of this box: a plain device-to-device copy (torch copy_, read + write of
    `mib` MiB each way), best of `reps` after a warm-up, as GB/s of bytes moved."""
    import torch
    src = torch.empty(mib << 18, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    cur = torch.cuda.current_stream(dev)
    best = None
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(cur)
        dst.copy_(src)
        b.record(cur)
        b.synchronize()
        t = a.elapsed_time(b)
        best = t if best is None else min(best, t)
    nbytes = 2 * src.numel() * 4
    del src, dst
    torch.cuda.empty_cache()
    return {"gbps": round(nbytes / (best * 1e-3) / 1e9, 1), "bytes": nbytes, "ms": round(best, 4),
            "method": f"torch copy_ of {mib} MiB device to device (read + write counted), best of {reps}"}


def cosine_leg(_C, grid_feats, steps, warmup):
    """The voxel-wise feature cosine loss (the consumer of grid_feats, reference
    src/cuda_feats_loss.cu) on this config's grid: grid_feats of the G2V forward against a
    synthetic target, 80 % of voxels visible, labels 0..2.  Forward and backward times are the
    library calls' own HIP event spans (the forward includes its one host wait for the count)."""
    import torch
    dev = grid_feats.device
    X, Y, Z, C = grid_feats.shape
    gen = torch.Generator().manual_seed(11)
    label = torch.randint(0, 3, (X, Y, Z), generator=gen).to(torch.float32).to(dev)
    mask = (torch.rand((X, Y, Z), generator=gen) < 0.8).to(dev)
    target = torch.randn((X, Y, Z, C), generator=gen).to(dev)
    gout = torch.ones((), device=dev)

    def run(p, t, esize):
        for _ in range(warmup):
            _, cnt, _ = _C.CudaFeatsCosinelossForward(label, mask, p, t)
            _C.CudaFeatsCosinelossBackward(gout, label, mask, p, t, cnt)
        fwd = bwd = 0.0
        for _ in range(steps):
            _, cnt, f_s = _C.CudaFeatsCosinelossForward(label, mask, p, t)
            grad, b_s = _C.CudaFeatsCosinelossBackward(gout, label, mask, p, t, cnt)
            fwd += f_s
            bwd += b_s
            del grad
        V = X * Y * Z
        fwd_ms, bwd_ms = fwd * 1e3 / steps, bwd * 1e3 / steps
        # compulsory bytes: label + mask of every voxel, both rows of each valid voxel, and the
        # gradient of every voxel (written)
        fwd_b = 5 * V + 2 * esize * cnt * C
        bwd_b = 5 * V + 2 * esize * cnt * C + esize * V * C
        gf, gb = fwd_b / (fwd_ms * 1e-3) / 1e9, bwd_b / (bwd_ms * 1e-3) / 1e9
        return cnt, {"fwd_ms": round(fwd_ms, 4), "bwd_ms": round(bwd_ms, 4), "fwd_bytes": fwd_b,
                     "bwd_bytes": bwd_b, "fwd_gbps": round(gf, 1), "bwd_gbps": round(gb, 1),
                     "fwd_frac": round(gf / HBM_PEAK_GBPS, 4), "bwd_frac": round(gb / HBM_PEAK_GBPS, 4)}

    cnt, res = run(grid_feats, target, 4)
    out = {"grid": [X, Y, Z], "feat_dim": C, "valid_voxels": cnt}
    out.update(res)
    # the same loss on bfloat16 copies of grid_feats and the target (half the row bytes)
    pb, tb = grid_feats.to(torch.bfloat16), target.to(torch.bfloat16)
    _, out["bf16"] = run(pb, tb, 2)
    del pb, tb
    out["data"] = "grid_feats of the G2V forward vs randn target (seed 11), synthetic labels and mask"
    return out


def cosine_fused_leg(w, md, od, cd, fd, gDd, steps, warmup):
    """Voxelizer + feature cosine loss, fwd+bwd of density.gD + loss: chained (the two modules and
    autograd: the loss's backward writes the (X,Y,Z,C) gradient of grid_feats, the voxelizer's
    reads it back) against PyCudaGaussianVoxelizerCosineLoss (that gradient formed inside the
    feature-gradient kernels).  ms per step on the current stream's HIP events (host waits
    included), and the step's peak allocation."""
    import torch
    from CudaGaussianVoxelizer import (PyCudaFeatsCosineLoss, PyCudaGaussianVoxelizer,
                                       PyCudaGaussianVoxelizerCosineLoss, _lib)
    dev = md.device
    X, Y, Z = _grid(w)
    C = fd.shape[1]
    gen = torch.Generator().manual_seed(11)
    label = torch.randint(0, 3, (X, Y, Z), generator=gen).to(torch.float32).to(dev)
    mask = (torch.rand((X, Y, Z), generator=gen) < 0.8).to(dev)
    target = torch.randn((X, Y, Z, C), generator=gen).to(dev)
    one = torch.ones((), device=dev)
    vox = PyCudaGaussianVoxelizer(w.voxel_size, w.voxel_range)
    cos = PyCudaFeatsCosineLoss(w.voxel_size, w.voxel_range)
    fused = PyCudaGaussianVoxelizerCosineLoss(w.voxel_size, w.voxel_range)
    leaves = [t.detach().requires_grad_(True) for t in (md, od, cd, fd)]

    def chained():
        density, grid_feats, _ = vox(*leaves)
        loss, _ = cos(label, mask, grid_feats, target)
        torch.autograd.backward([density, loss], [gDd, one])

    def fused_step():
        density, loss, _, _ = fused(leaves[0], leaves[1], leaves[2], leaves[3], label, mask, target)
        torch.autograd.backward([density, loss], [gDd, one])

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        cur = torch.cuda.current_stream()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(cur)
        for _ in range(steps):
            for t in leaves:
                t.grad = None
            fn()
        b.record(cur)
        b.synchronize()
        ms = round(a.elapsed_time(b) / steps, 4)
        peak = round((torch.cuda.max_memory_allocated() - base) / 1e9, 3)
        # the library's own kernels over as many further steps (HIP event pairs per launch)
        _lib.profile_reset()
        _lib.profile_enable(True)
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        _lib.profile_enable(False)
        prof = _lib.profile_report()
        _lib.profile_reset()
        top = sorted(prof.items(), key=lambda kv: -kv[1][1])[:6]
        return ms, peak, {k: round(v[1] / steps, 4) for k, v in top}

    ch_ms, ch_gb, ch_k = timed(chained)
    fu_ms, fu_gb, fu_k = timed(fused_step)
    return {"grid": [X, Y, Z], "feat_dim": C, "chained_ms": ch_ms, "fused_ms": fu_ms,
            "speedup": round(ch_ms / fu_ms, 3), "chained_step_peak_gb": ch_gb, "fused_step_peak_gb": fu_gb,
            "chained_kernels_ms": ch_k, "fused_kernels_ms": fu_k,
            "data": "the G2V workload with a randn target (seed 11), 80 % of voxels visible, labels 0..2; "
                    "objective density.gD + loss"}


def _grid(w):
    from CudaGaussianVoxelizer import _C
    return _C.grid_dims(w.voxel_size, w.voxel_range)[0]


def covariance_leg(_C, n, steps):
    """Covariances from scales and rotations (reference test/gaussian_voxelizer.py:14-37) for the
    config's Gaussian count, forward and backward: HIP event spans on the current stream, averaged
    over `steps` calls (10 warm-up calls first)."""
    import torch
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(12)
    s = (torch.rand(n, 3, generator=g) + 0.1).to(dev)
    q = torch.randn(n, 4, generator=g).to(dev)
    gc = torch.randn(n, 9, generator=g).to(dev)
    for _ in range(10):
        _C.covariance_from_scale_rotation(s, q)
        _C.covariance_from_scale_rotation_backward(s, q, gc)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    cur = torch.cuda.current_stream(dev)
    ev[0].record(cur)
    for _ in range(steps):
        _C.covariance_from_scale_rotation(s, q)
    ev[1].record(cur)
    for _ in range(steps):
        _C.covariance_from_scale_rotation_backward(s, q, gc)
    ev[2].record(cur)
    ev[2].synchronize()
    fwd_us = ev[0].elapsed_time(ev[1]) * 1e3 / steps
    bwd_us = ev[1].elapsed_time(ev[2]) * 1e3 / steps
    fwd_b, bwd_b = 64 * n, 92 * n   # scales + quaternion in, covariance out; plus grad_cov in, two grads out
    return {"n_gaussians": n, "fwd_us": round(fwd_us, 2), "bwd_us": round(bwd_us, 2),
            "fwd_bytes": fwd_b, "bwd_bytes": bwd_b,
            "note": "back-to-back calls; at this size launch-latency bound, not HBM bound"}


def batched_leg(steps, warmup, per_scene=True):
    """B scenes per call against one call per scene, on the reference's recorded training batch
    (tests/golden/mmdet_debug_inputs.npz: 6 groups of 300 Gaussians, 200x200x16 grid) with
    synthetic 64-D features: fwd+bwd through the module, wall time per batch."""
    import time
    import torch
    from CudaGaussianVoxelizer import PyCudaGaussianVoxelizer
    from tests import workloads as W
    dev = torch.device("cuda", 0)
    m, o, c, vs, vr = W.mmdet_fixture()
    B, n, C = 6, 300, 64
    m, o, c = m.reshape(B, n, 3).to(dev), o.reshape(B, n).to(dev), c.reshape(B, n, 9).to(dev)
    f = torch.randn(B, n, C, generator=torch.Generator().manual_seed(13)).to(dev)
    vox = PyCudaGaussianVoxelizer(list(vs), list(vr))
    leaves = [t.clone().requires_grad_() for t in (m, o, c, f)]
    # all-ones upstream gradients materialised before timing, as in the main step
    with torch.no_grad():
        d0, g0, _ = vox(*leaves)
    gD, gF = torch.ones_like(d0), torch.ones_like(g0)
    del d0, g0

    def batched():
        for t in leaves:
            t.grad = None
        d, g, _ = vox(*leaves)
        torch.autograd.backward([d, g], [gD, gF])

    def looped():
        for b in range(B):
            d, g, _ = vox(*[t[b].detach().requires_grad_() for t in leaves])
            torch.autograd.backward([d, g], [gD[b], gF[b]])

    res = {}
    for name, fn in (("batched", batched), ("per_scene", looped))[:2 if per_scene else 1]:
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        res[name + "_ms"] = round((time.perf_counter() - t0) * 1e3 / steps, 3)
    res.update({"scenes": B, "gaussians_per_scene": n, "feat_dim": C, "grid": [200, 200, 16],
                "data": "recorded batch inputs, randn features (seed 13), all-ones upstream grads materialised before timing"})
    return res


def bf16_leg(md, od, cd, fd, gDd, gFd, vox, steps, warmup):
    """The benchmark step with bfloat16 features (grid_feats and the feature gradient in bfloat16,
    the all-ones upstream gradient of grid_feats in bfloat16 as autograd hands it over and as the
    backward multiplies it)."""
    import time
    import torch
    fb = fd.detach().to(torch.bfloat16).requires_grad_(True)
    gFb = gFd.to(torch.bfloat16)
    leaves = [t for t in (md, od, cd)] + [fb]

    def step():
        for t in leaves:
            t.grad = None
        density, grid_feats, stats = vox(md, od, cd, fb)
        torch.autograd.backward([density, grid_feats], [gDd, gFb])
        return stats

    for _ in range(warmup):
        step()
    fwd = bwd = 0.0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        st = step()
        fwd += float(st[0])
        bwd += float(st[1])
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    return {"ms_per_step": round(ms, 4), "fwd_ms": round(fwd * 1e3 / steps, 4), "bwd_ms": round(bwd * 1e3 / steps, 4),
            "note": "same workload with features, grid_feats and grad_features in bfloat16"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is not supported "
              "(the G2V path runs on a single MI355X; sharding it across GPUs is not built)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from CudaGaussianVoxelizer import _C, _lib
    from tests import workloads as W

    if args.batched_only:
        torch.cuda.set_device(torch.device("cuda", 0))
        res = batched_leg(max(args.steps, 5), args.warmup, per_scene=False)
        print(json.dumps({"metric": "batched scenes fwd+bwd ms (recorded batch, 6 x 300 Gaussians, 64-D)",
                          "value": res["batched_ms"], "unit": "ms", "higher_is_better": False,
                          "batched_scenes": res}), flush=True)
        return

    w = W.CONFIGS[args.config]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    m, o, c, f = W.generate(w, seed=0)
    gD, gF = W.upstream_grads(w)
    C = 0 if f is None else f.shape[1]
    (X, Y, Z), (Tx, Ty, Tz) = _C.grid_dims(w.voxel_size, w.voxel_range)
    if gF is None:
        gF = torch.zeros(X, Y, Z, 0)
    md, od, cd = m.to(dev), o.to(dev), c.to(dev)
    fd = None if f is None else f.to(dev)
    gDd, gFd = gD.to(dev), gF.to(dev)
    vs = torch.tensor(w.voxel_size, dtype=torch.float32, device=dev)
    vr = torch.tensor(w.voxel_range, dtype=torch.float32, device=dev)

    # one step = the reference's module (PyCudaGaussianVoxelizer) forward + autograd backward
    from CudaGaussianVoxelizer import PyCudaGaussianVoxelizer
    vox = PyCudaGaussianVoxelizer(w.voxel_size, w.voxel_range)
    leaves = [t.requires_grad_(True) for t in (md, od, cd) + (() if fd is None else (fd,))]
    outs_grads = [gDd] if C == 0 else [gDd, gFd]

    def step():
        for t in leaves:
            t.grad = None
        density, grid_feats, stats = vox(md, od, cd, fd)
        torch.autograd.backward([density] if C == 0 else [density, grid_feats], outs_grads)
        return stats

    for _ in range(args.warmup):
        step()
    # timed region: K steps of the product path, no instrumentation beyond one event per step
    # boundary on the current stream (for the median)
    fwd_s = bwd_s = 0.0
    torch.cuda.synchronize()
    resident = torch.cuda.memory_allocated(dev)     # inputs and upstream gradients
    torch.cuda.reset_peak_memory_stats(dev)
    cur = torch.cuda.current_stream(dev)
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    t0 = time.perf_counter()
    marks[0].record(cur)
    for i in range(args.steps):
        stats = step()
        marks[i + 1].record(cur)
        fwd_s += float(stats[0])
        bwd_s += float(stats[1])
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    step_ms = sorted(marks[i].elapsed_time(marks[i + 1]) for i in range(args.steps))
    median_ms = step_ms[len(step_ms) // 2] if len(step_ms) % 2 else 0.5 * (step_ms[len(step_ms) // 2 - 1] + step_ms[len(step_ms) // 2])
    peak = torch.cuda.max_memory_allocated(dev)
    memory = {"peak_allocated_gb": round(peak / 1e9, 3), "resident_inputs_gb": round(resident / 1e9, 3),
              "step_peak_gb": round((peak - resident) / 1e9, 3),
              "reference_gb": 4.9 if args.config == 3 else (3.7 if args.config == 2 else None),
              "note": ("torch caching-allocator peak over the timed steps (all device memory the step "
                       "holds: inputs, upstream gradients, outputs and the library's workspaces); "
                       "step_peak_gb leaves out the inputs and upstream gradients resident before the "
                       "step; reference_gb: README.md:98, 1x L40S")}
    # per-kernel times: K more steps with a HIP event pair around every launch of the library,
    # recorded on the stream each kernel runs on (the events add host work, so these steps are
    # timed separately and reported as instrumented_ms_per_step)
    _lib.profile_reset()
    _lib.profile_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    _lib.profile_enable(False)
    prof = _lib.profile_report()
    ms_instr = (t1 - t0) * 1e3 / args.steps
    # workload statistics (untimed): one more forward through the reference-compatible _C call
    with torch.no_grad():
        out = _C.gaussian_voxelizer_forward(md.detach(), od.detach(), cd.detach(), vs, vr,
                                            None if fd is None else fd.detach())
    N = m.shape[0]
    V = X * Y * Z
    T = Tx * Ty * Tz
    M = int(out[7].numel())
    P = int(out[4].to(torch.int64).sum().item())         # in-box (Gaussian, voxel) pairs
    MR = region_pairs(out[2].cpu().numpy(), out[3].cpu().numpy(), Tz) if C else 0
    fwd_b, bwd_b, per_kernel, compulsory = algorithmic_bytes(N, C, V, M, T, MR)
    gbps = (fwd_b + bwd_b) / (ms * 1e-3) / 1e9

    if args.copy_probe_mib > 0:   # a plain copy of known size, the scale of the PMC byte counters
        src = torch.empty(args.copy_probe_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    peak_copy = copy_peak(dev, args.copy_peak_mib) if args.copy_peak_mib > 0 else None
    meas_peak = peak_copy["gbps"] if peak_copy else None

    kernels = {k: {"launches": n_, "avg_ms": round(t_ / max(n_, 1), 4), "total_ms_per_step": round(t_ / args.steps, 4)}
               for k, (n_, t_) in sorted(prof.items(), key=lambda kv: -kv[1][1])}
    dom = max(prof.items(), key=lambda kv: kv[1][1])[0] if prof else None
    roofline = None
    if dom:
        n_, t_ = prof[dom]
        avg_s = t_ / n_ * 1e-3
        bytes_k = per_kernel.get(dom.split("<")[0])   # template arguments are not part of the name
        traffic = None
        tpath = os.path.join(ROOT, "profiles", "pmc_traffic.json")
        if os.path.exists(tpath):
            with open(tpath) as fh:
                tr = json.load(fh).get(f"cfg{args.config}", {}).get(dom)
            if tr:
                traffic = tr.get("bytes_per_launch")
        comp = compulsory.get(dom.split("<")[0])
        if comp is not None:
            # achieved = the launch's share of the step's compulsory bytes (each input read once,
            # each output written once; no intermediates of the design, no second reads) / its
            # average duration
            ach = comp / avg_s / 1e9
            roofline = {"kernel": dom, "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4), "traffic": traffic,
                        "algorithmic_bytes": comp, "avg_ms": round(avg_s * 1e3, 4),
                        "measured_peak": meas_peak,
                        "frac_measured_peak": None if not meas_peak else round(ach / meas_peak, 4),
                        # the same launch credited with every byte its own inputs and outputs take
                        # once, the design's intermediates included (split weights, pair partials)
                        "design_bytes": bytes_k,
                        "design_frac": None if bytes_k is None else round(bytes_k / avg_s / 1e9 / HBM_PEAK_GBPS, 4)}

    covariance = batched = bf16 = None
    if not args.no_extra and C > 0:
        bf16 = bf16_leg(md, od, cd, fd, gDd, gFd, vox, args.steps, args.warmup)
    if not args.no_extra:
        covariance = covariance_leg(_C, N, max(args.steps, 10))
        batched = batched_leg(max(args.steps, 5), args.warmup)
    cosine = None
    if C > 0 and not args.no_cosine:
        cosine = cosine_leg(_C, out[5].detach(), args.steps, args.warmup)
        cosine["fused_backward"] = cosine_fused_leg(w, md, od, cd, fd, gDd, min(args.steps, 10), args.warmup)

    cpu = None
    if not args.no_cpu and args.gpus == 1:
        import numpy as np
        host = (m.numpy(), o.numpy(), c.numpy(), None if f is None else f.numpy(), gD.numpy(),
                None if C == 0 else gF.numpy())
        gpu_out = (out[0].cpu().numpy(), None if C == 0 else out[5].cpu().numpy())
        del out
        cpu = cpu_baseline(w, host, gpu_out, args.cpu_sample)

    flops = 2.0 * P * C + 4.0 * P * C    # forward W.F + backward (G.F^T and W^T.G) contractions
    res = {
        "metric": METRIC, "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": round(ms / PUBLISHED_FWD_BWD_MS, 6) if args.config == 3 else None,
        "vs_baseline_note": "value / 3200 ms (README Table 13 FW+BW on 1x L40S); lower is better",
        "dtype": "f32", "compute": "fp32 in/out; contractions as 3-term bf16-split MFMA with fp32 accumulation",
        "data": "synthetic (tests/workloads.py, seed 0; upstream grads per config)",
        "config": {"workload": w.name, "n_gaussians": N, "feat_dim": C, "grid": [X, Y, Z], "tiles": [Tx, Ty, Tz],
                   "g2t_pairs": M, "region_pairs": MR, "inbox_pairs": P, "upstream_grads": w.grads},
        "fwd_ms": round(fwd_s * 1e3 / args.steps, 4), "bwd_ms": round(bwd_s * 1e3 / args.steps, 4),
        "median_ms_per_step": round(median_ms, 4),
        "median_note": "median of the timed steps' intervals between HIP events recorded at each step boundary",
        "hbm_gbps": round(gbps, 1), "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "hbm_measured_peak": peak_copy,
        "hbm_frac_measured_peak": None if not meas_peak else round(gbps / meas_peak, 4),
        "compulsory_bytes": fwd_b + bwd_b,
        "fp32_equiv_tflops": round(flops / (ms * 1e-3) / 1e12, 2),
        "fp32_frac": round(flops / (ms * 1e-3) / 1e12 / FP32_PEAK_TFLOPS, 4),
        "fp32_note": ("F = 2 P C (forward) + 4 P C (backward) over the in-box pairs P, per step time, "
                      "against the 157.3 TFLOP/s fp32 peak"),
        "roofline": roofline, "memory": memory, "kernels": kernels, "instrumented_ms_per_step": round(ms_instr, 4),
        "kernels_note": ("per-kernel HIP event pairs over K further steps run right after the timed "
                         "region (instrumented_ms_per_step is their wall time per step)"),
        "cpu_baseline": cpu,
        "feats_cosine_loss": cosine,
        "covariance_from_scale_rotation": covariance,
        "batched_scenes": batched,
        "bf16_features": bf16,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
