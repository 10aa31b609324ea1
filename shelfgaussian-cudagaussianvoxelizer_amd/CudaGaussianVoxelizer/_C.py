"""Drop-in for the reference's pybind11 module ``CudaGaussianVoxelizer._C`` (src/bindings.cpp:7-64).

Same function names, keyword arguments, tuple layouts and error behaviour (``RuntimeError``)
as the reference; the work is done by libg2v_hip.so through its C ABI (include/g2v.h) on the
caller's current HIP stream.  Outputs and workspaces come from PyTorch's caching allocator.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

__all__ = ["gaussian_voxelizer_forward", "gaussian_voxelizer_backward", "gaussian_voxelizer_forward_batched",
           "CudaFeatsCosinelossForward", "CudaFeatsCosinelossBackward", "build_t2g", "grid_dims",
           "covariance_from_scale_rotation", "covariance_from_scale_rotation_backward"]


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _host_values(t, n, name):
    """Host floats of voxel_size / voxel_range.  Device tensors are read once per version."""
    if isinstance(t, torch.Tensor):
        if t.numel() != n:
            raise RuntimeError(f"{name} must have {n} elements, got {t.numel()}")
        if t.device.type == "cpu":
            return [float(v) for v in t.detach().reshape(-1).to(torch.float32).tolist()]
        cached = t.__dict__.get("_g2v_host")
        if cached is not None and cached[0] == t._version:
            return cached[1]
        vals = [float(v) for v in t.detach().reshape(-1).to(torch.float32).cpu().tolist()]
        t.__dict__["_g2v_host"] = (t._version, vals)
        return vals
    vals = [float(v) for v in t]
    if len(vals) != n:
        raise RuntimeError(f"{name} must have {n} elements, got {len(vals)}")
    return vals


def grid_dims(voxel_size, voxel_range):
    """((X, Y, Z), (Tx, Ty, Tz)) as the forward computes them (reference .cu:1511-1519)."""
    lib = _lib.load()
    vs = _lib.floats(_host_values(voxel_size, 3, "voxel_size"))
    vr = _lib.floats(_host_values(voxel_range, 6, "voxel_range"))
    dims = (ctypes.c_int * 3)()
    tiles = (ctypes.c_int * 3)()
    _lib.check(lib.g2v_grid_dims(vs, vr, dims, tiles), "g2v_grid_dims")
    return tuple(dims), tuple(tiles)


_GRIDS = {}


def _grid_of(voxel_size, voxel_range):
    """(vs, vr, dims, tiles) of a grid: the ctypes float arrays the C ABI takes and the grid and tile
    dimensions, kept per distinct (voxel_size, voxel_range) values."""
    vs_h = _host_values(voxel_size, 3, "voxel_size")
    vr_h = _host_values(voxel_range, 6, "voxel_range")
    key = tuple(vs_h) + tuple(vr_h)
    g = _GRIDS.get(key)
    if g is None:
        dims, tiles = grid_dims(vs_h, vr_h)
        g = (_lib.floats(vs_h), _lib.floats(vr_h), dims, tiles)
        if len(_GRIDS) < 64:
            _GRIDS[key] = g
    return g


def _f32_input(t, name, shape=None):
    if isinstance(t, torch.Tensor) and t.dtype == torch.float32 \
            and t.is_cuda and t.is_contiguous() and (shape is None or t.shape == shape):
        return t.detach()   # already what the kernels read
    return _f32_input_slow(t, name, shape)


def _f32_input_slow(t, name, shape=None):
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a GPU tensor, got {t.device}")
    if t.dtype != torch.float32:
        raise RuntimeError(f"expected scalar type Float for {name} but found {t.dtype}")
    if shape is not None:
        t = t.reshape(shape)
    return t.detach().contiguous()


_FEAT_DTYPES = {torch.float32: _lib.G2V_DTYPE_F32, torch.bfloat16: _lib.G2V_DTYPE_BF16}


def _feat_input(t, name):
    """Features: float32 or bfloat16 on the GPU (grid_feats and the feature gradient take the
    same type)."""
    if isinstance(t, torch.Tensor) and t.dtype in _FEAT_DTYPES and t.is_cuda and t.is_contiguous():
        return t.detach()
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a GPU tensor, got {t.device}")
    if t.dtype not in _FEAT_DTYPES:
        raise RuntimeError(f"expected scalar type Float or BFloat16 for {name} but found {t.dtype}")
    return t.detach().contiguous()


def _check_saved(t, name, dtype, device):
    if not isinstance(t, torch.Tensor) or t.dtype != dtype or not t.is_contiguous() or t.device != device:
        raise RuntimeError(f"{name} must be a contiguous {dtype} tensor on {device}")


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


_EVENTS = {}
_READY = {}


def _timing_events(device):
    """A (start, stop) pair of timing events per device and thread, reused by every call (each call
    records and synchronises both before it returns)."""
    import threading
    key = (device.index, threading.get_ident())
    ev = _EVENTS.get(key)
    if ev is None:
        ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        _EVENTS[key] = ev
    return ev


def _ready_event(device):
    """An event per device and thread that marks where a host wait ends (no timing)."""
    import threading
    key = (device.index, threading.get_ident())
    ev = _READY.get(key)
    if ev is None:
        ev = torch.cuda.Event()
        _READY[key] = ev
    return ev


class _OnDevice:
    """torch.cuda.device(dev) only when dev is not already the current device."""

    def __init__(self, dev):
        self.ctx = None if dev.index == torch.cuda.current_device() else torch.cuda.device(dev)

    def __enter__(self):
        if self.ctx is not None:
            self.ctx.__enter__()

    def __exit__(self, *exc):
        if self.ctx is not None:
            self.ctx.__exit__(*exc)
        return False


def gaussian_voxelizer_forward(means3D, opacity, covariances, voxel_size, voxel_range, features=None):
    """Gaussian voxelization forward pass.

    Args:
        means3D (N,3), opacity (N,) (or (N,1)), covariances (N,9) row-major 3x3 (or (N,3,3)),
        voxel_size (3,), voxel_range (6,) [x_min, y_min, z_min, x_max, y_max, z_max],
        features (N,C) or None.  All float32 on the GPU.
    Returns the reference's 9-tuple (src/cuda_gaussian_voxelizer.cu:1913):
        density (X,Y,Z), cov_inv (N,9), valid_voxel_lb (N,3) int32, valid_voxel_ub (N,3) int32,
        num_voxels_per_gaussian (N,) int32, grid_feats (X,Y,Z,C) (C = 0 without features),
        g2t_offsets (N+1,) int32, g2t_tile_ids (M,) int32, forward time in seconds.
    """
    return _forward(means3D, opacity, covariances, voxel_size, voxel_range, features, keep_t2g=False)[0]


def _forward(means3D, opacity, covariances, voxel_size, voxel_range, features, keep_t2g):
    """The forward; with keep_t2g it also returns, beside the 9-tuple, what the backward would
    otherwise recompute: the Tile->Gaussian CSR (sorted tiles, sorted Gaussians, tile offsets) and
    the backward plan (region pair offsets and their count, counted on the plan's one sync)."""
    lib = _lib.load()
    means = _f32_input(means3D, "means3D")
    if means.dim() != 2 or means.shape[1] != 3:
        raise RuntimeError(f"means3D must be (N, 3), got {tuple(means.shape)}")
    n = means.shape[0]
    dev = means.device
    op = _f32_input(opacity, "opacity", (n,))
    cov = _f32_input(covariances, "covariances", (n, 9))
    feats = None
    C = 0
    if features is not None:
        feats = _feat_input(features, "features")
        if feats.dim() != 2 or feats.shape[0] != n:
            raise RuntimeError(f"features must be (N, C) with N = {n}, got {tuple(feats.shape)}")
        C = feats.shape[1]
        if C == 0:
            feats = None
    vs, vr, (X, Y, Z), (Tx, Ty, Tz) = _grid_of(voxel_size, voxel_range)

    with _OnDevice(dev):
        cur = torch.cuda.current_stream(dev)
        stream = ctypes.c_void_p(cur.cuda_stream)
        i32 = dict(dtype=torch.int32, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        cov_inv = torch.empty(n, 9, **f32)
        lb = torch.empty(n, 3, **i32)
        ub = torch.empty(n, 3, **i32)
        nvox = torch.empty(n, **i32)
        g2t_offsets = torch.empty(n + 1, **i32)
        # the plan's workspace and, with keep_t2g, the backward plan's (the (region, Gaussian) pair
        # count is done here too, on the same wait; the backward reads that workspace later), in
        # one allocation
        pws = lib.g2v_forward_plan_workspace(n)
        pws_al = (pws + 255) & ~255
        # (without features the backward needs neither the CSR nor a plan: it walks the boxes)
        keep_csr = keep_t2g and feats is not None
        bws = max(1, lib.g2v_backward_plan_workspace(n)) if keep_csr else 0
        wsb = torch.empty(pws_al + bws, dtype=torch.uint8, device=dev)
        ws = wsb[:pws]
        bplan = wsb[pws_al:] if keep_csr else None
        counts = _pinned_counts(dev, 2)
        start, stop = _timing_events(dev)
        start.record(cur)
        _lib.check(lib.g2v_forward_plan_async(n, _ptr(means), _ptr(cov), vs, vr, _ptr(cov_inv), _ptr(lb),
                                              _ptr(ub), _ptr(nvox), _ptr(g2t_offsets), _ptr(ws), ws.numel(),
                                              _ptr(bplan), 0 if bplan is None else bplan.numel(), _ptr(counts),
                                              stream),
                   "gaussian_voxelizer_forward (plan)")
        ready = _ready_event(dev)
        ready.record(cur)
        # queued behind the plan, so that they run while this thread waits for the pair counts:
        # the features packed for the splat; then the outputs whose size does not depend on the
        # counts are allocated
        fdtype = torch.float32 if feats is None else feats.dtype
        fdt = _FEAT_DTYPES[fdtype]
        packed = None
        if feats is not None:
            packed = torch.empty(lib.g2v_forward_packed_bytes(n, C), dtype=torch.uint8, device=dev)
            _lib.check(lib.g2v_forward_pack_features(n, C, _ptr(feats), fdt, _ptr(packed), packed.numel(), stream),
                       "gaussian_voxelizer_forward (features)")
        density = torch.empty(X, Y, Z, **f32)
        grid_feats = torch.empty(X, Y, Z, C, dtype=fdtype, device=dev)
        t2g_toff = torch.empty(Tx * Ty * Tz + 1, **i32) if keep_csr else None
        ready.synchronize()
        M, MR = (int(v) for v in counts.tolist())
        for cnt, what in ((M, "Gaussian-tile"), (MR, "region-Gaussian")):
            if cnt > 2147483647:
                raise RuntimeError(f"gaussian_voxelizer_forward (plan): {cnt} {what} pairs exceed the int32 CSR "
                                   "(limit 2^31-1)")
        g2t_tile_ids = torch.empty(M, **i32)
        ws2 = torch.empty(lib.g2v_forward_splat_workspace(n, C, M, vs, vr), dtype=torch.uint8, device=dev)
        t2g = None
        csr = (None, None, None)
        if keep_t2g:
            if keep_csr:
                csr = (torch.empty(M, **i32), torch.empty(M, **i32), t2g_toff)
            t2g = dict(csr=csr, plan=bplan, num_region_pairs=MR, vs=vs, vr=vr, dims=(X, Y, Z))
        _lib.check(lib.g2v_forward_splat(n, C, _ptr(means), _ptr(op), _ptr(feats), fdt, _ptr(packed),
                                         0 if packed is None else packed.numel(), vs, vr,
                                         _ptr(cov_inv), _ptr(lb), _ptr(ub), _ptr(g2t_offsets), M,
                                         _ptr(g2t_tile_ids), _ptr(density), _ptr(grid_feats),
                                         _ptr(csr[0]), _ptr(csr[1]), _ptr(csr[2]),
                                         _ptr(ws2), ws2.numel(), stream),
                   "gaussian_voxelizer_forward (splat)")
        stop.record(cur)
        if keep_t2g:
            # the backward's outputs and workspace, allocated while the forward kernels run
            t2g["grads"] = (torch.empty(n, 3, **f32), torch.empty(n, 9, **f32), torch.empty(n, **f32),
                            torch.empty(n, C, dtype=fdtype, device=dev))
            t2g["ws"] = torch.empty(max(1, lib.g2v_backward_workspace(n, C, M, t2g["num_region_pairs"], vs, vr)),
                                    dtype=torch.uint8, device=dev) if C > 0 else None
            # the backward's gradient-independent kernels, queued behind the forward (after its
            # stop event): they run while this thread waits and hands over to the backward
            if C > 0:
                _lib.check(lib.g2v_backward_prepare(n, C, vs, vr, _ptr(lb), _ptr(ub), _ptr(feats), fdt, M,
                                                    t2g["num_region_pairs"], _ptr(csr[0]), _ptr(csr[1]),
                                                    _ptr(bplan), _ptr(t2g["ws"]), t2g["ws"].numel(), stream),
                           "gaussian_voxelizer_forward (backward preparation)")
                t2g["prepared"] = True
        stop.synchronize()
        fwd_sec = start.elapsed_time(stop) / 1000.0
    return (density, cov_inv, lb, ub, nvox, grid_feats, g2t_offsets, g2t_tile_ids, fwd_sec), t2g


def gaussian_voxelizer_backward(grad_output, grad_feats_output, means3D, opacity, cov_inv, voxel_size,
                                voxel_range, valid_voxel_lb, valid_voxel_ub, num_voxels_per_gaussian,
                                g2t_offsets, g2t_tile_ids, density, grid_feats, features=None):
    """Gaussian voxelization backward pass (reference src/cuda_gaussian_voxelizer.cu:1920-2057).

    Returns the reference's 5-tuple: grad_means (N,3), grad_cov (N,9), grad_opacity (N,),
    grad_feats (N,C) (N,0 without features), backward time in seconds.
    """
    return _backward(grad_output, grad_feats_output, means3D, opacity, cov_inv, voxel_size, voxel_range,
                     valid_voxel_lb, valid_voxel_ub, num_voxels_per_gaussian, g2t_offsets, g2t_tile_ids,
                     density, grid_feats, features, t2g=None)


def gaussian_voxelizer_backward_cosine(grad_output, grad_loss, pseudo_dino_gt, coef, num_valid_voxel, means3D,
                                       opacity, cov_inv, voxel_size, voxel_range, valid_voxel_lb, valid_voxel_ub,
                                       num_voxels_per_gaussian, g2t_offsets, g2t_tile_ids, density, grid_feats,
                                       features):
    """gaussian_voxelizer_backward with the feature cosine loss's gradient as the upstream gradient
    of grid_feats, fused (g2v_backward_cosine): the (X,Y,Z,C) gradient that the reference's
    CudaFeatsCosinelossBackward writes and its voxelizer backward reads (src/cuda_feats_loss.cu:
    311-366, src/cuda_gaussian_voxelizer.cu:1920-2057) is formed per voxel inside the kernels.
    grad_loss: the upstream gradient of the loss (one-element GPU tensor); coef and num_valid_voxel
    as _cosine_forward(..., want_coef=True) returned them for this grid_feats and pseudo_dino_gt
    (float32, C % 4 == 0).  Returns gaussian_voxelizer_backward's 5-tuple."""
    gl = grad_loss.detach().to(device=means3D.device, dtype=torch.float32).reshape(1).contiguous()
    return _backward(grad_output, None, means3D, opacity, cov_inv, voxel_size, voxel_range, valid_voxel_lb,
                     valid_voxel_ub, num_voxels_per_gaussian, g2t_offsets, g2t_tile_ids, density, grid_feats,
                     features, t2g=None, cosine=(gl, pseudo_dino_gt, coef, num_valid_voxel))


def _backward(grad_output, grad_feats_output, means3D, opacity, cov_inv, voxel_size, voxel_range,
              valid_voxel_lb, valid_voxel_ub, num_voxels_per_gaussian, g2t_offsets, g2t_tile_ids,
              density, grid_feats, features, t2g, timed=True, cosine=None):
    """The backward; t2g is what _forward(keep_t2g=True) returned beside the 9-tuple, or None.
    With t2g the saved tensors are the forward's own outputs (already checked there), and the
    grid, plan, outputs and workspace come from the forward: only the upstream gradients are
    checked here.  cosine = (grad_loss, pseudo_dino_gt, coef, num_valid_voxel): the upstream
    gradient of grid_feats is the cosine loss's, formed inside the kernels (grad_feats_output is
    ignored)."""
    lib = _lib.load()
    if not isinstance(means3D, torch.Tensor) or means3D.device.type != "cuda":
        raise RuntimeError("means3D must be a GPU tensor")
    dev = means3D.device
    f32, i32 = torch.float32, torch.int32
    trusted = t2g is not None and "grads" in t2g
    if trusted:
        vs, vr = t2g["vs"], t2g["vr"]
        X, Y, Z = t2g["dims"]
        _check_saved(grad_output, "grad_output", f32, dev)
    else:
        for t, name in ((grad_output, "grad_output"), (means3D, "means3D"), (opacity, "opacity"),
                        (cov_inv, "cov_inv"), (density, "density")):
            _check_saved(t, name, f32, dev)
        _check_saved(grid_feats, "grid_feats", grid_feats.dtype if grid_feats.dtype in _FEAT_DTYPES else f32, dev)
        for t, name in ((valid_voxel_lb, "valid_voxel_lb"), (valid_voxel_ub, "valid_voxel_ub"),
                        (num_voxels_per_gaussian, "num_voxels_per_gaussian"), (g2t_offsets, "g2t_offsets"),
                        (g2t_tile_ids, "g2t_tile_ids")):
            _check_saved(t, name, i32, dev)
        vs_h = _host_values(voxel_size, 3, "voxel_size")
        vr_h = _host_values(voxel_range, 6, "voxel_range")
        vs, vr = _lib.floats(vs_h), _lib.floats(vr_h)
        (X, Y, Z), _ = grid_dims(vs_h, vr_h)
    n = means3D.shape[0]
    if g2t_offsets.numel() != n + 1:
        raise RuntimeError(f"g2t_offsets must have N+1 = {n + 1} elements, got {g2t_offsets.numel()}")
    if tuple(grad_output.shape) != (X, Y, Z):
        raise RuntimeError(f"grad_output must be {(X, Y, Z)}, got {tuple(grad_output.shape)}")
    C = 0
    feats = gF = None
    fdtype = f32
    if features is not None:
        if not trusted:
            _check_saved(features, "features", features.dtype if features.dtype in _FEAT_DTYPES else f32, dev)
        C = features.shape[1]
        fdtype = features.dtype
        if C > 0:
            feats = features
            if grid_feats.dtype != fdtype:
                raise RuntimeError(f"grid_feats ({grid_feats.dtype}) and features ({fdtype}) differ in type")
            if cosine is not None:
                grad_feats_output = cosine[1]   # checked as the stand-in upstream tensor
                coef, gl = cosine[2], cosine[0]
                _check_saved(coef, "coef", f32, dev)
                _check_saved(gl, "grad_loss", f32, dev)
                if tuple(coef.shape) != (X * Y * Z, 2) or gl.numel() != 1:
                    raise RuntimeError(f"coef must be ({X * Y * Z}, 2) and grad_loss one element")
                if fdtype != f32 or C % 4 != 0:
                    raise RuntimeError("the fused cosine gradient takes float32 features with C % 4 == 0")
            else:
                # the upstream feature gradient is taken in the features' type (a float32 gradient of
                # bfloat16 features is rounded to bfloat16, a bfloat16 one of float32 features widened)
                if isinstance(grad_feats_output, torch.Tensor) and grad_feats_output.dtype != fdtype \
                        and grad_feats_output.dtype in _FEAT_DTYPES:
                    grad_feats_output = grad_feats_output.to(fdtype).contiguous()
            _check_saved(grad_feats_output, "pseudo_dino_gt" if cosine is not None else "grad_feats_output",
                         fdtype, dev)
            if tuple(grad_feats_output.shape) != (X, Y, Z, C) or tuple(grid_feats.shape) != (X, Y, Z, C):
                raise RuntimeError("grad_feats_output and grid_feats must be (X, Y, Z, C)")
            gF = grad_feats_output
    fdt = _FEAT_DTYPES[fdtype]
    M = g2t_tile_ids.numel()

    with _OnDevice(dev):
        cur = torch.cuda.current_stream(dev)
        stream = ctypes.c_void_p(cur.cuda_stream)
        if trusted:   # allocated by the forward
            grad_means, grad_cov, grad_opacity, grad_feats = t2g["grads"]
        else:
            grad_means = torch.empty(n, 3, dtype=f32, device=dev)
            grad_cov = torch.empty(n, 9, dtype=f32, device=dev)
            grad_opacity = torch.empty(n, dtype=f32, device=dev)
            grad_feats = torch.empty(n, C, dtype=fdtype, device=dev)
        if timed:
            start, stop = _timing_events(dev)
            start.record(cur)
        if C == 0:   # the density-only backward walks the boxes: no plan, no workspace
            plan_ws, MR = None, 0
        elif t2g is not None:   # planned by the forward
            plan_ws, MR = t2g["plan"], t2g["num_region_pairs"]
        else:
            plan_ws = torch.empty(max(1, lib.g2v_backward_plan_workspace(n)), dtype=torch.uint8, device=dev)
            MR = ctypes.c_longlong(0)
            _lib.check(lib.g2v_backward_plan(n, C, vs, vr, _ptr(valid_voxel_lb), _ptr(valid_voxel_ub),
                                             _ptr(plan_ws), plan_ws.numel(), ctypes.byref(MR), stream),
                       "gaussian_voxelizer_backward (plan)")
            MR = int(MR.value)
        if C == 0:
            ws = None
        elif trusted:
            ws = t2g["ws"]
        else:
            ws = torch.empty(max(1, lib.g2v_backward_workspace(n, C, M, MR, vs, vr)), dtype=torch.uint8, device=dev)
        csr = t2g["csr"] if t2g else (None, None, None)
        # the forward queued the gradient-independent part into this workspace
        prepared = bool(trusted and C > 0 and t2g.get("prepared"))
        if cosine is not None and C > 0:
            grad_loss, _, coef, num_valid = cosine
            _lib.check(lib.g2v_backward_cosine(n, C, _ptr(grad_output), _ptr(grad_loss), _ptr(gF), _ptr(coef),
                                               int(num_valid), _ptr(means3D), _ptr(opacity), _ptr(cov_inv), vs, vr,
                                               _ptr(valid_voxel_lb), _ptr(valid_voxel_ub),
                                               _ptr(num_voxels_per_gaussian), _ptr(g2t_offsets),
                                               _ptr(g2t_tile_ids), M, MR, _ptr(density), _ptr(grid_feats),
                                               _ptr(feats), fdt, _ptr(grad_means), _ptr(grad_cov),
                                               _ptr(grad_opacity), _ptr(grad_feats), _ptr(csr[0]), _ptr(csr[1]),
                                               _ptr(csr[2]), _ptr(plan_ws), _ptr(ws), ws.numel(), int(prepared),
                                               stream),
                       "gaussian_voxelizer_backward_cosine")
        else:
            entry = lib.g2v_backward_prepared if prepared else lib.g2v_backward
            _lib.check(entry(n, C, _ptr(grad_output), _ptr(gF), _ptr(means3D), _ptr(opacity),
                             _ptr(cov_inv), vs, vr, _ptr(valid_voxel_lb), _ptr(valid_voxel_ub),
                             _ptr(num_voxels_per_gaussian), _ptr(g2t_offsets), _ptr(g2t_tile_ids),
                             M, MR, _ptr(density), _ptr(grid_feats), _ptr(feats), fdt,
                             _ptr(grad_means), _ptr(grad_cov), _ptr(grad_opacity),
                             _ptr(grad_feats), _ptr(csr[0]), _ptr(csr[1]), _ptr(csr[2]),
                             _ptr(plan_ws), _ptr(ws), 0 if ws is None else ws.numel(), stream),
                       "gaussian_voxelizer_backward")
        bwd_sec = 0.0
        if timed:
            stop.record(cur)
            stop.synchronize()
            bwd_sec = start.elapsed_time(stop) / 1000.0
    return (grad_means, grad_cov, grad_opacity, grad_feats, bwd_sec)


_COUNTS = {}


def _pinned_counts(dev, k):
    """A reusable pinned (k,) int64 host buffer per device and thread (count read-back)."""
    import threading
    key = (dev.index, threading.get_ident())
    buf = _COUNTS.get(key)
    if buf is None or buf.numel() < k:
        buf = torch.empty(max(k, 16), dtype=torch.int64, pin_memory=True)
        _COUNTS[key] = buf
    return buf[:k]


def gaussian_voxelizer_forward_batched(means3D, opacity, covariances, voxel_size, voxel_range, features=None):
    """Forward of B scenes on one grid in one call: means3D (B,N,3), opacity (B,N) or (B,N,1),
    covariances (B,N,9) or (B,N,3,3), features (B,N,C) or None.

    The B scenes run as one problem of B N Gaussians (one launch per kernel for the whole batch,
    one host wait for its pair counts).  Returns a list of B 9-tuples laid out as
    gaussian_voxelizer_forward's, each equal to that of the scene alone; the density and
    grid_feats of scene b are the views [b] of one (B,X,Y,Z) and one (B,X,Y,Z,C) tensor, and the
    time in every tuple is that of the whole batch.
    """
    return _forward_batched(means3D, opacity, covariances, voxel_size, voxel_range, features, keep_t2g=False)[0]


def _forward_batched(means3D, opacity, covariances, voxel_size, voxel_range, features, keep_t2g):
    """Batched forward.  Returns ([9-tuple per scene], density (B,X,Y,Z), grid_feats (B,X,Y,Z,C),
    batch) where batch holds what _backward_batched needs (the batch plan, the batch's
    Tile->Gaussian CSR, the prepared backward workspace) with keep_t2g, else None."""
    lib = _lib.load()
    means = _f32_input(means3D, "means3D")
    if means.dim() != 3 or means.shape[2] != 3:
        raise RuntimeError(f"batched means3D must be (B, N, 3), got {tuple(means.shape)}")
    B, n = means.shape[0], means.shape[1]
    dev = means.device
    op = _f32_input(opacity, "opacity", (B, n))
    cov = _f32_input(covariances, "covariances", (B, n, 9))
    feats = None
    C = 0
    if features is not None:
        feats = _feat_input(features, "features")
        if feats.dim() != 3 or tuple(feats.shape[:2]) != (B, n):
            raise RuntimeError(f"features must be (B, N, C) with B, N = {B}, {n}, got {tuple(feats.shape)}")
        C = feats.shape[2]
        if C == 0:
            feats = None
    vs_h = _host_values(voxel_size, 3, "voxel_size")
    vr_h = _host_values(voxel_range, 6, "voxel_range")
    vs, vr = _lib.floats(vs_h), _lib.floats(vr_h)
    (X, Y, Z), (Tx, Ty, Tz) = grid_dims(vs_h, vr_h)
    T = Tx * Ty * Tz
    if B == 0:
        f32 = dict(dtype=torch.float32, device=dev)
        return [], torch.empty(0, X, Y, Z, **f32), torch.empty(0, X, Y, Z, C, dtype=torch.float32 if feats is None
                                                                 else feats.dtype, device=dev), None

    with _OnDevice(dev):
        cur = torch.cuda.current_stream(dev)
        stream = ctypes.c_void_p(cur.cuda_stream)
        i32 = dict(dtype=torch.int32, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        cov_inv = torch.empty(B, n, 9, **f32)
        lb = torch.empty(B, n, 3, **i32)
        ub = torch.empty(B, n, 3, **i32)
        nvox = torch.empty(B, n, **i32)
        g2t_offsets = torch.empty(B, n + 1, **i32)
        pws = lib.g2v_batch_plan_workspace(B, n)
        if pws == 0:
            raise RuntimeError(f"batch of {B} scenes x {n} Gaussians exceeds the int32 Gaussian index")
        plan = torch.empty(pws, dtype=torch.uint8, device=dev)
        counts_dev = torch.empty(B + 1, dtype=torch.int64, device=dev)
        # outputs whose size does not depend on the plan's counts, allocated before its host wait
        density = torch.empty(B, X, Y, Z, **f32)
        fdtype = torch.float32 if feats is None else feats.dtype
        fdt = _FEAT_DTYPES[fdtype]
        grid_feats = torch.empty(B, X, Y, Z, C, dtype=fdtype, device=dev)
        start, stop = _timing_events(dev)
        start.record(cur)
        # the (region, Gaussian) pair count of the backward rides on the same launches and wait
        want_bwd = 1 if (keep_t2g and C > 0) else 0
        _lib.check(lib.g2v_batch_forward_plan(B, n, _ptr(means), _ptr(cov), vs, vr, _ptr(cov_inv), _ptr(lb), _ptr(ub),
                                              _ptr(nvox), _ptr(g2t_offsets), _ptr(plan), pws, want_bwd,
                                              _ptr(counts_dev), stream),
                   "gaussian_voxelizer_forward_batched (plan)")
        counts = _pinned_counts(dev, B + 1)
        counts.copy_(counts_dev, non_blocking=True)
        cur.synchronize()   # the one host wait of the batch
        cnt = counts.tolist()
        Ms, MR = [int(v) for v in cnt[:B]], int(cnt[B])
        M = sum(Ms)
        if M > 2147483647 or MR > 2147483647:
            raise RuntimeError(f"batch pair counts {M}, {MR} exceed the int32 CSR")
        g2t_tile_ids = torch.empty(M, **i32)
        ws = torch.empty(lib.g2v_batch_forward_splat_workspace(B, n, C, M, vs, vr), dtype=torch.uint8, device=dev)
        csr = (torch.empty(M, **i32), torch.empty(M, **i32), torch.empty(B * T + 1, **i32)) if keep_t2g \
            else (None, None, None)
        _lib.check(lib.g2v_batch_forward_splat(B, n, C, _ptr(means), _ptr(op), _ptr(feats), fdt, vs, vr, _ptr(cov_inv),
                                               _ptr(lb), _ptr(ub), _ptr(plan), pws, M, _ptr(g2t_tile_ids),
                                               _ptr(density), _ptr(grid_feats), _ptr(csr[0]), _ptr(csr[1]),
                                               _ptr(csr[2]), _ptr(ws), ws.numel(), stream),
                   "gaussian_voxelizer_forward_batched (splat)")
        stop.record(cur)
        batch = None
        if keep_t2g:
            # the backward's outputs and workspace, and its gradient-independent kernels queued
            # behind the forward (after its stop event), as for one scene
            batch = dict(B=B, n=n, C=C, fdt=fdt, M=M, MR=MR, vs=vs, vr=vr, plan=plan, csr=csr, cov_inv=cov_inv,
                         lb=lb, ub=ub, density=density, grid_feats=grid_feats, prepared=False)
            batch["grads"] = (torch.empty(B, n, 3, **f32), torch.empty(B, n, 9, **f32), torch.empty(B, n, **f32),
                              torch.empty(B, n, C, dtype=fdtype, device=dev))
            batch["ws"] = torch.empty(max(1, lib.g2v_batch_backward_workspace(B, n, C, M, MR, vs, vr)),
                                      dtype=torch.uint8, device=dev)
            if C > 0:
                _lib.check(lib.g2v_batch_backward_prepare(B, n, C, vs, vr, _ptr(lb), _ptr(ub), _ptr(feats), fdt, M, MR,
                                                          _ptr(csr[0]), _ptr(csr[1]), _ptr(plan), pws,
                                                          _ptr(batch["ws"]), batch["ws"].numel(), stream),
                           "gaussian_voxelizer_forward_batched (backward preparation)")
                batch["prepared"] = True
        stop.synchronize()
        fwd_sec = start.elapsed_time(stop) / 1000.0
    out, off = [], 0
    for b in range(B):
        out.append((density[b], cov_inv[b], lb[b], ub[b], nvox[b], grid_feats[b], g2t_offsets[b],
                    g2t_tile_ids[off:off + Ms[b]], fwd_sec))
        off += Ms[b]
    return out, density, grid_feats, batch


def _backward_batched(grad_density, grad_feats, means, opacity, features, batch):
    """Backward of _forward_batched(keep_t2g=True): grad_density (B,X,Y,Z), grad_feats (B,X,Y,Z,C)
    (or None: zero); batch = its fourth result.  One g2v_batch_backward call for the B scenes.
    Returns the gradients (B,N,3), (B,N,9), (B,N), (B,N,C) and the time of the batch."""
    lib = _lib.load()
    dev = means.device
    B, n, C, fdt = batch["B"], batch["n"], batch["C"], batch["fdt"]
    gD = _f32_input(grad_density, "grad_density", tuple(batch["density"].shape))
    gF = None
    if C > 0:
        gfeat = batch["grid_feats"]
        gF = grad_feats if grad_feats is not None and grad_feats.shape[-1] > 0 else torch.zeros_like(gfeat)
        if tuple(gF.shape) != tuple(gfeat.shape):
            raise RuntimeError(f"grad_feats_output must be {tuple(gfeat.shape)}, got {tuple(gF.shape)}")
        gF = gF.to(gfeat.dtype).contiguous()
    gm, gc, go, gf = batch["grads"]
    csr, plan = batch["csr"], batch["plan"]
    with _OnDevice(dev):
        cur = torch.cuda.current_stream(dev)
        start, stop = _timing_events(dev)
        start.record(cur)
        _lib.check(lib.g2v_batch_backward(B, n, C, _ptr(gD), _ptr(gF), _ptr(means), _ptr(opacity), _ptr(batch["cov_inv"]),
                                          batch["vs"], batch["vr"], _ptr(batch["lb"]), _ptr(batch["ub"]), batch["M"],
                                          batch["MR"], _ptr(batch["density"]), _ptr(batch["grid_feats"]),
                                          _ptr(features), fdt, _ptr(gm), _ptr(gc), _ptr(go), _ptr(gf), _ptr(csr[0]),
                                          _ptr(csr[1]), _ptr(csr[2]), _ptr(plan), plan.numel(), _ptr(batch["ws"]),
                                          batch["ws"].numel(), 1 if batch["prepared"] else 0,
                                          ctypes.c_void_p(cur.cuda_stream)),
                   "gaussian_voxelizer_backward (batched)")
        stop.record(cur)
        stop.synchronize()
        bwd_sec = start.elapsed_time(stop) / 1000.0
    return gm, gc, go, gf, bwd_sec


def build_t2g(voxel_size, voxel_range, valid_voxel_lb, valid_voxel_ub, g2t_offsets, g2t_tile_ids):
    """The forward's internal Tile->Gaussian CSR, for inspection and parity tests.

    Returns a dict: sorted_tiles (M,), sorted_gauss (M,), tile_offsets (T+1,), and the run-length
    encoding unique_tiles (U,), counts (U,), runs_offsets (U+1,), num_runs.
    """
    lib = _lib.load()
    dev = g2t_offsets.device
    n = g2t_offsets.numel() - 1
    M = g2t_tile_ids.numel()
    vs, vr = _lib.floats(_host_values(voxel_size, 3, "voxel_size")), _lib.floats(_host_values(voxel_range, 6, "voxel_range"))
    (_, tiles) = grid_dims(list(vs), list(vr))
    T = tiles[0] * tiles[1] * tiles[2]
    with torch.cuda.device(dev):
        i32 = dict(dtype=torch.int32, device=dev)
        out = dict(sorted_tiles=torch.empty(M, **i32), sorted_gauss=torch.empty(M, **i32),
                   tile_offsets=torch.empty(T + 1, **i32), unique_tiles=torch.empty(T, **i32),
                   counts=torch.empty(T, **i32), runs_offsets=torch.empty(T + 1, **i32),
                   num_runs=torch.empty(1, **i32))
        ws = torch.empty(lib.g2v_t2g_workspace(n, M, vs, vr), dtype=torch.uint8, device=dev)
        _lib.check(lib.g2v_build_t2g(n, vs, vr, _ptr(valid_voxel_lb), _ptr(valid_voxel_ub),
                                     _ptr(g2t_offsets), _ptr(g2t_tile_ids), M, _ptr(out["sorted_tiles"]),
                                     _ptr(out["sorted_gauss"]), _ptr(out["tile_offsets"]),
                                     _ptr(out["unique_tiles"]), _ptr(out["counts"]),
                                     _ptr(out["runs_offsets"]), _ptr(out["num_runs"]), _ptr(ws),
                                     ws.numel(), _stream(dev)),
                   "build_t2g")
        U = int(out["num_runs"].item())
    out["num_runs"] = U
    out["unique_tiles"] = out["unique_tiles"][:U]
    out["counts"] = out["counts"][:U]
    out["runs_offsets"] = out["runs_offsets"][:U + 1]
    return out


def _cosine_inputs(voxel_label, occ_gt_mask_camera, grid_feats, pseudo_dino_gt):
    """The reference's input checks (src/cuda_feats_loss.cu:158-161: dtype, contiguity, device; a
    failure is a RuntimeError) plus the shape agreement its 3-D / 4-D accessors assume.  grid_feats
    may also be bfloat16 (as the voxelizer returns it for bfloat16 features); pseudo_dino_gt then
    has to be bfloat16 too."""
    fdtype = grid_feats.dtype if isinstance(grid_feats, torch.Tensor) and grid_feats.dtype in _FEAT_DTYPES \
        else torch.float32
    for t, name, dt in ((voxel_label, "voxel_label", torch.float32),
                        (occ_gt_mask_camera, "occ_gt_mask_camera", torch.bool),
                        (grid_feats, "grid_feats", fdtype),
                        (pseudo_dino_gt, "pseudo_dino_gt", fdtype)):
        if not isinstance(t, torch.Tensor) or t.dtype != dt or not t.is_contiguous() or t.device.type != "cuda":
            raise RuntimeError(f"{name} must be a contiguous {dt} GPU tensor")
    if voxel_label.dim() != 3 or grid_feats.dim() != 4:
        raise RuntimeError("voxel_label must be (X, Y, Z) and grid_feats (X, Y, Z, C)")
    dims = tuple(voxel_label.shape)
    if (tuple(occ_gt_mask_camera.shape) != dims or tuple(grid_feats.shape[:3]) != dims
            or tuple(pseudo_dino_gt.shape) != tuple(grid_feats.shape)):
        raise RuntimeError(f"shape mismatch: voxel_label {dims}, occ_gt_mask_camera "
                           f"{tuple(occ_gt_mask_camera.shape)}, grid_feats {tuple(grid_feats.shape)}, "
                           f"pseudo_dino_gt {tuple(pseudo_dino_gt.shape)}")
    dev = grid_feats.device
    for t, name in ((voxel_label, "voxel_label"), (occ_gt_mask_camera, "occ_gt_mask_camera"),
                    (pseudo_dino_gt, "pseudo_dino_gt")):
        if t.device != dev:
            raise RuntimeError(f"{name} is on {t.device}, grid_feats on {dev}")
    return voxel_label.numel(), grid_feats.shape[3], dev, _FEAT_DTYPES[fdtype]


def CudaFeatsCosinelossForward(voxel_label, occ_gt_mask_camera, grid_feats, pseudo_dino_gt):
    """Voxel-wise cosine loss (reference src/cuda_feats_loss.cu:154-231, bound at src/bindings.cpp:67-83).

    Args: voxel_label (X,Y,Z) float32, occ_gt_mask_camera (X,Y,Z) bool, grid_feats and
    pseudo_dino_gt (X,Y,Z,C) float32 (or both bfloat16), all contiguous on the GPU.
    Returns the reference's 3-tuple: the mean over valid voxels (mask and label > 0) of
    1 - cos(grid_feats, pseudo_dino_gt) as a 0-dim GPU tensor (0 without valid voxels), the number
    of valid voxels (int) and the forward time in seconds.
    """
    loss, cnt, fwd_sec, _ = _cosine_forward(voxel_label, occ_gt_mask_camera, grid_feats, pseudo_dino_gt, False)
    return loss, cnt, fwd_sec


def _cosine_forward(voxel_label, occ_gt_mask_camera, grid_feats, pseudo_dino_gt, want_coef):
    """CudaFeatsCosinelossForward; want_coef also returns the (X*Y*Z, 2) float32 tensor of the
    voxels' unscaled gradient coefficients (g2v_cosine_loss_forward_coef), else None."""
    lib = _lib.load()
    V, C, dev, fdt = _cosine_inputs(voxel_label, occ_gt_mask_camera, grid_feats, pseudo_dino_gt)
    with _OnDevice(dev):
        cur = torch.cuda.current_stream(dev)
        loss = torch.empty((), dtype=torch.float32, device=dev)
        cnt_dev = torch.empty((), dtype=torch.int32, device=dev)
        ws = torch.empty(lib.g2v_cosine_loss_workspace(V, C), dtype=torch.uint8, device=dev)
        coef = torch.empty(V, 2, dtype=torch.float32, device=dev) if want_coef else None
        cnt = ctypes.c_int(0)
        start, stop = _timing_events(dev)
        start.record(cur)
        args = (V, C, _ptr(voxel_label), _ptr(occ_gt_mask_camera), _ptr(grid_feats), _ptr(pseudo_dino_gt), fdt,
                _ptr(loss), _ptr(cnt_dev), ctypes.byref(cnt))
        tail = (_ptr(ws), ws.numel(), ctypes.c_void_p(cur.cuda_stream))
        if want_coef:
            _lib.check(lib.g2v_cosine_loss_forward_coef(*args, _ptr(coef), *tail), "CudaFeatsCosinelossForward")
        else:
            _lib.check(lib.g2v_cosine_loss_forward(*args, *tail), "CudaFeatsCosinelossForward")
        stop.record(cur)
        stop.synchronize()
        fwd_sec = start.elapsed_time(stop) / 1000.0
    return loss, int(cnt.value), fwd_sec, coef


def CudaFeatsCosinelossBackward(grad_output, voxel_label, occ_gt_mask_camera, grid_feats, pseudo_dino_gt,
                                num_valid_voxel):
    """Gradient of the cosine loss with respect to grid_feats (reference src/cuda_feats_loss.cu:311-366,
    bound at src/bindings.cpp:85-104).

    grad_output is the upstream gradient of the scalar loss (one element); it is read on the GPU,
    without the reference's host round trip.  Returns (grad_grid_feats (X,Y,Z,C), backward time in
    seconds); the gradient is zero on invalid voxels and has grid_feats' type (a bfloat16 gradient is
    the float value rounded to nearest even).
    """
    lib = _lib.load()
    V, C, dev, fdt = _cosine_inputs(voxel_label, occ_gt_mask_camera, grid_feats, pseudo_dino_gt)
    if not isinstance(grad_output, torch.Tensor) or grad_output.numel() != 1:
        raise RuntimeError("grad_output must be a one-element tensor")
    with _OnDevice(dev):
        cur = torch.cuda.current_stream(dev)
        gout = grad_output.detach().to(device=dev, dtype=torch.float32).reshape(1).contiguous()
        grad_p = torch.empty_like(grid_feats)
        start, stop = _timing_events(dev)
        start.record(cur)
        _lib.check(lib.g2v_cosine_loss_backward(V, C, _ptr(gout), _ptr(voxel_label), _ptr(occ_gt_mask_camera),
                                                _ptr(grid_feats), _ptr(pseudo_dino_gt), fdt, int(num_valid_voxel),
                                                _ptr(grad_p), ctypes.c_void_p(cur.cuda_stream)),
                   "CudaFeatsCosinelossBackward")
        stop.record(cur)
        stop.synchronize()
        bwd_sec = start.elapsed_time(stop) / 1000.0
    return grad_p, bwd_sec


def _scale_rot_inputs(scales, rotations):
    sc = _f32_input(scales, "scales")
    if sc.dim() < 1 or sc.shape[-1] != 3:
        raise RuntimeError(f"scales must be (N, 3), got {tuple(sc.shape)}")
    n = sc.numel() // 3
    rot = _f32_input(rotations, "rotations")
    if tuple(rot.shape) != tuple(sc.shape[:-1]) + (4,):
        raise RuntimeError(f"rotations must be (N, 4) matching scales {tuple(sc.shape)}, got {tuple(rot.shape)}")
    if rot.device != sc.device:
        raise RuntimeError(f"rotations are on {rot.device}, scales on {sc.device}")
    return sc.reshape(-1, 3), rot.reshape(-1, 4), n


def covariance_from_scale_rotation(scales, rotations):
    """Covariances (N, 9) row-major from scales (N, 3) and rotation quaternions (N, 4, real part
    first, normalised here): (R diag(s)) (R diag(s))^T, as ShelfGaussian builds them before the
    voxelizer (reference test/gaussian_voxelizer.py:14-37)."""
    lib = _lib.load()
    sc, rot, n = _scale_rot_inputs(scales, rotations)
    dev = sc.device
    with _OnDevice(dev):
        cov = torch.empty(n, 9, dtype=torch.float32, device=dev)
        _lib.check(lib.g2v_covariance_from_scale_rotation(n, _ptr(sc), _ptr(rot), _ptr(cov), _stream(dev)),
                   "covariance_from_scale_rotation")
    return cov


def covariance_from_scale_rotation_backward(scales, rotations, grad_cov):
    """(grad_scales (N, 3), grad_rotations (N, 4)) for grad_cov (N, 9) = dL/dcovariances."""
    lib = _lib.load()
    sc, rot, n = _scale_rot_inputs(scales, rotations)
    dev = sc.device
    g = _f32_input(grad_cov, "grad_cov")
    if g.numel() != 9 * n:
        raise RuntimeError(f"grad_cov must have N x 9 = {9 * n} elements, got {g.numel()}")
    if g.device != dev:
        raise RuntimeError(f"grad_cov is on {g.device}, scales on {dev}")
    with _OnDevice(dev):
        gs = torch.empty(n, 3, dtype=torch.float32, device=dev)
        gq = torch.empty(n, 4, dtype=torch.float32, device=dev)
        _lib.check(lib.g2v_covariance_from_scale_rotation_backward(n, _ptr(sc), _ptr(rot), _ptr(g), _ptr(gs),
                                                                   _ptr(gq), _stream(dev)),
                   "covariance_from_scale_rotation_backward")
    return gs, gq
