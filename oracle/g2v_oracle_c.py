"""ctypes front end of the C oracle (oracle/g2v_oracle.c).

TEST INFRASTRUCTURE ONLY: used by tests/ and by bench.py's cpu_baseline leg as the
checker and the CPU baseline, never by the product package.  Build with
``make -C oracle`` (``__graft_entry__.build()`` does it).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libg2v_oracle.so")
_lib = None

_fp = ctypes.POINTER(ctypes.c_float)
_ip = ctypes.POINTER(ctypes.c_int)
_dp = ctypes.POINTER(ctypes.c_double)


def build():
    import subprocess
    subprocess.check_call(["make", "-s", "-C", _HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"C oracle not built ({LIB_PATH}); run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        L.g2vo_g2t.restype = ctypes.c_longlong
        L.g2vo_max_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t) if a is not None else None


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def boxes(means, cov, vs, vr):
    means, cov = _f32(means).reshape(-1, 3), _f32(cov).reshape(-1, 9)
    n = means.shape[0]
    vs, vr = _f32(vs).reshape(3), _f32(vr).reshape(6)
    out = dict(lb=np.zeros((n, 3), np.int32), ub=np.zeros((n, 3), np.int32),
               nvox=np.zeros(n, np.int32), tile_lo=np.zeros((n, 3), np.int32),
               tile_hi=np.zeros((n, 3), np.int32), ntiles=np.zeros(n, np.int32),
               cov_inv=np.zeros((n, 9), np.float32))
    lib().g2vo_boxes(n, _p(means, _fp), _p(cov, _fp), _p(vs, _fp), _p(vr, _fp),
                     _p(out["lb"], _ip), _p(out["ub"], _ip), _p(out["nvox"], _ip),
                     _p(out["tile_lo"], _ip), _p(out["tile_hi"], _ip), _p(out["ntiles"], _ip),
                     _p(out["cov_inv"], _fp))
    return out


def csr(tile_lo, tile_hi, tiles):
    """Both CSRs: (g2t_offsets, g2t_tile_ids, g2t_gauss_ids, tile_offsets, sorted_gauss)."""
    tile_lo = np.ascontiguousarray(tile_lo, np.int32)
    tile_hi = np.ascontiguousarray(tile_hi, np.int32)
    n = tile_lo.shape[0]
    tl = np.asarray(tiles, np.int32)
    off = np.zeros(n + 1, np.int32)
    M = lib().g2vo_g2t(n, _p(tile_lo, _ip), _p(tile_hi, _ip), _p(tl, _ip), _p(off, _ip), None, None)
    tid = np.zeros(M, np.int32)
    gid = np.zeros(M, np.int32)
    lib().g2vo_g2t(n, _p(tile_lo, _ip), _p(tile_hi, _ip), _p(tl, _ip), _p(off, _ip),
                   _p(tid, _ip), _p(gid, _ip))
    T = int(np.prod(tiles))
    toff = np.zeros(T + 1, np.int32)
    sg = np.zeros(M, np.int32)
    lib().g2vo_t2g(ctypes.c_longlong(M), _p(tid, _ip), _p(gid, _ip), T, _p(toff, _ip), _p(sg, _ip))
    return off, tid, gid, toff, sg


def forward(means, opacity, cov_inv64, lb, ub, vs, vr, tile_offsets, sorted_gauss, features,
            dims, tile_range=None, nthreads=0):
    means, opacity = _f32(means), _f32(opacity)
    cov_inv64 = np.ascontiguousarray(cov_inv64, np.float64)
    lb, ub = np.ascontiguousarray(lb, np.int32), np.ascontiguousarray(ub, np.int32)
    vs, vr = _f32(vs).reshape(3), _f32(vr).reshape(6)
    n = means.shape[0]
    C = 0 if features is None else features.shape[1]
    feats = None if features is None else _f32(features)
    X, Y, Z = dims
    density = np.zeros(X * Y * Z, np.float64)
    grid = np.zeros(X * Y * Z * C, np.float64) if C else None
    T = len(tile_offsets) - 1
    t0, t1 = (0, T) if tile_range is None else tile_range
    lib().g2vo_forward(n, C, _p(means, _fp), _p(opacity, _fp), _p(cov_inv64, _dp), _p(lb, _ip),
                       _p(ub, _ip), _p(vs, _fp), _p(vr, _fp),
                       _p(np.ascontiguousarray(tile_offsets, np.int32), _ip),
                       _p(np.ascontiguousarray(sorted_gauss, np.int32), _ip), _p(feats, _fp),
                       _p(density, _dp), _p(grid, _dp), t0, t1, nthreads)
    return density.reshape(X, Y, Z), (grid.reshape(X, Y, Z, C) if C else None)


def backward(means, opacity, cov_inv64, lb, ub, vs, vr, g2t_offsets, g2t_tile_ids, features,
             density, grid_feats, grad_density, grad_feats, g_range=None, nthreads=0):
    means, opacity = _f32(means), _f32(opacity)
    cov_inv64 = np.ascontiguousarray(cov_inv64, np.float64)
    lb, ub = np.ascontiguousarray(lb, np.int32), np.ascontiguousarray(ub, np.int32)
    vs, vr = _f32(vs).reshape(3), _f32(vr).reshape(6)
    n = means.shape[0]
    C = 0 if features is None else features.shape[1]
    gm = np.zeros((n, 3)); gc = np.zeros((n, 9)); go = np.zeros(n)
    gf = np.zeros((n, C)) if C else None
    g0, g1 = (0, n) if g_range is None else g_range
    lib().g2vo_backward(n, C, _p(means, _fp), _p(opacity, _fp), _p(cov_inv64, _dp), _p(lb, _ip),
                        _p(ub, _ip), _p(vs, _fp), _p(vr, _fp),
                        _p(np.ascontiguousarray(g2t_offsets, np.int32), _ip),
                        _p(np.ascontiguousarray(g2t_tile_ids, np.int32), _ip),
                        _p(None if features is None else _f32(features), _fp),
                        _p(_f32(density), _fp), _p(None if grid_feats is None else _f32(grid_feats), _fp),
                        _p(_f32(grad_density), _fp),
                        _p(None if grad_feats is None else _f32(grad_feats), _fp),
                        _p(gm, _dp), _p(gc, _dp), _p(go, _dp), _p(gf, _dp), g0, g1, nthreads)
    return gm, gc, go, gf


def max_threads():
    return int(lib().g2vo_max_threads())
