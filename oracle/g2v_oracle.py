"""CPU oracle for the Gaussian-to-Voxel (G2V) splatting path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this module;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker.

It restates, in numpy, what the reference computes (file:line references are
relative to the reference repository root):

* ``grid_dims``      -- voxel/tile grid sizes   src/cuda_gaussian_voxelizer.cu:1511-1519
* ``gaussian_boxes`` -- 3-sigma voxel box, tile box, inverse covariance
                        src/cuda_gaussian_voxelizer.cu:348-536, :201-220
* ``g2t_csr``        -- Gaussian->Tile CSR      src/cuda_gaussian_voxelizer.cu:1605-1615, :228-286
* ``t2g_csr``        -- Tile->Gaussian CSR (stable sort by tile, run-length encode, offsets)
                        src/cuda_gaussian_voxelizer.cu:1673-1772
* ``forward_f64``    -- density + density-weighted feature average, float64
                        src/cuda_gaussian_voxelizer.cu:7-136, :767-966, :1848-1849;
                        test/test_reference.py:57-79
* ``backward_f64``   -- closed-form gradients, float64
                        src/cuda_gaussian_voxelizer.cu:1226-1297, :1304-1362, :1376-1482, :1995-1996
* ``covariance_from_scale_rotation_f64`` / ``..._grad_f64`` -- covariances R diag(s) (R diag(s))^T
                        from scales and rotation quaternions, and the chain rule back to them
                        test/gaussian_voxelizer.py:14-37
* ``cosine_loss_f64`` / ``cosine_loss_grad_f64`` -- the voxel-wise feature cosine loss (mean over
                        valid voxels) and its gradient with respect to grid_feats, float64
                        src/cuda_feats_loss.cu:45-231 (forward), :233-366 (backward)

The box and CSR functions are exact float32/int32 restatements: the HIP kernels
must match them bit for bit.  The splat and gradient functions are float64
brute force; the HIP kernels match them within the tolerances of the parity
tests.  How each function is pinned (closed forms, invariants, autograd,
gradcheck, the README's toy CSR) is listed in the parity tests under tests/.
"""
from __future__ import annotations

import numpy as np

TILE = 4                 # 4x4x4 voxel tiles (include/utils.cuh:50-52)
EPS = np.float32(1e-6)   # density clamp (include/utils.cuh:80)
DET_EPS = np.float32(1e-6)  # determinant clamp (src/cuda_gaussian_voxelizer.cu:200,206)


def _f32(x):
    return np.asarray(x, dtype=np.float32)


def grid_dims(voxel_size, voxel_range):
    """Voxel grid (X, Y, Z) and tile grid (Tx, Ty, Tz).

    Follows src/cuda_gaussian_voxelizer.cu:1512-1519: float32 ``(r_hi - r_lo) / s``
    truncated toward zero, tiles ``ceil(dim / 4)``.
    """
    s = _f32(voxel_size).reshape(3)
    r = _f32(voxel_range).reshape(6)
    dims = []
    for a in range(3):
        q = np.float32(np.float32(r[a + 3] - r[a]) / s[a])
        dims.append(int(np.trunc(q)))
    tiles = [(d + TILE - 1) // TILE for d in dims]
    return tuple(dims), tuple(tiles)


def _cvt_i32(x):
    """float32 -> int32 the way the GPU converts (saturating, NaN -> 0)."""
    x = np.asarray(x, dtype=np.float64)
    out = np.where(np.isnan(x), 0.0, x)
    out = np.clip(out, -2147483648.0, 2147483647.0)
    return out.astype(np.int64).astype(np.int32)


def invert_3x3(cov):
    """Adjugate inverse of each row-major 3x3 in float32 (src/cuda_gaussian_voxelizer.cu:201-220).

    ``|det| < 1e-6`` is replaced by ``+1e-6`` (this flips the sign of small negative
    determinants, as the reference does).  Every product and sum is rounded to
    float32 separately, in the order the reference writes them.
    """
    A = _f32(cov).reshape(-1, 9)
    a = [A[:, i] for i in range(9)]
    with np.errstate(all="ignore"):
        det = (a[0] * (a[4] * a[8] - a[5] * a[7])
               - a[1] * (a[3] * a[8] - a[5] * a[6])) + a[2] * (a[3] * a[7] - a[4] * a[6])
        det = np.where(np.abs(det) < DET_EPS, DET_EPS, det).astype(np.float32)
        inv_det = (np.float32(1.0) / det).astype(np.float32)
        out = np.empty_like(A)
        out[:, 0] = (a[4] * a[8] - a[5] * a[7]) * inv_det
        out[:, 1] = -(a[1] * a[8] - a[2] * a[7]) * inv_det
        out[:, 2] = (a[1] * a[5] - a[2] * a[4]) * inv_det
        out[:, 3] = -(a[3] * a[8] - a[5] * a[6]) * inv_det
        out[:, 4] = (a[0] * a[8] - a[2] * a[6]) * inv_det
        out[:, 5] = -(a[0] * a[5] - a[2] * a[3]) * inv_det
        out[:, 6] = (a[3] * a[7] - a[4] * a[6]) * inv_det
        out[:, 7] = -(a[0] * a[7] - a[1] * a[6]) * inv_det
        out[:, 8] = (a[0] * a[4] - a[1] * a[3]) * inv_det
    return out


def gaussian_boxes(means, cov, voxel_size, voxel_range):
    """Per-Gaussian voxel box, tile box and inverse covariance (exact float32).

    Follows src/cuda_gaussian_voxelizer.cu:348-536:
      sigma = sqrtf(diag);  lower/upper = mu -/+ 3*sigma (no fused multiply-add);
      clamp to the range with fmaxf/fminf (a NaN bound becomes the range face);
      idx = (int)floorf((v - r_lo) / s), clamped to [0, dim-1];
      empty if any lo > hi  ->  lb = 0, ub = -1, nvox = 0, tiles (0, -1), ntiles 0, cov_inv 0.
    Returns a dict of int32 / float32 arrays.
    """
    mu = _f32(means).reshape(-1, 3)
    C = _f32(cov).reshape(-1, 9)
    n = mu.shape[0]
    s = _f32(voxel_size).reshape(3)
    r = _f32(voxel_range).reshape(6)
    dims, tiles = grid_dims(s, r)
    with np.errstate(all="ignore"):
        sig = np.sqrt(C[:, [0, 4, 8]]).astype(np.float32)
        three_sig = (np.float32(3.0) * sig).astype(np.float32)
        lower = (mu - three_sig).astype(np.float32)
        upper = (mu + three_sig).astype(np.float32)
        lower = np.fmax(lower, r[:3][None, :]).astype(np.float32)
        upper = np.fmin(upper, r[3:][None, :]).astype(np.float32)
        lo = _cvt_i32(np.floor(((lower - r[:3][None, :]).astype(np.float32) / s[None, :]).astype(np.float32)))
        hi = _cvt_i32(np.floor(((upper - r[:3][None, :]).astype(np.float32) / s[None, :]).astype(np.float32)))
    lo = np.maximum(lo, 0)
    hi = np.minimum(hi, np.asarray(dims, dtype=np.int32)[None, :] - 1)
    empty = (lo > hi).any(axis=1)

    lb = np.where(empty[:, None], 0, lo).astype(np.int32)
    ub = np.where(empty[:, None], -1, hi).astype(np.int32)
    ext = (ub - lb + 1).astype(np.int64)
    nvox = np.where(empty, 0, ext.prod(axis=1)).astype(np.int32)

    tl = np.maximum(lb // TILE, 0)
    th = np.minimum(ub // TILE, np.asarray(tiles, dtype=np.int32)[None, :] - 1)
    tile_lo = np.where(empty[:, None], 0, tl).astype(np.int32)
    tile_hi = np.where(empty[:, None], -1, th).astype(np.int32)
    text = (tile_hi - tile_lo + 1).astype(np.int64)
    ntiles = np.where(empty, 0, text.prod(axis=1)).astype(np.int32)

    cov_inv = invert_3x3(C) if n else np.zeros((0, 9), np.float32)
    cov_inv[empty] = 0.0
    return dict(lb=lb, ub=ub, nvox=nvox, tile_lo=tile_lo, tile_hi=tile_hi,
                ntiles=ntiles, cov_inv=cov_inv.astype(np.float32), dims=dims, tiles=tiles)


def g2t_csr(tile_lo, tile_hi, tiles):
    """Gaussian->Tile CSR (src/cuda_gaussian_voxelizer.cu:1605-1615, :228-286).

    ``offsets[0] = 0``, ``offsets[g+1] = offsets[g] + ntiles[g]``; the tiles of a Gaussian
    are its tile box enumerated row-major (x slowest, z fastest), tile id
    ``(tx * Ty + ty) * Tz + tz``, so each row is ascending.
    """
    tile_lo = np.asarray(tile_lo, np.int64).reshape(-1, 3)
    tile_hi = np.asarray(tile_hi, np.int64).reshape(-1, 3)
    _, Ty, Tz = tiles
    ext = np.maximum(tile_hi - tile_lo + 1, 0)
    counts = ext.prod(axis=1)
    counts[(tile_hi < tile_lo).any(axis=1)] = 0
    offsets = np.zeros(len(counts) + 1, np.int64)
    np.cumsum(counts, out=offsets[1:])
    M = int(offsets[-1])
    tile_ids = np.empty(M, np.int32)
    gauss_ids = np.empty(M, np.int32)
    for g in np.nonzero(counts)[0]:
        x0, y0, z0 = tile_lo[g]
        x1, y1, z1 = tile_hi[g]
        tx, ty, tz = np.meshgrid(np.arange(x0, x1 + 1), np.arange(y0, y1 + 1),
                                 np.arange(z0, z1 + 1), indexing="ij")
        ids = ((tx * Ty + ty) * Tz + tz).reshape(-1)
        tile_ids[offsets[g]:offsets[g + 1]] = ids
        gauss_ids[offsets[g]:offsets[g + 1]] = g
    return offsets.astype(np.int32), tile_ids, gauss_ids


def t2g_csr(g2t_tile_ids, g2t_gauss_ids, num_tiles):
    """Tile->Gaussian CSR (src/cuda_gaussian_voxelizer.cu:1673-1772).

    A stable sort of the (tile, Gaussian) pairs by tile id (the input is in Gaussian
    order, so each tile's list comes out with ascending Gaussian ids), then a
    run-length encode of the sorted tile ids and an inclusive scan of the run
    lengths.  ``tile_offsets`` additionally gives the list bounds of every tile,
    empty ones included (``tile_offsets[t]..tile_offsets[t+1]``).
    """
    keys = np.asarray(g2t_tile_ids, np.int64)
    vals = np.asarray(g2t_gauss_ids, np.int32)
    order = np.argsort(keys, kind="stable")
    sorted_tiles = keys[order].astype(np.int32)
    sorted_gauss = vals[order]
    if len(keys):
        head = np.ones(len(keys), bool)
        head[1:] = sorted_tiles[1:] != sorted_tiles[:-1]
        starts = np.nonzero(head)[0]
        unique = sorted_tiles[starts]
        counts = np.diff(np.append(starts, len(keys))).astype(np.int32)
    else:
        unique = np.zeros(0, np.int32)
        counts = np.zeros(0, np.int32)
    runs_offsets = np.zeros(len(unique) + 1, np.int32)
    np.cumsum(counts, out=runs_offsets[1:])
    per_tile = np.bincount(keys, minlength=num_tiles).astype(np.int64) if len(keys) else np.zeros(num_tiles, np.int64)
    tile_offsets = np.zeros(num_tiles + 1, np.int32)
    np.cumsum(per_tile, out=tile_offsets[1:])
    return dict(sorted_tiles=sorted_tiles, sorted_gauss=sorted_gauss.astype(np.int32),
                unique_tiles=unique.astype(np.int32), counts=counts, num_runs=len(unique),
                runs_offsets=runs_offsets, tile_offsets=tile_offsets)


def _box_voxels(lb, ub):
    ext = ub - lb + 1
    if (ext <= 0).any():
        return np.zeros((0, 3), np.int64)
    g = np.meshgrid(*[np.arange(lb[a], ub[a] + 1) for a in range(3)], indexing="ij")
    return np.stack([x.reshape(-1) for x in g], axis=1).astype(np.int64)


def _centres(idx, voxel_size, voxel_range):
    s = np.asarray(voxel_size, np.float64).reshape(3)
    r = np.asarray(voxel_range, np.float64).reshape(6)
    return r[:3][None, :] + (idx + 0.5) * s[None, :]


def _cov_inv_f64(cov, cov_inv_f32=None):
    if cov_inv_f32 is not None:
        return np.asarray(cov_inv_f32, np.float64).reshape(-1, 3, 3)
    return np.linalg.inv(np.asarray(cov, np.float64).reshape(-1, 3, 3))


def forward_f64(means, opacity, cov, features, lb, ub, voxel_size, voxel_range,
                cov_inv=None, feature_gate=True):
    """Float64 brute force of the forward splat.

    Every Gaussian is evaluated at the centre ``r_lo + (idx + 0.5) * s`` of every voxel
    of its inclusive box [lb, ub]: ``w = o * exp(-0.5 * dx^T A dx)`` with ``dx = centre - mu``.
    ``D_v = sum_g w``; ``F_v = sum_g w f_g / max(D_v, 1e-6)``
    (test/test_reference.py:57-79; src/cuda_gaussian_voxelizer.cu:911-926, :1848-1849).
    With ``feature_gate`` only pairs with ``w > 0`` enter the feature sum
    (src/cuda_gaussian_voxelizer.cu:936), which changes nothing for non-negative opacity.
    ``cov_inv`` (float32, (N,9)) replaces the exact float64 inverse when given.
    Returns (density (X,Y,Z), grid_feats (X,Y,Z,C) or None).
    """
    mu = np.asarray(means, np.float64).reshape(-1, 3)
    o = np.asarray(opacity, np.float64).reshape(-1)
    n = mu.shape[0]
    dims, _ = grid_dims(voxel_size, voxel_range)
    X, Y, Z = dims
    Ainv = _cov_inv_f64(cov, cov_inv)
    f = None if features is None else np.asarray(features, np.float64).reshape(n, -1)
    density = np.zeros(X * Y * Z)
    fsum = None if f is None else np.zeros((X * Y * Z, f.shape[1]))
    lb = np.asarray(lb, np.int64).reshape(-1, 3)
    ub = np.asarray(ub, np.int64).reshape(-1, 3)
    for g in range(n):
        idx = _box_voxels(lb[g], ub[g])
        if len(idx) == 0:
            continue
        d = _centres(idx, voxel_size, voxel_range) - mu[g]
        m = np.einsum("ki,ij,kj->k", d, Ainv[g], d)
        w = o[g] * np.exp(-0.5 * m)
        lin = (idx[:, 0] * Y + idx[:, 1]) * Z + idx[:, 2]
        density[lin] += w
        if f is not None:
            wf = np.where(w > 0, w, 0.0) if feature_gate else w
            fsum[lin] += wf[:, None] * f[g][None, :]
    density = density.reshape(X, Y, Z)
    if f is None:
        return density, None
    grid = fsum / np.maximum(density.reshape(-1), float(EPS))[:, None]
    return density, grid.reshape(X, Y, Z, f.shape[1])


def backward_f64(grad_density, grad_feats, means, opacity, cov, features, lb, ub,
                 voxel_size, voxel_range, density=None, grid_feats=None, cov_inv=None):
    """Float64 closed-form gradients of the forward splat.

    Per (Gaussian g, voxel v in its box), with w = o e, e = exp(-0.5 dx^T A dx), q = A dx,
    inv = 1 / max(D_v, eps), act = D_v >= eps:
        t_v  = act ? sum_c gF_vc F_vc : 0                       (src/cuda_gaussian_voxelizer.cu:1995-1996, :1450)
        u_gv = sum_c gF_vc f_gc
        gw   = gD_v + (u_gv - t_v) inv        (gw = gD_v without features, :1353)
        d mu    += gw w q                      (:1254-1274)
        d Sigma += 0.5 gw w q q^T   (written symmetric, :1277-1297)
        d o     += gw e
        d f_g   += gF_v w inv                  (:1454-1459)
    These equal autograd of ``forward_f64`` through an exact inverse for symmetric Sigma.
    Returns (grad_means (N,3), grad_cov (N,9), grad_opacity (N,), grad_features (N,C) or None).
    """
    mu = np.asarray(means, np.float64).reshape(-1, 3)
    o = np.asarray(opacity, np.float64).reshape(-1)
    n = mu.shape[0]
    dims, _ = grid_dims(voxel_size, voxel_range)
    X, Y, Z = dims
    Ainv = _cov_inv_f64(cov, cov_inv)
    lb = np.asarray(lb, np.int64).reshape(-1, 3)
    ub = np.asarray(ub, np.int64).reshape(-1, 3)
    gD = np.asarray(grad_density, np.float64).reshape(-1)
    has_f = features is not None
    if density is None or (has_f and grid_feats is None):
        density, grid_feats = forward_f64(means, opacity, cov, features, lb, ub, voxel_size,
                                          voxel_range, cov_inv=cov_inv)
    D = np.asarray(density, np.float64).reshape(-1)
    inv = 1.0 / np.maximum(D, float(EPS))
    act = D >= float(EPS)
    g_mu = np.zeros((n, 3))
    g_cov = np.zeros((n, 3, 3))
    g_o = np.zeros(n)
    if has_f:
        f = np.asarray(features, np.float64).reshape(n, -1)
        gF = np.asarray(grad_feats, np.float64).reshape(X * Y * Z, -1)
        Fv = np.asarray(grid_feats, np.float64).reshape(X * Y * Z, -1)
        t = np.where(act, np.einsum("vc,vc->v", gF, Fv), 0.0)
        g_f = np.zeros_like(f)
    for g in range(n):
        idx = _box_voxels(lb[g], ub[g])
        if len(idx) == 0:
            continue
        d = _centres(idx, voxel_size, voxel_range) - mu[g]
        q = d @ Ainv[g].T
        e = np.exp(-0.5 * np.einsum("ki,ki->k", d, q))
        w = o[g] * e
        lin = (idx[:, 0] * Y + idx[:, 1]) * Z + idx[:, 2]
        gw = gD[lin].copy()
        if has_f:
            u = gF[lin] @ f[g]
            gw += (u - t[lin]) * inv[lin]
            g_f[g] = (w * inv[lin]) @ gF[lin]
        gwd = gw * w
        g_mu[g] = gwd @ q
        g_cov[g] = 0.5 * np.einsum("k,ki,kj->ij", gwd, q, q)
        g_o[g] = gw @ e
    return (g_mu, g_cov.reshape(n, 9), g_o, g_f if has_f else None)


def _rotmat_f64(q):
    """Rotation matrices of the normalised quaternions q (N,4), real part first
    (test/gaussian_voxelizer.py:14-28)."""
    q = np.asarray(q, dtype=np.float64)
    q = q / np.sqrt((q * q).sum(-1, keepdims=True))
    r, x, y, z = q[:, 0], q[:, 1], q[:, 2], q[:, 3]
    R = np.empty((q.shape[0], 3, 3))
    R[:, 0, 0] = 1 - 2 * (y * y + z * z)
    R[:, 0, 1] = 2 * (x * y - r * z)
    R[:, 0, 2] = 2 * (x * z + r * y)
    R[:, 1, 0] = 2 * (x * y + r * z)
    R[:, 1, 1] = 1 - 2 * (x * x + z * z)
    R[:, 1, 2] = 2 * (y * z - r * x)
    R[:, 2, 0] = 2 * (x * z - r * y)
    R[:, 2, 1] = 2 * (y * z + r * x)
    R[:, 2, 2] = 1 - 2 * (x * x + y * y)
    return R, q


def covariance_from_scale_rotation_f64(scales, rotations):
    """(N,9) covariances (R diag(s)) (R diag(s))^T, float64 (test/gaussian_voxelizer.py:30-37)."""
    R, _ = _rotmat_f64(rotations)
    M = R * np.asarray(scales, dtype=np.float64)[:, None, :]
    return (M @ M.transpose(0, 2, 1)).reshape(-1, 9)


def covariance_from_scale_rotation_grad_f64(scales, rotations, grad_cov):
    """(grad_scales (N,3), grad_rotations (N,4)) for grad_cov (N,9) = dL/dSigma, float64: the
    chain rule through Sigma = M M^T, M = R diag(s), R(q / |q|)."""
    s = np.asarray(scales, dtype=np.float64)
    q0 = np.asarray(rotations, dtype=np.float64)
    R, q = _rotmat_f64(q0)
    G = np.asarray(grad_cov, dtype=np.float64).reshape(-1, 3, 3)
    M = R * s[:, None, :]
    dM = (G + G.transpose(0, 2, 1)) @ M
    ds = (dM * R).sum(1)
    dR = dM * s[:, None, :]
    r, x, y, z = q[:, 0], q[:, 1], q[:, 2], q[:, 3]
    zero = np.zeros_like(r)
    # dR/dq^ for each quaternion component, as (N,3,3) matrices
    J = {
        0: [[zero, -2 * z, 2 * y], [2 * z, zero, -2 * x], [-2 * y, 2 * x, zero]],
        1: [[zero, 2 * y, 2 * z], [2 * y, -4 * x, -2 * r], [2 * z, 2 * r, -4 * x]],
        2: [[-4 * y, 2 * x, 2 * r], [2 * x, zero, 2 * z], [-2 * r, 2 * z, -4 * y]],
        3: [[-4 * z, -2 * r, 2 * x], [2 * r, -4 * z, 2 * y], [2 * x, 2 * y, zero]],
    }
    dqh = np.stack([(np.moveaxis(np.array(J[k]), 2, 0) * dR).sum((1, 2)) for k in range(4)], axis=1)
    norm = np.sqrt((q0 * q0).sum(-1, keepdims=True))
    dq = (dqh - q * (q * dqh).sum(-1, keepdims=True)) / norm
    return ds, dq


def cosine_valid(voxel_label, occ_mask):
    """Voxels that count: visible and labelled (src/cuda_feats_loss.cu:67-68, :255)."""
    return np.asarray(occ_mask, dtype=bool) & (np.asarray(voxel_label, dtype=np.float32) > 0)


def _cosine_terms(p, g):
    p = np.asarray(p, dtype=np.float64)
    g = np.asarray(g, dtype=np.float64)
    return p, g, (p * g).sum(-1), (p * p).sum(-1), (g * g).sum(-1)


def cosine_loss_f64(voxel_label, occ_mask, grid_feats, pseudo_gt):
    """(mean loss, valid count) of src/cuda_feats_loss.cu:45-231.

    Per valid voxel 1 - p.g / (sqrt(max(|p|^2, eps)) sqrt(max(|g|^2, eps)) + eps) (:94-99); the
    loss is the sum over valid voxels divided by their number, 0 when there is none (:205-212).
    """
    valid = cosine_valid(voxel_label, occ_mask)
    _, _, dot, pp, gg = _cosine_terms(grid_feats, pseudo_gt)
    eps = float(EPS)
    lv = 1.0 - dot / (np.sqrt(np.maximum(pp, eps)) * np.sqrt(np.maximum(gg, eps)) + eps)
    cnt = int(valid.sum())
    return (float(lv[valid].sum()) / cnt if cnt > 0 else 0.0), cnt


def cosine_loss_grad_f64(grad_out, voxel_label, occ_mask, grid_feats, pseudo_gt, num_valid_voxel):
    """d loss / d grid_feats of src/cuda_feats_loss.cu:233-366, float64.

    grad_out / count * (c1 g + c2 p) with c1 = -1/D, D = a b + eps, c2 = p.g b / (a D^2) when
    |p|^2 > eps (else 0), a, b the clamped norms (:278-291); zero on invalid voxels (:255-261);
    1/count is 0 when count is 0 (:319).
    """
    valid = cosine_valid(voxel_label, occ_mask)
    p, g, dot, pp, gg = _cosine_terms(grid_feats, pseudo_gt)
    eps = float(EPS)
    a = np.sqrt(np.maximum(pp, eps))
    b = np.sqrt(np.maximum(gg, eps))
    D = a * b + eps
    c1 = -1.0 / D
    c2 = np.where(pp > eps, dot * b / (a * D * D), 0.0)
    inv = 1.0 / num_valid_voxel if num_valid_voxel > 0 else 0.0
    scale = float(grad_out) * inv
    grad = scale * (c1[..., None] * g + c2[..., None] * p)
    grad[~valid] = 0.0
    return grad


def rel_err(a, b):
    """L2-relative error ||a - b|| / ||b|| (test/test_reference.py:82-83)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
