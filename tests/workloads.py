"""Synthetic workloads of the G2V splatting path (benchmark configs 1-5 and test cases).

The generator follows the order of test/test_reference.py:30-45 (reference repository):
means, opacity, rotation (QR of randn), variances, covariance R diag(var) R^T flattened
to 9, features -- on the CPU generator, then moved to the device by the caller.
"""
from __future__ import annotations

import os

from dataclasses import dataclass, field
from typing import Optional, Tuple

import torch

RANGE_SMALL = (-10.0, -10.0, -1.0, 10.0, 10.0, 2.2)     # 50 x 50 x 8 voxels
RANGE_PAPER = (-40.0, -40.0, -1.0, 40.0, 40.0, 5.4)     # 200 x 200 x 16 voxels
VOXEL = (0.4, 0.4, 0.4)


@dataclass
class Workload:
    name: str
    n: int
    feat_dim: Optional[int]          # None -> density only
    voxel_range: Tuple[float, ...] = RANGE_PAPER
    voxel_size: Tuple[float, ...] = VOXEL
    var_range: Tuple[float, float] = (0.5, 2.5)
    mean_pad: float = 0.0            # means drawn from the range expanded by this much
    grads: str = "ones"              # "ones" or "randn" upstream gradients
    num_outside: int = 0             # extra Gaussians centred just beyond x_max
    extra: dict = field(default_factory=dict)


CONFIGS = {
    1: Workload("cfg1_50x50x8_n2000_c64", 2000, 64, voxel_range=RANGE_SMALL, grads="ones"),
    2: Workload("cfg2_200x200x16_n9000_c768", 9000, 768, grads="randn"),
    3: Workload("cfg3_200x200x16_n18000_c1024", 18000, 1024, grads="ones"),
    4: Workload("cfg4_200x200x16_n18000_c512_wide", 18000, 512, var_range=(2.0, 12.0),
                mean_pad=4.0, grads="randn"),
    5: Workload("cfg5_200x200x16_n200000_density", 200000, None, var_range=(0.1, 0.6),
                grads="randn"),
}


def generate(w: Workload, seed: int = 0):
    """(means3D (N,3), opacity (N,), covariances (N,9), features (N,C) or None), float32 CPU."""
    g = torch.Generator().manual_seed(seed)
    if w.extra.get("fixture") == "mmdet":   # the recorded batch, with seeded synthetic features
        means, opacity, cov, _, _ = mmdet_fixture()
        feats = None if w.feat_dim is None else torch.randn(means.shape[0], w.feat_dim, generator=g)
        return means, opacity, cov, feats
    box = w.extra.get("mean_box", w.voxel_range)   # means drawn in this box (default: the grid's range)
    lo = torch.tensor(box[:3], dtype=torch.float32) - w.mean_pad
    hi = torch.tensor(box[3:], dtype=torch.float32) + w.mean_pad
    means = torch.rand(w.n, 3, generator=g) * (hi - lo) + lo
    if w.num_outside:
        lo0 = torch.tensor(w.voxel_range[:3], dtype=torch.float32)
        hi0 = torch.tensor(w.voxel_range[3:], dtype=torch.float32)
        out = torch.rand(w.num_outside, 3, generator=g) * (hi0 - lo0) + lo0
        out[:, 0] = hi0[0] + torch.rand(w.num_outside, generator=g) * 1.5
        means = torch.cat([means, out])
    n = means.shape[0]
    opacity = torch.rand(n, generator=g)
    R, _ = torch.linalg.qr(torch.randn(n, 3, 3, generator=g))
    a, b = w.var_range
    var = torch.rand(n, 3, generator=g) * (b - a) + a
    cov = (R @ torch.diag_embed(var) @ R.mT).reshape(n, 9)
    feats = None if w.feat_dim is None else torch.randn(n, w.feat_dim, generator=g)
    return (means.contiguous(), opacity.contiguous(), cov.contiguous(),
            None if feats is None else feats.contiguous())


def grid_shape(w: Workload):
    import numpy as np
    s = np.asarray(w.voxel_size, np.float32)
    r = np.asarray(w.voxel_range, np.float32)
    return tuple(int(np.float32(np.float32(r[a + 3] - r[a]) / s[a])) for a in range(3))


def upstream_grads(w: Workload, seed: int = 1):
    """(grad_density (X,Y,Z), grad_feats (X,Y,Z,C) or None), float32 CPU, materialised."""
    X, Y, Z = grid_shape(w)
    C = w.feat_dim
    if w.grads == "ones":
        gD = torch.ones(X, Y, Z)
        gF = None if C is None else torch.ones(X, Y, Z, C)
    else:
        g = torch.Generator().manual_seed(seed)
        gD = torch.randn(X, Y, Z, generator=g)
        gF = None if C is None else torch.randn(X, Y, Z, C, generator=g)
    return gD, gF


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def mmdet_fixture():
    """The reference's recorded ShelfGaussian batch (tests/golden/mmdet_debug_inputs.npz, written by
    tests/golden/make_mmdet_fixture.py): 1,800 Gaussians, many centred far outside the grid, with
    float16 covariances up to 31 m^2 on the diagonal.  Returns (means (N,3), opacity (N,),
    covariances (N,9)) as float32 CPU tensors, the covariances widened from float16 as the
    reference's test/test_data_from_mmdetection.py does, and the voxel size and range."""
    import numpy as np
    d = np.load(os.path.join(GOLDEN, "mmdet_debug_inputs.npz"))
    m = torch.from_numpy(d["means3D"].astype(np.float32))
    o = torch.from_numpy(d["opacity"].astype(np.float32))
    c = torch.from_numpy(d["covariances_f16"].astype(np.float32))
    return m, o, c, tuple(float(v) for v in d["voxel_size"]), tuple(float(v) for v in d["voxel_range"])


def mmdet_workload(feat_dim=None, grads="randn"):
    """Workload of the recorded batch (see mmdet_fixture) on its own grid."""
    return Workload("mmdet_debug_batch" + ("" if feat_dim is None else f"_c{feat_dim}"), 1800, feat_dim,
                    voxel_range=RANGE_PAPER, voxel_size=VOXEL, grads=grads, extra={"fixture": "mmdet"})
