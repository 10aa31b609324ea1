"""GPU tests of the batched (multi-scene) API: B scenes on one grid in one call, one host wait for
the whole batch's plan (run on the MI355X box with -m gpu).

Bars: every scene's outputs equal the single-scene call's bit for bit (same kernels on the same
inputs), for the forward 9-tuple and for the module's gradients; one scene checked against the
oracle as well.  Covers scenes of different sizes (padding with Gaussians outside the grid), an
empty scene, density-only and feature batches, and the reference's recorded batch split into its
six groups of 300 Gaussians (tests/golden/mmdet_debug_inputs.npz).
"""
import sys

import numpy as np
import pytest
import torch

from oracle import g2v_oracle as O
from tests import workloads as W

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _setup():
    import CudaGaussianVoxelizer._lib as L
    L.load()


def _C():
    from CudaGaussianVoxelizer import _C
    return _C


def _batch(B, n, C, seed, vr=W.RANGE_SMALL):
    ms, os_, cs, fs = [], [], [], []
    for b in range(B):
        w = W.Workload(f"b{b}", n, C, voxel_range=vr, var_range=(0.2, 2.0))
        m, o, c, f = W.generate(w, seed=seed + b)
        if b == 1:   # a scene with fewer Gaussians: the rest sit far outside the grid
            m[n // 2:] = 1000.0
        if b == 2 and B > 3:   # an empty scene
            m[:] = -1000.0
        ms.append(m)
        os_.append(o)
        cs.append(c)
        if f is not None:
            fs.append(f)
    return (torch.stack(ms), torch.stack(os_), torch.stack(cs), torch.stack(fs) if fs else None)


@pytest.mark.parametrize("C", [None, 24])
def test_batched_forward_equals_single_scene_calls(C):
    dev = torch.device("cuda")
    m, o, c, f = _batch(4, 700, C, seed=20)
    vs = torch.tensor(W.VOXEL, device=dev)
    vr = torch.tensor(W.RANGE_SMALL, device=dev)
    say(f"[batched] forward B=4 C={C}")
    outs = _C().gaussian_voxelizer_forward_batched(m.to(dev), o.to(dev), c.to(dev), vs, vr,
                                                   None if f is None else f.to(dev))
    assert len(outs) == 4
    for b in range(4):
        ref = _C().gaussian_voxelizer_forward(m[b].to(dev), o[b].to(dev), c[b].to(dev), vs, vr,
                                              None if f is None else f[b].to(dev))
        for k in range(8):
            assert torch.equal(outs[b][k], ref[k]), (b, k)
    assert outs[2][7].numel() == 0 and not outs[2][0].any()   # the empty scene
    # one scene against the oracle
    b = 1
    ob = O.gaussian_boxes(m[b].numpy(), c[b].numpy(), np.array(W.VOXEL, np.float32),
                          np.array(W.RANGE_SMALL, np.float32))
    D, F = O.forward_f64(m[b].numpy(), o[b].numpy(), c[b].numpy(), None if f is None else f[b].numpy(),
                         ob["lb"], ob["ub"], np.array(W.VOXEL, np.float32), np.array(W.RANGE_SMALL, np.float32))
    assert O.rel_err(outs[b][0].cpu().numpy(), D) < 1e-4


# B = 6 puts two scenes on each of the first two of the four side streams; the batch runs twice in
# a row (the second call reuses the streams and the memory of the first)
@pytest.mark.parametrize("B,C", [(3, None), (3, 16), (6, 16)])
def test_batched_module_gradients_equal_single_scene_module(B, C):
    from CudaGaussianVoxelizer import PyCudaGaussianVoxelizer
    dev = torch.device("cuda")
    m, o, c, f = _batch(B, 500, C, seed=40)
    vox = PyCudaGaussianVoxelizer(voxel_size=list(W.VOXEL), voxel_range=list(W.RANGE_SMALL))
    say(f"[batched] module B={B} C={C}")
    g = torch.Generator().manual_seed(3)
    gD = gF = None
    for rep in range(2):
        leaves = [t.to(dev).requires_grad_() for t in (m, o, c)] + ([] if f is None else [f.to(dev).requires_grad_()])
        density, grid_feats, stats = vox(leaves[0], leaves[1], leaves[2], None if f is None else leaves[3])
        assert density.shape[0] == B and grid_feats.shape[0] == B and stats[0] > 0
        if gD is None:
            gD = torch.randn(*density.shape, generator=g).to(dev)
            gF = torch.randn(*grid_feats.shape, generator=g).to(dev)
        torch.autograd.backward([density] if f is None else [density, grid_feats], [gD] if f is None else [gD, gF])
        assert stats[1] > 0
        if rep == 0:
            first = [t.grad.clone() for t in leaves]
    for a, t in zip(first, leaves):
        assert torch.equal(a, t.grad)
    for b in range(B):
        lb_ = [t[b].detach().clone().requires_grad_() for t in (leaves[0], leaves[1], leaves[2])]
        fb = None if f is None else leaves[3][b].detach().clone().requires_grad_()
        d1, f1, _ = vox(lb_[0], lb_[1], lb_[2], fb)
        assert torch.equal(d1, density[b].detach()) and torch.equal(f1, grid_feats[b].detach())
        torch.autograd.backward([d1] if f is None else [d1, f1], [gD[b]] if f is None else [gD[b], gF[b]])
        assert torch.equal(lb_[0].grad, leaves[0].grad[b])
        assert torch.equal(lb_[1].grad, leaves[1].grad[b])
        assert torch.equal(lb_[2].grad, leaves[2].grad[b])
        if f is not None:
            assert torch.equal(fb.grad, leaves[3].grad[b])


def test_batched_recorded_batch():
    """The recorded batch (1, 6, 300) as 6 scenes of 300 Gaussians."""
    from CudaGaussianVoxelizer import PyCudaGaussianVoxelizer
    dev = torch.device("cuda")
    m, o, c, vs, vr = W.mmdet_fixture()
    m, o, c = m.reshape(6, 300, 3), o.reshape(6, 300), c.reshape(6, 300, 9)
    vox = PyCudaGaussianVoxelizer(voxel_size=list(vs), voxel_range=list(vr))
    say("[batched] recorded batch 6 x 300")
    density, _, stats = vox(m.to(dev), o.to(dev), c.to(dev))
    for b in range(6):
        ref = _C().gaussian_voxelizer_forward(m[b].to(dev), o[b].to(dev), c[b].to(dev), vox.voxel_size,
                                              vox.voxel_range)
        assert torch.equal(ref[0], density[b])


def test_batched_input_errors():
    dev = torch.device("cuda")
    vs = torch.tensor(W.VOXEL, device=dev)
    vr = torch.tensor(W.RANGE_SMALL, device=dev)
    with pytest.raises(RuntimeError):
        _C().gaussian_voxelizer_forward_batched(torch.zeros(2, 5, 2, device=dev), torch.zeros(2, 5, device=dev),
                                                torch.zeros(2, 5, 9, device=dev), vs, vr)
    with pytest.raises(RuntimeError):
        _C().gaussian_voxelizer_forward_batched(torch.zeros(2, 5, 3, device=dev), torch.zeros(2, 5, device=dev),
                                                torch.zeros(2, 5, 9, device=dev), vs, vr, torch.zeros(3, 5, 4, device=dev))
