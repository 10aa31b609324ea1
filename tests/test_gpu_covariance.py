"""GPU parity of the covariance construction from scales and rotations (libg2v_hip.so:
g2v_covariance_from_scale_rotation[_backward]) against the float64 oracle, and of the voxelizer
module fed with scales and rotations (run on the MI355X box with -m gpu).

Bars: covariances and both gradients L2-relative < 1e-5 (float32 kernels vs float64); the
module's scale and rotation gradients equal the covariance backward applied to the voxelizer's
grad_cov (same kernels: identical bits); boxes and CSR bit-exact against the oracle on the
covariances the kernel produced.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import g2v_oracle as O
from tests import workloads as W

pytestmark = pytest.mark.gpu

TOL = 1e-5


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


def _sq(n, seed):
    g = torch.Generator().manual_seed(seed)
    s = torch.rand(n, 3, generator=g) * 1.5 + 0.05
    q = torch.randn(n, 4, generator=g) * (torch.rand(n, 1, generator=g) + 0.5)
    return s, q


@pytest.mark.parametrize("n", [1, 257, 20000])
def test_covariance_parity(n):
    say(f"[cov] n={n}")
    s, q = _sq(n, n)
    dev = torch.device("cuda")
    cov = _C().covariance_from_scale_rotation(s.to(dev), q.to(dev))
    exp = O.covariance_from_scale_rotation_f64(s.numpy(), q.numpy())
    assert O.rel_err(cov.cpu().numpy(), exp) < TOL
    G = torch.randn(n, 9, generator=torch.Generator().manual_seed(1))
    gs, gq = _C().covariance_from_scale_rotation_backward(s.to(dev), q.to(dev), G.to(dev))
    egs, egq = O.covariance_from_scale_rotation_grad_f64(s.numpy(), q.numpy(), G.numpy())
    assert O.rel_err(gs.cpu().numpy(), egs) < TOL
    assert O.rel_err(gq.cpu().numpy(), egq) < TOL


def test_covariance_empty_and_errors():
    dev = torch.device("cuda")
    cov = _C().covariance_from_scale_rotation(torch.zeros(0, 3, device=dev), torch.zeros(0, 4, device=dev))
    assert cov.shape == (0, 9)
    with pytest.raises(RuntimeError):
        _C().covariance_from_scale_rotation(torch.ones(4, 3, device=dev), torch.ones(4, 3, device=dev))
    with pytest.raises(RuntimeError):
        _C().covariance_from_scale_rotation(torch.ones(4, 3, device=dev).double(), torch.ones(4, 4, device=dev))


def test_module_with_scales_and_rotations():
    from CudaGaussianVoxelizer import PyCudaGaussianVoxelizer
    from tests.test_gpu_parity import _check_boxes_and_csr, _oracle_boxes_csr
    dev = torch.device("cuda")
    w = W.Workload("scale_rot", 1500, 24, voxel_range=W.RANGE_SMALL)
    m, o, _, f = W.generate(w, seed=3)
    s, q = _sq(m.shape[0], 5)
    s = s * 0.8
    say("[cov] module with scales and rotations")
    vox = PyCudaGaussianVoxelizer(voxel_size=list(w.voxel_size), voxel_range=list(w.voxel_range))
    sd = s.to(dev).requires_grad_()
    qd = q.to(dev).requires_grad_()
    md, od, fd = m.to(dev), o.to(dev), f.to(dev)
    density, grid_feats, _ = vox(md, od, None, fd, scales=sd, rotations=qd)
    gD = torch.randn(*density.shape, device=dev)
    gF = torch.randn(*grid_feats.shape, device=dev)
    torch.autograd.backward([density, grid_feats], [gD, gF])
    # the same chain by hand: covariances, voxelizer, covariance backward
    cov = _C().covariance_from_scale_rotation(s.to(dev), q.to(dev))
    out = _C().gaussian_voxelizer_forward(md, od, cov, vox.voxel_size, vox.voxel_range, fd)
    assert torch.equal(out[0], density.detach()) and torch.equal(out[5], grid_feats.detach())
    g = _C().gaussian_voxelizer_backward(gD, gF, md, od, out[1], vox.voxel_size, vox.voxel_range, out[2], out[3],
                                         out[4], out[6], out[7], out[0], out[5], fd)
    gs, gq = _C().covariance_from_scale_rotation_backward(s.to(dev), q.to(dev), g[1])
    assert torch.equal(gs, sd.grad) and torch.equal(gq, qd.grad)
    # boxes and CSR of the kernel's covariances are the oracle's, bit for bit
    c32 = cov.cpu()
    b, off, tid, gid, toff, sg, vs, vr = _oracle_boxes_csr(w, m, c32)
    _check_boxes_and_csr(w, out, b, off, tid, gid, toff)
    # and the covariances themselves match the float64 construction
    assert O.rel_err(c32.numpy(), O.covariance_from_scale_rotation_f64(s.numpy(), q.numpy())) < TOL


def test_module_needs_covariances_or_scales_and_rotations():
    from CudaGaussianVoxelizer import PyCudaGaussianVoxelizer
    dev = torch.device("cuda")
    vox = PyCudaGaussianVoxelizer()
    with pytest.raises(RuntimeError):
        vox(torch.zeros(2, 3, device=dev), torch.zeros(2, device=dev), None, scales=torch.ones(2, 3, device=dev))
