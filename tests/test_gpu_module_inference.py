"""GPU tests of the module's handling of what the backward reuses (run with -m gpu).

* A forward after which no backward can come (torch.no_grad(), or no input requiring grad)
  keeps no Tile->Gaussian CSR and queues none of the backward's gradient-independent kernels
  (feature split, (region, Gaussian) CSR, row table): the library's per-kernel launch record shows
  none of them, and the outputs equal those of a forward with grad enabled, bit for bit.
* The batched module with non-contiguous features (a temporary contiguous copy is what the
  scenes' side streams read) and caller-stream allocations between forward and backward gives the
  per-scene module's outputs and gradients, bit for bit.
"""
import sys

import pytest
import torch

from tests import workloads as W

pytestmark = pytest.mark.gpu

# kernels of the backward preparation (g2v_backward_prepare)
_PREP = ("k_split_chunks", "k_fill_cells", "k_region_rows", "k_region_table")


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _launched(fn):
    """Names of the library kernels launched by fn(), and fn's result."""
    from CudaGaussianVoxelizer import _lib
    torch.cuda.synchronize()
    _lib.profile_reset()
    _lib.profile_enable(True)
    try:
        res = fn()
        torch.cuda.synchronize()
    finally:
        _lib.profile_enable(False)
    names = set(_lib.profile_report())
    _lib.profile_reset()
    return names, res


def _prep_kernels(names):
    return sorted(n for n in names if any(p in n for p in _PREP))


def _scene(n=1500, C=24, seed=7, B=None):
    w = W.Workload("inf", n, C, voxel_range=W.RANGE_SMALL, num_outside=20)
    if B is None:
        return W.generate(w, seed=seed)
    parts = [W.generate(w, seed=seed + b) for b in range(B)]
    return tuple(torch.stack([p[k] for p in parts]) for k in range(4))


@pytest.mark.parametrize("batched", [False, True])
def test_inference_forward_prepares_no_backward(batched):
    from CudaGaussianVoxelizer import PyCudaGaussianVoxelizer
    dev = torch.device("cuda")
    m, o, c, f = _scene(B=3 if batched else None)
    vox = PyCudaGaussianVoxelizer(voxel_size=list(W.VOXEL), voxel_range=list(W.RANGE_SMALL))
    md, od, cd, fd = (t.to(dev) for t in (m, o, c, f))
    say(f"[inference] batched={batched}")
    leaves = [t.clone().requires_grad_() for t in (md, od, cd, fd)]
    names_grad, (d0, g0, _) = _launched(lambda: vox(*leaves))
    assert _prep_kernels(names_grad), names_grad          # a training forward prepares the backward
    with torch.no_grad():
        names_ng, (d1, g1, s1) = _launched(lambda: vox(*leaves))
    assert not _prep_kernels(names_ng), _prep_kernels(names_ng)
    names_plain, (d2, g2, _) = _launched(lambda: vox(md, od, cd, fd))   # nothing requires grad
    assert not _prep_kernels(names_plain), _prep_kernels(names_plain)
    for d, g in ((d1, g1), (d2, g2)):
        assert torch.equal(d, d0.detach()) and torch.equal(g, g0.detach())
    assert s1[0] > 0
    # a forward that kept nothing can still be differentiated through the reference-signature path
    # (the Function called directly with need_backward=False rebuilds what it needs)
    from CudaGaussianVoxelizer import _CudaGaussianVoxelizeFunction, _CudaGaussianVoxelizeBatchedFunction
    fn = _CudaGaussianVoxelizeBatchedFunction if batched else _CudaGaussianVoxelizeFunction
    l2 = [t.clone().requires_grad_() for t in (md, od, cd, fd)]
    d3, g3, _ = fn.apply(l2[0], l2[1], l2[2], vox.voxel_size, vox.voxel_range, l2[3], False)
    (d3.sum() + g3.sum()).backward()
    (d0.sum() + g0.sum()).backward()
    for a, b in zip(l2, leaves):
        assert torch.equal(a.grad, b.grad)


def test_batched_noncontiguous_features_with_caller_allocations():
    from CudaGaussianVoxelizer import PyCudaGaussianVoxelizer
    dev = torch.device("cuda")
    B, n, C = 4, 900, 16
    m, o, c, f = _scene(n=n, C=2 * C, seed=30, B=B)
    vox = PyCudaGaussianVoxelizer(voxel_size=list(W.VOXEL), voxel_range=list(W.RANGE_SMALL))
    say("[batched] non-contiguous features, caller-stream allocations between forward and backward")
    leaves = [t.to(dev).requires_grad_() for t in (m, o, c, f)]
    feats = leaves[3][:, :, ::2]                 # (B, n, C), not contiguous
    assert not feats.is_contiguous()
    density, grid_feats, _ = vox(leaves[0], leaves[1], leaves[2], feats)
    # the caller's stream reuses freed memory at once (the forward's temporary feature copy among it)
    junk = [torch.full((1 << 20,), float(k), device=dev) for k in range(16)]
    g = torch.Generator().manual_seed(5)
    gD = torch.randn(*density.shape, generator=g).to(dev)
    gF = torch.randn(*grid_feats.shape, generator=g).to(dev)
    torch.autograd.backward([density, grid_feats], [gD, gF])
    del junk
    for b in range(B):
        lb_ = [leaves[k][b].detach().clone().requires_grad_() for k in range(3)]
        fb = leaves[3][b, :, ::2].detach().contiguous().requires_grad_()
        d1, f1, _ = vox(lb_[0], lb_[1], lb_[2], fb)
        assert torch.equal(d1, density[b].detach()) and torch.equal(f1, grid_feats[b].detach())
        torch.autograd.backward([d1, f1], [gD[b], gF[b]])
        assert torch.equal(lb_[0].grad, leaves[0].grad[b])
        assert torch.equal(lb_[1].grad, leaves[1].grad[b])
        assert torch.equal(lb_[2].grad, leaves[2].grad[b])
        assert torch.equal(fb.grad, leaves[3].grad[b, :, ::2])
        assert not leaves[3].grad[b, :, 1::2].any()
