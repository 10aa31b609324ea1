"""GPU tests of the feature cosine loss's gradient fused into the voxelizer's backward
(g2v_backward_cosine through PyCudaGaussianVoxelizerCosineLoss and
_C.gaussian_voxelizer_backward_cosine; run with -m gpu).

The fused kernels form k1 pseudo_gt + k2 grid_feats per voxel inside the feature-gradient phases
instead of reading a materialised gradient of grid_feats.  Bars:
* against the chained path (PyCudaGaussianVoxelizer -> PyCudaFeatsCosineLoss -> autograd, which
  writes that gradient and reads it back): forward outputs and loss identical, every input
  gradient within L2-relative 1e-4;
* against the float64 oracle chain (cosine_loss_grad_f64 -> backward_f64): 1e-3, the backward bar.
Cases: 64 channels on the 50 x 50 x 8 grid; 1024 channels (32 K chunks); 4 channels (one 16-byte
row piece); lists longer than one
256-entry pass of phase A (its t_v from the rows); a grid whose dimensions are not multiples of 4
(voxels past the grid in boundary tiles); no valid voxel (k = 0); the un-prepared entry point
(CSR rebuilt from the reference's backward arguments); and types the fused kernels do not take
(C % 4 != 0, bfloat16), which the module chains instead.  The library's launch record shows which
kernels ran.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import g2v_oracle as O
from tests import workloads as W

pytestmark = pytest.mark.gpu

TOL = 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


CASES = {
    "c64": W.Workload("c64", 1500, 64, voxel_range=W.RANGE_SMALL, num_outside=20),
    "c1024": W.Workload("c1024", 900, 1024, voxel_range=W.RANGE_SMALL),
    "long_lists": W.Workload("wide", 3000, 32, var_range=(2.0, 12.0), mean_pad=4.0),
    "ragged_grid": W.Workload("ragged", 1200, 16, voxel_range=(-10.0, -10.0, -1.0, 9.6, 9.2, 1.8)),
    "four_channels": W.Workload("c4", 1200, 4, voxel_range=W.RANGE_SMALL),
}


def _loss_inputs(shape, C, seed, valid_frac=0.7):
    g = torch.Generator().manual_seed(seed)
    dev = torch.device("cuda")
    label = torch.randint(-1, 3, shape, generator=g).to(torch.float32).to(dev)
    mask = (torch.rand(shape, generator=g) < valid_frac).to(dev)
    target = torch.randn(shape + (C,), generator=g).to(dev)
    gD = torch.randn(shape, generator=g).to(dev)
    return label, mask, target, gD


def _launched(fn):
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


def _both(w, seed=0, valid_frac=0.7, gl=1.7, feats_dtype=torch.float32):
    """Chained and fused runs of density.gD + gl * loss on the same inputs: (outputs, grads) of each
    and the kernel names of the fused backward."""
    from CudaGaussianVoxelizer import (PyCudaFeatsCosineLoss, PyCudaGaussianVoxelizer,
                                       PyCudaGaussianVoxelizerCosineLoss)
    dev = torch.device("cuda")
    m, o, c, f = W.generate(w, seed=seed)
    f = f.to(feats_dtype)
    shape = W.grid_shape(w)
    label, mask, target, gD = _loss_inputs(shape, f.shape[1], seed + 11, valid_frac)
    target = target.to(feats_dtype)
    glt = torch.tensor(gl, device=dev)
    vox = PyCudaGaussianVoxelizer(list(w.voxel_size), list(w.voxel_range))
    cos = PyCudaFeatsCosineLoss(list(w.voxel_size), list(w.voxel_range))
    fused = PyCudaGaussianVoxelizerCosineLoss(list(w.voxel_size), list(w.voxel_range))

    a = [t.to(dev).requires_grad_() for t in (m, o, c, f)]
    d1, g1, _ = vox(*a)
    l1, _ = cos(label, mask, g1, target)
    torch.autograd.backward([d1, l1], [gD, glt])

    b = [t.to(dev).requires_grad_() for t in (m, o, c, f)]
    d2, l2, g2, stats = fused(b[0], b[1], b[2], b[3], label, mask, target)
    assert g2.requires_grad   # grid_feats keeps its gradient path (unused here: None reaches the backward)
    names, _ = _launched(lambda: torch.autograd.backward([d2, l2], [gD, glt]))
    assert stats[0] > 0 and stats[1] > 0
    return (d1, g1, l1), (d2, g2, l2), [t.grad for t in a], [t.grad for t in b], names, \
        (m, o, c, f, label, mask, target, gD)


def _fused_kernels(names):
    return any("k_bwd_tile<true, false, true>" in n for n in names) and \
        any("k_bwd_region<false, true, true>" in n for n in names)


@pytest.mark.parametrize("name", list(CASES))
def test_fused_equals_chained(name):
    w = CASES[name]
    say(f"[cosine fused] {name}: n={w.n} C={w.feat_dim} grid={W.grid_shape(w)}")
    (d1, g1, l1), (d2, g2, l2), ga, gb, names, _ = _both(w)
    assert torch.equal(d1, d2) and torch.equal(g1, g2) and torch.equal(l1, l2)
    assert _fused_kernels(names), sorted(names)
    assert not any("k_cos_bwd" in n for n in names), sorted(names)   # no gradient of grid_feats written
    errs = [O.rel_err(y.cpu().numpy(), x.cpu().numpy()) for x, y in zip(ga, gb)]
    say(f"   rel err means/opacity/cov/features vs chained: {errs}")
    assert max(errs) < TOL, errs


@pytest.mark.parametrize("name", list(CASES))
def test_fused_against_the_f64_oracle_chain(name):
    w = CASES[name]
    say(f"[cosine fused] float64 oracle chain, {name}")
    _, (d2, g2, l2), _, gb, _, (m, o, c, f, label, mask, target, gD) = _both(w, gl=2.3)
    vs, vr = np.array(w.voxel_size, np.float32), np.array(w.voxel_range, np.float32)
    bx = O.gaussian_boxes(m.numpy(), c.numpy(), vs, vr)
    lab, msk, tgt = label.cpu().numpy(), mask.cpu().numpy(), target.cpu().numpy()
    gfe = g2.detach().cpu().numpy()
    count = int(O.cosine_valid(lab, msk).sum())
    gF = O.cosine_loss_grad_f64(2.3, lab, msk, gfe, tgt, count)
    ref = O.backward_f64(gD.cpu().numpy(), gF, m.numpy(), o.numpy(), c.numpy(), f.numpy(), bx["lb"], bx["ub"], vs, vr,
                         density=d2.detach().cpu().numpy(), grid_feats=gfe, cov_inv=bx["cov_inv"])
    got = [gb[0], gb[2], gb[1], gb[3]]   # means, cov, opacity, features (the oracle's order)
    errs = [O.rel_err(g.cpu().numpy().reshape(r.shape), r) for g, r in zip(got, ref)]
    say(f"   rel err vs oracle: {errs}")
    assert max(errs) < 1e-3, errs


def test_fused_no_valid_voxel():
    """Nothing valid: count 0, every k = 0; the gradients are the density term's alone."""
    w = CASES["c64"]
    say("[cosine fused] no valid voxel")
    (d1, g1, l1), (d2, g2, l2), ga, gb, names, _ = _both(w, valid_frac=0.0)
    assert float(l2.detach()) == 0.0 and torch.equal(l1, l2)
    assert _fused_kernels(names)
    errs = [O.rel_err(y.cpu().numpy(), x.cpu().numpy()) for x, y in zip(ga, gb)]
    assert max(errs[:3]) < TOL, errs
    assert not gb[3].any() and not ga[3].any()   # features: only the loss reaches them


def test_unprepared_entry_point_rebuilds_the_csr():
    """_C.gaussian_voxelizer_backward_cosine from the reference's backward arguments (no kept CSR,
    no prepared workspace) against the chained entry points."""
    from CudaGaussianVoxelizer import _C
    w = CASES["ragged_grid"]
    dev = torch.device("cuda")
    say("[cosine fused] un-prepared entry point")
    m, o, c, f = (t.to(dev) for t in W.generate(w, seed=4))
    vs = torch.tensor(w.voxel_size, device=dev)
    vr = torch.tensor(w.voxel_range, device=dev)
    out = _C.gaussian_voxelizer_forward(m, o, c, vs, vr, f)
    label, mask, target, gD = _loss_inputs(tuple(out[0].shape), f.shape[1], 21)
    loss, cnt, _, coef = _C._cosine_forward(label, mask, out[5], target, True)
    loss0, cnt0, _ = _C.CudaFeatsCosinelossForward(label, mask, out[5], target)
    assert torch.equal(loss, loss0) and cnt == cnt0
    gl = torch.tensor([0.8], device=dev)
    gF, _ = _C.CudaFeatsCosinelossBackward(gl, label, mask, out[5], target, cnt)
    ref = _C.gaussian_voxelizer_backward(gD, gF, m, o, out[1], vs, vr, out[2], out[3], out[4], out[6], out[7],
                                         out[0], out[5], f)
    got = _C.gaussian_voxelizer_backward_cosine(gD, gl, target, coef, cnt, m, o, out[1], vs, vr, out[2], out[3],
                                                out[4], out[6], out[7], out[0], out[5], f)
    errs = [O.rel_err(got[k].cpu().numpy(), ref[k].cpu().numpy()) for k in range(4)]
    say(f"   rel err means/cov/opacity/features: {errs}")
    assert max(errs) < TOL, errs


@pytest.mark.parametrize("dtype,C", [(torch.float32, 30), (torch.bfloat16, 64)])
def test_types_outside_the_fused_kernels_chain(dtype, C):
    """C % 4 != 0 or bfloat16: the module chains the loss's backward into the voxelizer's; the
    results are the separate modules'."""
    w = W.Workload("chain", 1200, C, voxel_range=W.RANGE_SMALL)
    say(f"[cosine fused] chained fallback {dtype} C={C}")
    (d1, g1, l1), (d2, g2, l2), ga, gb, names, _ = _both(w, feats_dtype=dtype)
    assert torch.equal(d1, d2) and torch.equal(g1, g2) and torch.equal(l1, l2)
    assert not _fused_kernels(names)
    assert any("k_cos_bwd" in n for n in names)
    for x, y in zip(ga, gb):
        assert torch.equal(x, y)


def test_fused_input_errors_raise():
    from CudaGaussianVoxelizer import _C
    dev = torch.device("cuda")
    w = CASES["c64"]
    m, o, c, f = (t.to(dev) for t in W.generate(w, seed=1))
    vs = torch.tensor(w.voxel_size, device=dev)
    vr = torch.tensor(w.voxel_range, device=dev)
    out = _C.gaussian_voxelizer_forward(m, o, c, vs, vr, f)
    label, mask, target, gD = _loss_inputs(tuple(out[0].shape), f.shape[1], 3)
    _, cnt, _, coef = _C._cosine_forward(label, mask, out[5], target, True)
    gl = torch.ones(1, device=dev)
    args = lambda cf, tg: (gD, gl, tg, cf, cnt, m, o, out[1], vs, vr, out[2], out[3], out[4], out[6], out[7],
                           out[0], out[5], f)
    with pytest.raises(RuntimeError):   # coefficients of the wrong size
        _C.gaussian_voxelizer_backward_cosine(*args(coef[:-1].contiguous(), target))
    with pytest.raises(RuntimeError):   # target of another shape
        _C.gaussian_voxelizer_backward_cosine(*args(coef, target[..., :32].contiguous()))


def test_grid_feats_used_elsewhere_too():
    """grid_feats of the fused module also feeds another loss: its gradient reaches the Gaussians
    (the module then chains), and every input gradient equals the separate modules' with the same
    second use."""
    from CudaGaussianVoxelizer import (PyCudaFeatsCosineLoss, PyCudaGaussianVoxelizer,
                                       PyCudaGaussianVoxelizerCosineLoss)
    w = CASES["c64"]
    dev = torch.device("cuda")
    say("[cosine fused] grid_feats used by a second loss")
    m, o, c, f = W.generate(w, seed=6)
    label, mask, target, gD = _loss_inputs(W.grid_shape(w), f.shape[1], 7)
    wgt = torch.randn(W.grid_shape(w) + (f.shape[1],), generator=torch.Generator().manual_seed(8)).to(dev)
    a = [t.to(dev).requires_grad_() for t in (m, o, c, f)]
    d1, g1, _ = PyCudaGaussianVoxelizer(list(w.voxel_size), list(w.voxel_range))(*a)
    l1, _ = PyCudaFeatsCosineLoss()(label, mask, g1, target)
    ((d1 * gD).sum() + 1.3 * l1 + (g1 * wgt).sum()).backward()
    b = [t.to(dev).requires_grad_() for t in (m, o, c, f)]
    d2, l2, g2, _ = PyCudaGaussianVoxelizerCosineLoss(list(w.voxel_size), list(w.voxel_range))(*b, label, mask, target)
    ((d2 * gD).sum() + 1.3 * l2 + (g2 * wgt).sum()).backward()
    errs = [O.rel_err(y.grad.cpu().numpy(), x.grad.cpu().numpy()) for x, y in zip(a, b)]
    say(f"   rel err means/opacity/cov/features vs chained: {errs}")
    assert max(errs) < TOL, errs
    # the second use moves the gradients: without it they differ
    c_ = [t.to(dev).requires_grad_() for t in (m, o, c, f)]
    d3, l3, _, _ = PyCudaGaussianVoxelizerCosineLoss(list(w.voxel_size), list(w.voxel_range))(*c_, label, mask, target)
    ((d3 * gD).sum() + 1.3 * l3).backward()
    assert O.rel_err(c_[3].grad.cpu().numpy(), b[3].grad.cpu().numpy()) > 1e-2


def test_loss_alone_backward():
    """loss.backward() alone: the density and grid_feats outputs get no gradient (None reaches the
    fused backward, no zero-filled tensors are made) and the gradients equal the chained ones."""
    from CudaGaussianVoxelizer import (PyCudaFeatsCosineLoss, PyCudaGaussianVoxelizer,
                                       PyCudaGaussianVoxelizerCosineLoss)
    w = CASES["c64"]
    dev = torch.device("cuda")
    say("[cosine fused] loss alone")
    m, o, c, f = W.generate(w, seed=2)
    label, mask, target, _ = _loss_inputs(W.grid_shape(w), f.shape[1], 5)
    a = [t.to(dev).requires_grad_() for t in (m, o, c, f)]
    _, g1, _ = PyCudaGaussianVoxelizer(list(w.voxel_size), list(w.voxel_range))(*a)
    l1, _ = PyCudaFeatsCosineLoss()(label, mask, g1, target)
    l1.backward()
    b = [t.to(dev).requires_grad_() for t in (m, o, c, f)]
    _, l2, _, _ = PyCudaGaussianVoxelizerCosineLoss(list(w.voxel_size), list(w.voxel_range))(*b, label, mask,
                                                                                               target)
    l2.backward()
    errs = [O.rel_err(y.grad.cpu().numpy(), x.grad.cpu().numpy()) for x, y in zip(a, b)]
    say(f"   rel err means/opacity/cov/features vs chained: {errs}")
    assert max(errs) < TOL, errs
