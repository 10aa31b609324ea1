"""GPU tests of bfloat16 feature I/O (features, grid_feats and the feature gradient in bfloat16;
run on the MI355X box with -m gpu).

With bfloat16 features the kernels split each feature into itself and a zero low part, so the
float32 path fed with the same values (features.bfloat16().float()) multiplies exactly the same
operands.  Bars:
  * density: identical to the float32 path on the same values;
  * grid_feats: the float32 path's grid_feats rounded to bfloat16 (nearest even), bit for bit;
  * gradients of means, covariances, opacity: within rel 1e-5 of the float32 path (fed the upstream
    feature gradient rounded to bfloat16, as the bfloat16 path takes it) when no tile list needs a
    second pass (the only place grid_feats itself is read back).  They are not bit-equal: the
    bfloat16 path sums u = gF . f over 64-channel chunks, the float32 path over 32-channel ones,
    so the float32 partial sums are grouped differently;
  * the feature gradient is the float32 path's rounded to bfloat16, bit for bit (its products do
    not depend on that grouping);
  * against the float64 oracle on the rounded features: density rel < 1e-4, grid_feats and the
    feature gradient rel < 1e-2 (bfloat16 output rounding, 2^-9 relative per element).
"""
import sys

import numpy as np
import pytest
import torch

from oracle import g2v_oracle as O
from oracle import g2v_oracle_c as OC
from tests import workloads as W

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _setup():
    import CudaGaussianVoxelizer._lib as L
    L.load()
    OC.lib()


def _C():
    from CudaGaussianVoxelizer import _C
    return _C


# lists of at most 256 Gaussians per tile (one pass of the feature backward): about 100 per tile
CASES = {
    "small_grid_c64": W.Workload("bf_c64", 700, 64, voxel_range=W.RANGE_SMALL, var_range=(0.2, 1.5)),
    "odd_channels_13": W.Workload("bf_c13", 500, 13, voxel_range=W.RANGE_SMALL, var_range=(0.2, 1.5)),
    "c256": W.Workload("bf_c256", 600, 256, voxel_range=W.RANGE_SMALL, var_range=(0.2, 1.5)),
    # 16-byte grad_feats loads need 8 bfloat16 channels per piece: C = 20 takes the element loads
    "c20_element_loads": W.Workload("bf_c20", 600, 20, voxel_range=W.RANGE_SMALL, var_range=(0.2, 1.5)),
    "single_channel": W.Workload("bf_c1", 600, 1, voxel_range=W.RANGE_SMALL, var_range=(0.2, 1.5)),
}


def _args(w, m, o, c):
    dev = torch.device("cuda")
    return m.to(dev), o.to(dev), c.to(dev), torch.tensor(w.voxel_size, device=dev), torch.tensor(w.voxel_range, device=dev)


@pytest.mark.parametrize("name", list(CASES))
def test_bf16_features_match_float32_path(name):
    w = CASES[name]
    m, o, c, f = W.generate(w, seed=9)
    fb = f.to(torch.bfloat16)
    dev = torch.device("cuda")
    md, od, cd, vs, vr = _args(w, m, o, c)
    say(f"[bf16] {name} forward")
    ob = _C().gaussian_voxelizer_forward(md, od, cd, vs, vr, fb.to(dev))
    of = _C().gaussian_voxelizer_forward(md, od, cd, vs, vr, fb.float().to(dev))
    assert ob[5].dtype == torch.bfloat16 and of[5].dtype == torch.float32
    assert torch.equal(ob[0], of[0])
    assert torch.equal(ob[5], of[5].to(torch.bfloat16))
    for k in (1, 2, 3, 4, 6, 7):
        assert torch.equal(ob[k], of[k])
    # oracle on the rounded features
    b = O.gaussian_boxes(m.numpy(), c.numpy(), np.array(w.voxel_size, np.float32), np.array(w.voxel_range, np.float32))
    D, F = O.forward_f64(m.numpy(), o.numpy(), c.numpy(), fb.float().numpy(), b["lb"], b["ub"],
                         np.array(w.voxel_size, np.float32), np.array(w.voxel_range, np.float32))
    assert O.rel_err(ob[0].cpu().numpy(), D) < 1e-4
    assert O.rel_err(ob[5].float().cpu().numpy(), F) < 1e-2
    # backward
    say(f"[bf16] {name} backward")
    assert int(torch.diff(_C().build_t2g(vs, vr, ob[2], ob[3], ob[6], ob[7])["tile_offsets"]).max()) <= 256
    g = torch.Generator().manual_seed(4)
    gD = torch.randn(*ob[0].shape, generator=g).to(dev)
    gF = torch.randn(*ob[5].shape, generator=g).bfloat16().float().to(dev)   # bfloat16 values
    gb = _C().gaussian_voxelizer_backward(gD, gF.bfloat16(), md, od, ob[1], vs, vr, ob[2], ob[3], ob[4], ob[6],
                                          ob[7], ob[0], ob[5], fb.to(dev))
    gf = _C().gaussian_voxelizer_backward(gD, gF, md, od, of[1], vs, vr, of[2], of[3], of[4], of[6], of[7],
                                          of[0], of[5], fb.float().to(dev))
    assert gb[3].dtype == torch.bfloat16
    for k in range(3):
        assert O.rel_err(gb[k].cpu().numpy(), gf[k].cpu().numpy()) < 1e-5, k
    assert torch.equal(gb[3], gf[3].to(torch.bfloat16))
    ref = O.backward_f64(gD.cpu().numpy(), gF.cpu().numpy(), m.numpy(), o.numpy(), c.numpy(), fb.float().numpy(),
                         b["lb"], b["ub"], np.array(w.voxel_size, np.float32), np.array(w.voxel_range, np.float32),
                         density=ob[0].cpu().numpy(), grid_feats=of[5].cpu().numpy())
    assert O.rel_err(gb[0].cpu().numpy(), ref[0]) < 1e-3
    assert O.rel_err(gb[3].float().cpu().numpy(), ref[3]) < 1e-2


def test_bf16_long_lists_against_oracle():
    """Tile lists longer than one pass read grid_feats back (in bfloat16 here): oracle bars."""
    w = W.Workload("bf_long", 3000, 32, voxel_range=W.RANGE_SMALL, var_range=(0.5, 2.5))
    m, o, c, f = W.generate(w, seed=2)
    fb = f.to(torch.bfloat16)
    dev = torch.device("cuda")
    md, od, cd, vs, vr = _args(w, m, o, c)
    say("[bf16] long lists")
    ob = _C().gaussian_voxelizer_forward(md, od, cd, vs, vr, fb.to(dev))
    assert int(torch.diff(_C().build_t2g(vs, vr, ob[2], ob[3], ob[6], ob[7])["tile_offsets"]).max()) > 256
    g = torch.Generator().manual_seed(5)
    gD = torch.randn(*ob[0].shape, generator=g).to(dev)
    gF = torch.randn(*ob[5].shape, generator=g).bfloat16().float().to(dev)   # bfloat16 values
    # a float32 upstream gradient of bfloat16 features is rounded to bfloat16 (exact here)
    gb = _C().gaussian_voxelizer_backward(gD, gF, md, od, ob[1], vs, vr, ob[2], ob[3], ob[4], ob[6], ob[7],
                                          ob[0], ob[5], fb.to(dev))
    vsn, vrn = np.array(w.voxel_size, np.float32), np.array(w.voxel_range, np.float32)
    b = O.gaussian_boxes(m.numpy(), c.numpy(), vsn, vrn)
    Ainv = np.linalg.inv(c.numpy().reshape(-1, 3, 3).astype(np.float64)).reshape(-1, 9)
    off, tid, _, _, _ = OC.csr(b["tile_lo"], b["tile_hi"], b["tiles"])
    ref = OC.backward(m.numpy(), o.numpy(), Ainv, b["lb"], b["ub"], vsn, vrn, off, tid, fb.float().numpy(),
                      ob[0].cpu().numpy(), ob[5].float().cpu().numpy(), gD.cpu().numpy(), gF.cpu().numpy())
    assert O.rel_err(gb[0].cpu().numpy(), ref[0]) < 1e-3
    assert O.rel_err(gb[1].cpu().numpy(), ref[1]) < 1e-3
    assert O.rel_err(gb[2].cpu().numpy(), ref[2]) < 1e-3
    assert O.rel_err(gb[3].float().cpu().numpy(), ref[3]) < 1e-2


def test_bf16_module_and_batched():
    from CudaGaussianVoxelizer import PyCudaGaussianVoxelizer
    dev = torch.device("cuda")
    w = CASES["small_grid_c64"]
    m, o, c, f = W.generate(w, seed=3)
    vox = PyCudaGaussianVoxelizer(voxel_size=list(w.voxel_size), voxel_range=list(w.voxel_range))
    say("[bf16] module")
    fr = f.to(torch.bfloat16).to(dev).requires_grad_()
    mr = m.to(dev).requires_grad_()
    density, grid_feats, stats = vox(mr, o.to(dev), c.to(dev), fr)
    assert grid_feats.dtype == torch.bfloat16 and density.dtype == torch.float32
    (density.sum() + grid_feats.float().sum()).backward()
    assert fr.grad.dtype == torch.bfloat16 and torch.isfinite(fr.grad.float()).all() and stats[1] > 0
    # batched: two scenes, each equal to the single-scene call
    say("[bf16] batched")
    mb = torch.stack([m, m + 0.3]).to(dev)
    ob_ = torch.stack([o, o]).to(dev)
    cb = torch.stack([c, c]).to(dev)
    fbb = torch.stack([f, f]).to(torch.bfloat16).to(dev)
    outs = _C().gaussian_voxelizer_forward_batched(mb, ob_, cb, vox.voxel_size, vox.voxel_range, fbb)
    for s in range(2):
        ref = _C().gaussian_voxelizer_forward(mb[s], ob_[s], cb[s], vox.voxel_size, vox.voxel_range, fbb[s])
        assert torch.equal(outs[s][5], ref[5]) and torch.equal(outs[s][0], ref[0])


def test_unsupported_feature_type_raises():
    dev = torch.device("cuda")
    w = CASES["small_grid_c64"]
    m, o, c, f = W.generate(w, seed=1)
    md, od, cd, vs, vr = _args(w, m, o, c)
    with pytest.raises(RuntimeError):
        _C().gaussian_voxelizer_forward(md, od, cd, vs, vr, f.to(torch.float16).to(dev))


def test_half_covariances_of_the_recorded_batch():
    """The recorded batch keeps float16 covariances: the module widens them on the device, so the
    outputs equal those of float32 covariances with the same values, and the covariance gradient
    comes back in float16."""
    from CudaGaussianVoxelizer import PyCudaGaussianVoxelizer
    dev = torch.device("cuda")
    m, o, c, vs, vr = W.mmdet_fixture()
    c16 = c.to(torch.float16)   # exact: the fixture's covariances are float16 values
    vox = PyCudaGaussianVoxelizer(voxel_size=list(vs), voxel_range=list(vr))
    say("[bf16] float16 covariances")
    ch = c16.to(dev).requires_grad_()
    d16, _, _ = vox(m.to(dev), o.to(dev), ch)
    d32, _, _ = vox(m.to(dev), o.to(dev), c.to(dev))
    assert torch.equal(d16, d32)
    d16.sum().backward()
    assert ch.grad.dtype == torch.float16 and torch.isfinite(ch.grad.float()).all()
