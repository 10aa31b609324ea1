"""GPU parity of the HIP feature cosine loss (libg2v_hip.so: g2v_cosine_loss_forward/backward)
against the float64 CPU oracle (run on the MI355X box with -m gpu).

Bars: valid-voxel count exact; loss rel < 1e-4; gradient L2-relative < 1e-4 (float32 kernels vs
the float64 restatement of src/cuda_feats_loss.cu:45-366).  Cases cover the three kernel shapes
(16-byte rows held in registers, 16-byte rows too long for registers, any row through scalar
loads), small rows that share a wave between voxels, misaligned rows, empty and all-invalid
grids, rows below the norm clamp, the autograd module, and the module chained behind the
voxelizer.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import g2v_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-4


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


def _inputs(shape, C, seed, valid_frac=0.6, misalign=False):
    g = torch.Generator().manual_seed(seed)
    p = torch.randn(shape + (C,), generator=g)
    q = torch.randn(shape + (C,), generator=g)
    label = torch.randint(-1, 3, shape, generator=g).to(torch.float32)
    mask = torch.rand(shape, generator=g) < valid_frac
    dev = torch.device("cuda")
    if misalign:
        # contiguous tensors whose data starts 4 bytes past a 16-byte boundary
        def shifted(t):
            buf = torch.empty(t.numel() + 1, device=dev)
            v = buf[1:].view(t.shape)
            v.copy_(t.to(dev))
            return v
        pd, qd = shifted(p), shifted(q)
    else:
        pd, qd = p.to(dev), q.to(dev)
    return label, mask, p, q, label.to(dev), mask.to(dev), pd, qd


def _check(shape, C, seed, gout=1.0, **kw):
    label, mask, p, q, ld, md, pd, qd = _inputs(shape, C, seed, **kw)
    say(f"[cosine] shape={shape} C={C} seed={seed} {kw}")
    loss, cnt, fwd_sec = _C().CudaFeatsCosinelossForward(ld, md, pd, qd)
    exp_loss, exp_cnt = O.cosine_loss_f64(label.numpy(), mask.numpy(), p.numpy(), q.numpy())
    assert cnt == exp_cnt
    assert loss.shape == () and loss.device.type == "cuda"
    if exp_cnt > 0:
        assert abs(loss.item() - exp_loss) <= TOL * abs(exp_loss)
    else:
        assert loss.item() == 0.0
    go = torch.tensor(gout, device="cuda")
    grad, bwd_sec = _C().CudaFeatsCosinelossBackward(go, ld, md, pd, qd, cnt)
    exp = O.cosine_loss_grad_f64(gout, label.numpy(), mask.numpy(), p.numpy(), q.numpy(), cnt)
    got = grad.cpu().numpy()
    assert got.shape == exp.shape
    invalid = ~(mask.numpy() & (label.numpy() > 0))
    assert not got[invalid].any()
    if exp_cnt > 0:
        if C > 1:
            assert O.rel_err(got, exp) < TOL
        else:
            # one channel: cos = +-1 exactly and the gradient g (p^2 b / (a D) - 1) / D is what
            # the eps terms leave of two cancelling parts, in the reference's float32 as here;
            # the error is measured against the size of those parts
            pd64, qd64 = p.numpy().astype(np.float64), q.numpy().astype(np.float64)
            a = np.sqrt(np.maximum(pd64 ** 2, O.EPS))
            b = np.sqrt(np.maximum(qd64 ** 2, O.EPS))
            parts = abs(gout) / exp_cnt * 2 * np.abs(qd64) / (a * b + float(O.EPS))
            parts[invalid] = 0
            assert np.linalg.norm(got - exp) <= TOL * np.linalg.norm(parts)
    assert fwd_sec > 0 and bwd_sec > 0
    return loss, grad


@pytest.mark.parametrize("shape,C", [
    ((50, 50, 8), 64),      # config-1 grid, 16 lanes per voxel
    ((20, 20, 16), 1024),   # one wave per voxel, 4 vectors per lane
    ((13, 7, 5), 768),      # 3 vectors per lane, odd grid
    ((9, 9, 4), 2048),      # 8 vectors per lane
    ((6, 5, 4), 3000),      # too long for registers: two-pass kernel
    ((11, 3, 7), 30),       # C % 4 != 0: scalar loads
    ((4, 4, 4), 4),         # one vector per voxel
    ((3, 3, 3), 1),         # one channel
])
def test_cosine_parity(shape, C):
    _check(shape, C, seed=C)


def test_cosine_misaligned_rows():
    _check((10, 10, 4), 256, seed=3, misalign=True)


def test_cosine_upstream_scale():
    _check((8, 8, 8), 128, seed=4, gout=-2.5)


def test_cosine_no_valid_voxel():
    _check((6, 6, 6), 64, seed=5, valid_frac=0.0)


def test_cosine_all_valid_and_tiny_rows():
    label, mask, p, q, ld, md, pd, qd = _inputs((5, 5, 5), 16, 6)
    ld.fill_(1.0)
    md.fill_(True)
    pd[0, 0, 0] = 1e-5          # below the norm clamp: no p term in the gradient
    pd[1, 1, 1] = 0.0           # zero row
    loss, cnt, _ = _C().CudaFeatsCosinelossForward(ld, md, pd, qd)
    assert cnt == 125
    lab, msk, pp, qq = ld.cpu().numpy(), md.cpu().numpy(), pd.cpu().numpy(), qd.cpu().numpy()
    exp_loss, _ = O.cosine_loss_f64(lab, msk, pp, qq)
    assert abs(loss.item() - exp_loss) <= TOL * abs(exp_loss)
    grad, _ = _C().CudaFeatsCosinelossBackward(torch.ones((), device="cuda"), ld, md, pd, qd, cnt)
    assert O.rel_err(grad.cpu().numpy(), O.cosine_loss_grad_f64(1.0, lab, msk, pp, qq, cnt)) < TOL


def test_cosine_empty_grid():
    dev = torch.device("cuda")
    ld = torch.zeros(0, 4, 4, device=dev)
    md = torch.zeros(0, 4, 4, dtype=torch.bool, device=dev)
    pd = torch.zeros(0, 4, 4, 8, device=dev)
    loss, cnt, _ = _C().CudaFeatsCosinelossForward(ld, md, pd, pd.clone())
    assert cnt == 0 and loss.item() == 0.0
    grad, _ = _C().CudaFeatsCosinelossBackward(torch.ones((), device=dev), ld, md, pd, pd.clone(), 0)
    assert grad.shape == pd.shape


def test_cosine_deterministic():
    label, mask, p, q, ld, md, pd, qd = _inputs((30, 30, 8), 512, 7)
    a = _C().CudaFeatsCosinelossForward(ld, md, pd, qd)
    b = _C().CudaFeatsCosinelossForward(ld, md, pd, qd)
    assert a[0].item() == b[0].item() and a[1] == b[1]
    ga, _ = _C().CudaFeatsCosinelossBackward(torch.ones((), device="cuda"), ld, md, pd, qd, a[1])
    gb, _ = _C().CudaFeatsCosinelossBackward(torch.ones((), device="cuda"), ld, md, pd, qd, a[1])
    assert torch.equal(ga, gb)


def test_cosine_input_errors_raise():
    dev = torch.device("cuda")
    ld = torch.ones(4, 4, 4, device=dev)
    md = torch.ones(4, 4, 4, dtype=torch.bool, device=dev)
    pd = torch.randn(4, 4, 4, 8, device=dev)
    with pytest.raises(RuntimeError):
        _C().CudaFeatsCosinelossForward(ld, md.float(), pd, pd)            # mask must be bool
    with pytest.raises(RuntimeError):
        _C().CudaFeatsCosinelossForward(ld.double(), md, pd, pd)           # label must be float32
    with pytest.raises(RuntimeError):
        _C().CudaFeatsCosinelossForward(ld, md, pd.transpose(0, 1), pd)    # not contiguous
    with pytest.raises(RuntimeError):
        _C().CudaFeatsCosinelossForward(ld, md, pd, pd[..., :4].contiguous())   # shape mismatch
    with pytest.raises(RuntimeError):
        _C().CudaFeatsCosinelossForward(ld.cpu(), md, pd, pd)              # not on the GPU


def test_cosine_module_autograd():
    from CudaGaussianVoxelizer import PyCudaFeatsCosineLoss
    label, mask, p, q, ld, md, pd, qd = _inputs((16, 16, 8), 96, 8)
    x = pd.clone().requires_grad_(True)
    mod = PyCudaFeatsCosineLoss()
    loss, stats = mod(ld, md, x, qd)
    assert stats.device.type == "cpu" and stats.dtype == torch.float32 and stats[0] > 0
    (3.0 * loss).backward()
    assert stats[1] > 0
    _, cnt = O.cosine_loss_f64(label.numpy(), mask.numpy(), p.numpy(), q.numpy())
    exp = O.cosine_loss_grad_f64(3.0, label.numpy(), mask.numpy(), p.numpy(), q.numpy(), cnt)
    assert O.rel_err(x.grad.cpu().numpy(), exp) < TOL


def test_cosine_behind_the_voxelizer():
    """grid_feats of the voxelizer -> cosine loss -> backward through both modules: the features'
    gradient equals the voxelizer backward fed with the cosine gradient."""
    from CudaGaussianVoxelizer import PyCudaFeatsCosineLoss, PyCudaGaussianVoxelizer
    from tests import workloads as W
    w = W.CONFIGS[1]
    m, o, c, f = W.generate(w, seed=0)
    dev = torch.device("cuda")
    m, o, c, f = (t.to(dev) for t in (m, o, c, f))
    vox = PyCudaGaussianVoxelizer(w.voxel_size, w.voxel_range)
    cos = PyCudaFeatsCosineLoss(w.voxel_size, w.voxel_range)
    fr = f.clone().requires_grad_(True)
    density, grid_feats, _ = vox(m, o, c, fr)
    gen = torch.Generator().manual_seed(9)
    shape = tuple(density.shape)
    label = torch.randint(0, 3, shape, generator=gen).to(torch.float32).to(dev)
    mask = (torch.rand(shape, generator=gen) < 0.8).to(dev)
    target = torch.randn(shape + (f.shape[1],), generator=gen).to(dev)
    loss, _ = cos(label, mask, grid_feats, target)
    loss.backward()
    # the same chain by hand through the _C entry points
    _C = sys.modules["CudaGaussianVoxelizer._C"]
    out = _C.gaussian_voxelizer_forward(m, o, c, vox.voxel_size, vox.voxel_range, f)
    _, cnt, _ = _C.CudaFeatsCosinelossForward(label, mask, out[5], target)
    gF, _ = _C.CudaFeatsCosinelossBackward(torch.ones((), device=dev), label, mask, out[5], target, cnt)
    gD = torch.zeros_like(out[0])
    ref = _C.gaussian_voxelizer_backward(gD, gF, m, o, out[1], vox.voxel_size, vox.voxel_range, out[2], out[3],
                                         out[4], out[6], out[7], out[0], out[5], f)
    assert O.rel_err(fr.grad.cpu().numpy(), ref[3].cpu().numpy()) < 1e-6


# bfloat16 grid_feats and target: the kernels widen the values exactly and sum in float32 in the
# same order as the float32 path, so on the same values the loss and count are identical and the
# gradient is the float32 gradient rounded to bfloat16 (nearest even), bit for bit.  Cases: rows
# held in registers (C = 1024), rows too long for them (C = 2304), small rows sharing a wave
# (C = 16), scalar rows (C = 13) and rows not aligned to 8 bytes (2-byte offset).
@pytest.mark.parametrize("shape,C,misalign", [((24, 24, 8), 1024, False), ((8, 8, 4), 2304, False),
                                              ((32, 32, 8), 16, False), ((16, 16, 8), 13, False),
                                              ((16, 16, 8), 64, True)])
def test_cosine_bf16_equals_float32_path_on_the_same_values(shape, C, misalign):
    label, mask, p, q, ld, md, pd, qd = _inputs(shape, C, 21)
    dev = torch.device("cuda")
    if misalign:
        def shifted(t):
            buf = torch.empty(t.numel() + 1, dtype=torch.bfloat16, device=dev)
            v = buf[1:].view(t.shape)
            v.copy_(t.to(dev))
            return v
        pb, qb = shifted(pd.bfloat16()), shifted(qd.bfloat16())
    else:
        pb, qb = pd.bfloat16().contiguous(), qd.bfloat16().contiguous()
    say(f"[cosine bf16] shape={shape} C={C} misalign={misalign}")
    lb_, cb, _ = _C().CudaFeatsCosinelossForward(ld, md, pb, qb)
    lf, cf, _ = _C().CudaFeatsCosinelossForward(ld, md, pb.float().contiguous(), qb.float().contiguous())
    assert cb == cf and torch.equal(lb_, lf)
    go = torch.tensor(2.0, device=dev)
    gb, _ = _C().CudaFeatsCosinelossBackward(go, ld, md, pb, qb, cb)
    gf, _ = _C().CudaFeatsCosinelossBackward(go, ld, md, pb.float().contiguous(), qb.float().contiguous(), cf)
    assert gb.dtype == torch.bfloat16 and torch.equal(gb, gf.to(torch.bfloat16))
    # and against the float64 oracle on the rounded values
    exp_loss, exp_cnt = O.cosine_loss_f64(label.numpy(), mask.numpy(), pb.float().cpu().numpy(),
                                          qb.float().cpu().numpy())
    assert cb == exp_cnt and abs(lb_.item() - exp_loss) <= TOL * max(abs(exp_loss), 1e-12)


def test_cosine_bf16_mixed_types_raise():
    dev = torch.device("cuda")
    ld = torch.ones(4, 4, 4, device=dev)
    md = torch.ones(4, 4, 4, dtype=torch.bool, device=dev)
    pd = torch.randn(4, 4, 4, 8, device=dev)
    with pytest.raises(RuntimeError):
        _C().CudaFeatsCosinelossForward(ld, md, pd.bfloat16(), pd)    # target must match grid_feats
    with pytest.raises(RuntimeError):
        _C().CudaFeatsCosinelossForward(ld, md, pd.half(), pd.half())  # float16 is not supported


def test_cosine_bf16_behind_the_bf16_voxelizer():
    """bfloat16 features -> bfloat16 grid_feats -> cosine loss -> backward through both modules, with
    no float32 copy of grid_feats: the cosine gradient arrives in bfloat16 and the feature gradient
    comes back in bfloat16."""
    from CudaGaussianVoxelizer import PyCudaFeatsCosineLoss, PyCudaGaussianVoxelizer
    from tests import workloads as W
    w = W.CONFIGS[1]
    m, o, c, f = W.generate(w, seed=0)
    dev = torch.device("cuda")
    m, o, c = (t.to(dev) for t in (m, o, c))
    vox = PyCudaGaussianVoxelizer(w.voxel_size, w.voxel_range)
    cos = PyCudaFeatsCosineLoss(w.voxel_size, w.voxel_range)
    fr = f.to(dev).bfloat16().requires_grad_(True)
    density, grid_feats, _ = vox(m, o, c, fr)
    assert grid_feats.dtype == torch.bfloat16
    g = torch.Generator().manual_seed(5)
    label = torch.randint(0, 3, density.shape, generator=g).float().to(dev)
    mask = (torch.rand(density.shape, generator=g) < 0.7).to(dev)
    target = torch.randn(grid_feats.shape, generator=g).to(dev).bfloat16()
    say("[cosine bf16] behind the bf16 voxelizer")
    loss, _ = cos(label, mask, grid_feats, target)
    loss.backward()
    assert fr.grad.dtype == torch.bfloat16 and torch.isfinite(fr.grad.float()).all()
    # the same chain on float32 copies of the same values: the loss is identical
    gf = grid_feats.detach().float()
    lf, _, _ = _C().CudaFeatsCosinelossForward(label, mask, gf, target.float())
    assert torch.equal(loss.detach(), lf)
