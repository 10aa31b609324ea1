"""GPU parity of the box kernel on the degenerate Gaussians that the oracle pins on the CPU
(tests/test_oracle.py): singular covariances (det = 0 and a small negative det, both clamped to
+1e-6 as in src/cuda_gaussian_voxelizer.cu:201-220), zero variance, negative variance (sqrt gives
NaN and fmaxf/fminf turn the box into the whole axis, .cu:372-374, :418-424), a box edge on an
exact voxel boundary, Gaussians wholly outside each of the six faces (empty boxes, .cu:472-497)
and one centred outside that still reaches in (clipped, .cu:418-468).

Boxes, voxel counts, the bits of the inverse covariances and both CSRs are compared bit-exactly
with the oracle; density and grid_feats (rel 1e-4) and every gradient (rel 1e-3) against the
float64 oracle evaluated with the same float32 inverse covariances.  Runs through the C ABI via
the reference-compatible ``_C`` module.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import g2v_oracle as O
from tests import workloads as W

pytestmark = pytest.mark.gpu

VS = (0.4, 0.4, 0.4)
VR = tuple(W.RANGE_SMALL)   # 50 x 50 x 8 voxels


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _diag(*v):
    return np.diag(np.asarray(v, np.float32)).reshape(9)


def _cases(finite_only):
    """(name, mean, row-major covariance) of every degenerate case.  finite_only leaves out the
    non-symmetric singular matrix, whose clamped inverse (adjugate / 1e-6) sends the weights to
    infinity, so that density and gradients stay comparable."""
    lo, hi = np.asarray(VR[:3], np.float32), np.asarray(VR[3:], np.float32)
    cases = []
    # exact voxel boundary: mu - 3 sigma = -9.2, the lower edge of voxel 2
    var = np.float32((np.float32(0.8) / np.float32(3.0)) ** 2)
    sig = np.sqrt(var, dtype=np.float32)
    cases.append(("voxel_boundary", [np.float32(-9.2) + np.float32(3.0) * sig, 0.3, 0.5], _diag(var, 1.0, 0.2)))
    cases.append(("zero_variance", [0.1, 0.1, 0.1], _diag(0.0, 0.0, 0.0)))
    cases.append(("negative_variance", [0.0, 0.0, 0.0], _diag(-1.0, 1.0, 1.0)))
    # symmetric, small negative determinant: clamped to +1e-6 (the sign of the inverse flips)
    cases.append(("small_negative_det", [1.0, -2.0, 0.4], _diag(-1e-3, 1e-3, 1e-3)))
    # rank one, positive semi-definite: det = 0, adjugate 0, so the clamped inverse is 0 (w = o)
    v = np.array([0.6, 1.2, 0.3], np.float32)
    cases.append(("rank_one_psd", [-3.0, 4.0, 0.9], np.outer(v, v).reshape(9).astype(np.float32)))
    cases.append(("centred_outside_clipped", [11.5, 0.0, 0.0], _diag(1.0, 1.0, 1.0)))
    for axis in range(3):
        for side in (-1, 1):
            mu = np.zeros(3, np.float32)
            mu[axis] = (hi[axis] + 3.5) if side > 0 else (lo[axis] - 3.5)
            cases.append((f"outside_{'+-'[side < 0]}{'xyz'[axis]}", mu, _diag(1.0, 1.0, 1.0)))
    if not finite_only:
        cases.append(("singular_nonsymmetric", [2.0, 2.0, 0.5],
                      np.array([1, 2, 3, 2, 4, 6, 1, 1, 1], np.float32)))
    return cases


def _inputs(finite_only, seed=0, C=6):
    cases = _cases(finite_only)
    m = torch.tensor(np.array([np.asarray(c[1], np.float32) for c in cases]))
    cov = torch.tensor(np.array([c[2] for c in cases]))
    g = torch.Generator().manual_seed(seed)
    o = torch.rand(len(cases), generator=g) * 0.8 + 0.2
    f = torch.randn(len(cases), C, generator=g)
    return [c[0] for c in cases], m, o, cov, f


def _np(t):
    return t.detach().cpu().numpy()


def _forward(m, o, c, f):
    from CudaGaussianVoxelizer import _C
    dev = torch.device("cuda")
    out = _C.gaussian_voxelizer_forward(m.to(dev), o.to(dev), c.to(dev), torch.tensor(VS, device=dev),
                                        torch.tensor(VR, device=dev), f.to(dev))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("finite_only", [False, True])
def test_degenerate_boxes_and_csr_bit_exact(finite_only):
    from CudaGaussianVoxelizer import _C
    names, m, o, c, f = _inputs(finite_only)
    say(f"[degenerate boxes] {len(names)} Gaussians: {', '.join(names)}")
    out = _forward(m, o, c, f)
    vs, vr = np.array(VS, np.float32), np.array(VR, np.float32)
    b = O.gaussian_boxes(m.numpy(), c.numpy(), vs, vr)
    for k, name in enumerate(names):
        assert tuple(_np(out[2])[k]) == tuple(b["lb"][k]), name
        assert tuple(_np(out[3])[k]) == tuple(b["ub"][k]), name
        assert _np(out[4])[k] == b["nvox"][k], name
        np.testing.assert_array_equal(_np(out[1])[k].view(np.int32), b["cov_inv"][k].view(np.int32), err_msg=name)
    # the cases the oracle pins by hand come out as it says on the device too
    idx = {n: k for k, n in enumerate(names)}
    lb, ub = _np(out[2]), _np(out[3])
    assert tuple(lb[idx["zero_variance"]]) == (25, 25, 2) == tuple(ub[idx["zero_variance"]])
    assert lb[idx["negative_variance"]][0] == 0 and ub[idx["negative_variance"]][0] == 49
    assert lb[idx["small_negative_det"]][0] == 0 and ub[idx["small_negative_det"]][0] == 49
    assert _np(out[1])[idx["small_negative_det"]][0] > 0        # the sign flip of the det clamp
    assert not _np(out[1])[idx["rank_one_psd"]].any()           # adjugate 0 / 1e-6
    assert lb[idx["centred_outside_clipped"]][0] == 46 and ub[idx["centred_outside_clipped"]][0] == 49
    for name in names:
        if name.startswith("outside_"):
            k = idx[name]
            assert _np(out[4])[k] == 0 and tuple(lb[k]) == (0, 0, 0) and tuple(ub[k]) == (-1, -1, -1), name
            assert not _np(out[1])[k].any(), name
    off, tid, gid = O.g2t_csr(b["tile_lo"], b["tile_hi"], b["tiles"])
    np.testing.assert_array_equal(_np(out[6]), off)
    np.testing.assert_array_equal(_np(out[7]), tid)
    t = O.t2g_csr(tid, gid, int(np.prod(b["tiles"])))
    d = _C.build_t2g(VS, VR, out[2], out[3], out[6], out[7])
    np.testing.assert_array_equal(_np(d["sorted_tiles"]), t["sorted_tiles"])
    np.testing.assert_array_equal(_np(d["sorted_gauss"]), t["sorted_gauss"])
    np.testing.assert_array_equal(_np(d["tile_offsets"]), t["tile_offsets"])


def test_degenerate_forward_and_backward():
    from CudaGaussianVoxelizer import _C
    dev = torch.device("cuda")
    names, m, o, c, f = _inputs(True, seed=3)
    say(f"[degenerate fwd/bwd] {len(names)} Gaussians")
    out = _forward(m, o, c, f)
    vs, vr = np.array(VS, np.float32), np.array(VR, np.float32)
    b = O.gaussian_boxes(m.numpy(), c.numpy(), vs, vr)
    D, F = O.forward_f64(m.numpy(), o.numpy(), c.numpy(), f.numpy(), b["lb"], b["ub"], vs, vr,
                         cov_inv=b["cov_inv"])
    assert np.isfinite(D).all() and D.max() > 0
    eD, eF = O.rel_err(_np(out[0]), D), O.rel_err(_np(out[5]), F)
    say(f"   density {eD:.2e} grid_feats {eF:.2e}")
    assert eD < 1e-4 and eF < 1e-4
    X, Y, Z = b["dims"]
    g = torch.Generator().manual_seed(4)
    gD = torch.randn(X, Y, Z, generator=g)
    gF = torch.randn(X, Y, Z, f.shape[1], generator=g)
    res = _C.gaussian_voxelizer_backward(gD.to(dev), gF.to(dev), m.to(dev), o.to(dev), out[1],
                                         torch.tensor(VS, device=dev), torch.tensor(VR, device=dev), out[2], out[3],
                                         out[4], out[6], out[7], out[0], out[5], f.to(dev))
    torch.cuda.synchronize()
    ref = O.backward_f64(gD.numpy(), gF.numpy(), m.numpy(), o.numpy(), c.numpy(), f.numpy(), b["lb"], b["ub"],
                         vs, vr, density=_np(out[0]), grid_feats=_np(out[5]), cov_inv=b["cov_inv"])
    errs = [O.rel_err(_np(res[k]), ref[k]) for k in range(4)]
    say(f"   grads means/cov/opacity/features {errs}")
    assert max(errs) < 1e-3, errs
    # per Gaussian as well: the negative-variance case has weights up to e^50 and would hide the
    # others in a norm over all of them (a floor of 1e-7 of the largest row covers exact zeros,
    # e.g. the mean gradient of the zero-variance case, whose inverse covariance is 0)
    for k, what in enumerate(("means", "cov", "opacity", "features")):
        a = _np(res[k]).reshape(len(names), -1).astype(np.float64)
        r = ref[k].reshape(len(names), -1)
        scale = np.linalg.norm(r, axis=1)
        floor = 1e-7 * scale.max()
        for gi, name in enumerate(names):
            err = np.linalg.norm(a[gi] - r[gi])
            assert err <= 1e-3 * scale[gi] + floor, (what, name, err, scale[gi])
