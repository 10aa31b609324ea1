"""CPU pins of the covariance-construction oracle (oracle.g2v_oracle.covariance_from_scale_rotation_*).

Reference: test/gaussian_voxelizer.py:14-37 (quat_to_rotmat, get_covariance).  Pinned by:
  * closed forms: the identity rotation gives diag(s^2); a quarter turn about z swaps the x and y
    variances; a quaternion and any positive multiple of it give the same covariance;
  * invariants: symmetric, eigenvalues s^2, determinant (s_x s_y s_z)^2;
  * the gradient equals torch autograd (float64) of an independent torch statement and central
    finite differences; planted mistakes (no G + G^T symmetrisation, no 1/|q| of the quaternion
    normalisation) fail the autograd check.
"""
import numpy as np
import pytest
import torch

from oracle import g2v_oracle as O


def _sq(n, seed):
    rng = np.random.default_rng(seed)
    return rng.uniform(0.05, 3.0, (n, 3)), rng.standard_normal((n, 4)) * rng.uniform(0.5, 2.0, (n, 1))


def test_identity_rotation_gives_diagonal():
    s = np.array([[0.5, 2.0, 3.0]])
    cov = O.covariance_from_scale_rotation_f64(s, np.array([[1.0, 0, 0, 0]])).reshape(3, 3)
    np.testing.assert_allclose(cov, np.diag(s[0] ** 2), atol=1e-15)


def test_quarter_turn_about_z_swaps_x_and_y():
    s = np.array([[0.5, 2.0, 3.0]])
    h = np.sqrt(0.5)
    cov = O.covariance_from_scale_rotation_f64(s, np.array([[h, 0, 0, h]])).reshape(3, 3)
    np.testing.assert_allclose(cov, np.diag([4.0, 0.25, 9.0]), atol=1e-14)


def test_invariants_and_normalisation():
    s, q = _sq(50, 1)
    cov = O.covariance_from_scale_rotation_f64(s, q).reshape(-1, 3, 3)
    np.testing.assert_allclose(cov, cov.transpose(0, 2, 1), atol=1e-13)
    np.testing.assert_allclose(np.sort(np.linalg.eigvalsh(cov), 1), np.sort(s ** 2, 1), rtol=1e-10)
    np.testing.assert_allclose(np.linalg.det(cov), np.prod(s ** 2, 1), rtol=1e-10)
    np.testing.assert_allclose(O.covariance_from_scale_rotation_f64(s, 7.5 * q).reshape(-1, 3, 3), cov, atol=1e-13)


def _torch_cov(s, q):
    """Independent float64 torch statement, differentiated by autograd."""
    ts = torch.tensor(s, requires_grad=True)
    tq = torch.tensor(q, requires_grad=True)
    qn = tq / tq.norm(dim=-1, keepdim=True)
    w, x, y, z = qn.unbind(-1)
    R = torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
                     2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
                     2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1).reshape(-1, 3, 3)
    M = R @ torch.diag_embed(ts)
    return ts, tq, (M @ M.mT).reshape(-1, 9)


@pytest.mark.parametrize("seed", [2, 3])
def test_gradient_matches_torch_autograd(seed):
    s, q = _sq(40, seed)
    G = np.random.default_rng(seed + 10).standard_normal((40, 9))   # not symmetric on purpose
    ts, tq, cov = _torch_cov(s, q)
    np.testing.assert_allclose(cov.detach().numpy(), O.covariance_from_scale_rotation_f64(s, q), atol=1e-13)
    (cov * torch.tensor(G)).sum().backward()
    gs, gq = O.covariance_from_scale_rotation_grad_f64(s, q, G)
    assert O.rel_err(gs, ts.grad.numpy()) < 1e-12
    assert O.rel_err(gq, tq.grad.numpy()) < 1e-12


def test_gradient_matches_finite_differences():
    s, q = _sq(3, 4)
    G = np.random.default_rng(5).standard_normal((3, 9))
    gs, gq = O.covariance_from_scale_rotation_grad_f64(s, q, G)
    h = 1e-6

    def loss(s_, q_):
        return (O.covariance_from_scale_rotation_f64(s_, q_) * G).sum()

    fs, fq = np.zeros_like(s), np.zeros_like(q)
    for idx in np.ndindex(s.shape):
        a, b = s.copy(), s.copy()
        a[idx] += h
        b[idx] -= h
        fs[idx] = (loss(a, q) - loss(b, q)) / (2 * h)
    for idx in np.ndindex(q.shape):
        a, b = q.copy(), q.copy()
        a[idx] += h
        b[idx] -= h
        fq[idx] = (loss(s, a) - loss(s, b)) / (2 * h)
    assert O.rel_err(gs, fs) < 1e-7 and O.rel_err(gq, fq) < 1e-7


def test_planted_mistakes_are_caught():
    s, q = _sq(20, 6)
    G = np.random.default_rng(7).standard_normal((20, 9))
    ts, tq, cov = _torch_cov(s, q)
    (cov * torch.tensor(G)).sum().backward()
    # without the symmetrisation G + G^T: the scale gradient of G M alone
    R, _ = O._rotmat_f64(q)
    M = R * s[:, None, :]
    gs_bad = ((G.reshape(-1, 3, 3) @ M) * R).sum(1)
    assert O.rel_err(gs_bad, ts.grad.numpy()) > 0.1
    # without the 1/|q| of the normalisation (the quaternions here are not unit length)
    _, gq = O.covariance_from_scale_rotation_grad_f64(s, q, G)
    gq_bad = gq * np.linalg.norm(q, axis=1, keepdims=True)
    assert O.rel_err(gq_bad, tq.grad.numpy()) > 0.1
