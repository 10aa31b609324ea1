"""CPU pins of the cosine-loss oracle (oracle.g2v_oracle.cosine_loss_f64 / cosine_loss_grad_f64).

The reference is src/cuda_feats_loss.cu:45-366 (forward mean loss over the valid voxels, gradient
with respect to grid_feats).  What pins the restatement without running the reference:
  * closed forms of the per-voxel loss: parallel rows give eps-sized losses, antiparallel rows
    give 2 - eps-sized, orthogonal rows give exactly 1, rows below the norm clamp use sqrt(eps);
  * the valid-voxel rule (mask and label > 0; a label of exactly 0 or below is out) and the
    empty case (loss 0, count 0, zero gradient);
  * the gradient equals torch autograd of the loss (clamp_min / sqrt), which differentiates
    independently of the closed-form coefficients, and central finite differences;
  * planted mistakes (a flipped sign of the p coefficient, a dropped 1/count) fail those checks.
"""
import numpy as np
import pytest
import torch

from oracle import g2v_oracle as O

EPS = float(np.float32(1e-6))   # the reference's float eps (include/utils.cuh:80)


def _rows(shape, C, seed):
    rng = np.random.default_rng(seed)
    p = rng.standard_normal(shape + (C,)).astype(np.float32)
    g = rng.standard_normal(shape + (C,)).astype(np.float32)
    label = rng.integers(-1, 3, size=shape).astype(np.float32)
    mask = rng.random(shape) < 0.7
    return label, mask, p, g


def _all_valid(shape):
    return np.ones(shape, np.float32), np.ones(shape, bool)


def test_parallel_antiparallel_orthogonal_closed_forms():
    shape = (1, 1, 3)
    label, mask = _all_valid(shape)
    g = np.zeros(shape + (4,), np.float32)
    g[..., 0] = 2.0
    p = np.zeros_like(g)
    p[0, 0, 0, 0] = 3.0      # parallel: |p||g| = 6, dot = 6
    p[0, 0, 1, 0] = -3.0     # antiparallel
    p[0, 0, 2, 1] = 5.0      # orthogonal
    loss, cnt = O.cosine_loss_f64(label, mask, p, g)
    assert cnt == 3
    expect = [1 - 6 / (6 + EPS), 1 + 6 / (6 + EPS), 1.0]
    assert loss == pytest.approx(sum(expect) / 3, rel=1e-12)


def test_norm_clamp_below_eps():
    """|p|^2 < eps: the norm is sqrt(eps) (src/cuda_feats_loss.cu:96-98)."""
    label, mask = _all_valid((1, 1, 1))
    p = np.full((1, 1, 1, 2), 1e-4, np.float32)          # |p|^2 = 2e-8 < eps
    g = np.array([[[[3.0, 4.0]]]], np.float32)            # |g| = 5
    loss, _ = O.cosine_loss_f64(label, mask, p, g)
    dot = float(p[0, 0, 0] @ g[0, 0, 0].astype(np.float64))
    assert loss == pytest.approx(1 - dot / (np.sqrt(EPS) * 5 + EPS), rel=1e-12)


def test_valid_voxel_rule_and_mean():
    shape = (2, 2, 2)
    label, mask, p, g = _rows(shape, 5, 0)
    label[0, 0, 0], mask[0, 0, 0] = 0.0, True     # label exactly 0: out
    label[0, 0, 1], mask[0, 0, 1] = 2.0, False    # masked: out
    label[0, 1, 0], mask[0, 1, 0] = -1.0, True    # negative label: out
    label[1, 1, 1], mask[1, 1, 1] = 0.5, True     # in
    valid = mask & (label > 0)
    loss, cnt = O.cosine_loss_f64(label, mask, p, g)
    assert cnt == int(valid.sum()) and cnt >= 1
    per = [1 - float(a @ b) / (np.linalg.norm(a) * np.linalg.norm(b) + EPS)
           for a, b in zip(p.astype(np.float64)[valid], g.astype(np.float64)[valid])]
    assert loss == pytest.approx(np.mean(per), rel=1e-9)


def test_no_valid_voxel_gives_zero_loss_and_gradient():
    shape = (3, 2, 2)
    label, mask, p, g = _rows(shape, 6, 1)
    mask[:] = False
    loss, cnt = O.cosine_loss_f64(label, mask, p, g)
    assert (loss, cnt) == (0.0, 0)
    grad = O.cosine_loss_grad_f64(1.0, label, mask, p, g, cnt)
    assert not grad.any()


def _torch_loss(label, mask, p, g):
    """Float64 torch statement of the loss, differentiated by autograd."""
    valid = torch.tensor(mask & (label > 0))
    tp = torch.tensor(p, dtype=torch.float64, requires_grad=True)
    tg = torch.tensor(g, dtype=torch.float64)
    dot = (tp * tg).sum(-1)
    a = (tp * tp).sum(-1).clamp_min(EPS).sqrt()
    b = (tg * tg).sum(-1).clamp_min(EPS).sqrt()
    lv = 1 - dot / (a * b + EPS)
    n = int(valid.sum())
    loss = lv[valid].sum() / n
    return tp, loss


@pytest.mark.parametrize("seed,C", [(2, 7), (3, 32)])
def test_gradient_matches_torch_autograd(seed, C):
    shape = (3, 4, 2)
    label, mask, p, g = _rows(shape, C, seed)
    p[0, 0, 0] *= 1e-5        # one valid-or-not row below the norm clamp
    label[0, 0, 0], mask[0, 0, 0] = 1.0, True
    tp, loss = _torch_loss(label, mask, p, g)
    gout = 0.75
    (gout * loss).backward()
    _, cnt = O.cosine_loss_f64(label, mask, p, g)
    grad = O.cosine_loss_grad_f64(gout, label, mask, p, g, cnt)
    assert O.rel_err(grad, tp.grad.numpy()) < 1e-10
    assert loss.item() == pytest.approx(O.cosine_loss_f64(label, mask, p, g)[0], rel=1e-12)


def test_gradient_matches_finite_differences():
    shape = (2, 2, 1)
    label, mask = _all_valid(shape)
    rng = np.random.default_rng(4)
    p = rng.standard_normal(shape + (3,))
    g = rng.standard_normal(shape + (3,))
    _, cnt = O.cosine_loss_f64(label, mask, p, g)
    grad = O.cosine_loss_grad_f64(1.0, label, mask, p, g, cnt)
    h = 1e-6
    fd = np.zeros_like(p)
    for idx in np.ndindex(p.shape):
        q = p.copy()
        q[idx] += h
        lp = O.cosine_loss_f64(label, mask, q, g)[0]
        q[idx] -= 2 * h
        lm = O.cosine_loss_f64(label, mask, q, g)[0]
        fd[idx] = (lp - lm) / (2 * h)
    assert O.rel_err(grad, fd) < 1e-6


def test_planted_mistakes_are_caught_by_autograd():
    """The oracle's gradient with a flipped p coefficient, or without the 1/count, fails."""
    shape = (2, 3, 2)
    label, mask, p, g = _rows(shape, 9, 5)
    label[:], mask[:] = 1.0, True
    tp, loss = _torch_loss(label, mask, p, g)
    loss.backward()
    _, cnt = O.cosine_loss_f64(label, mask, p, g)
    good = O.cosine_loss_grad_f64(1.0, label, mask, p, g, cnt)
    assert O.rel_err(good, tp.grad.numpy()) < 1e-10
    # flipped sign of c2: grad' = c1 g - c2 p = 2 c1 g - grad (per row, scaled)
    gd = g.astype(np.float64)
    pd = p.astype(np.float64)
    a = np.sqrt(np.maximum((pd * pd).sum(-1), EPS))
    b = np.sqrt(np.maximum((gd * gd).sum(-1), EPS))
    c1 = -1.0 / (a * b + EPS) / cnt
    flipped = 2 * c1[..., None] * gd - good
    assert O.rel_err(flipped, tp.grad.numpy()) > 0.1
    assert O.rel_err(good * cnt, tp.grad.numpy()) > 0.1
