"""Pins for oracle/soft_ce.py (the stable soft cross-entropy of
mtp_glora/core/loss.py) that do not restate its formula:

* the probability form (log_softmax against softmax targets, loss.py:8-12)
  through torch's own log_softmax / softmax, as the reference's test does
  (loss.py:335-385), at its shapes and tolerances;
* the gradient against torch autograd of that form and against central
  finite differences;
* closed-form special cases: a one-hot teacher reduces to torch's
  cross_entropy; identical student and teacher give zero gradient and the
  entropy of softmax(x); a constant added to a row changes nothing.
"""
import numpy as np
import pytest
import torch

from oracle import soft_ce as sc


def _torch_prob_form(x, t):
    x = torch.as_tensor(x, dtype=torch.float64).requires_grad_()
    t = torch.as_tensor(t, dtype=torch.float64)
    loss = -(torch.softmax(t, dim=-1) * torch.log_softmax(x, dim=-1)).sum()
    loss.backward()
    return loss.item(), x.grad.numpy()


@pytest.mark.parametrize("shape,tol", [((4, 4, 4096), 2e-4), ((2, 3, 20011), 3e-4)])
def test_matches_torch_prob_form(shape, tol):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(*shape, generator=g).numpy()
    t = torch.randn(*shape, generator=g).numpy()
    ref_loss, ref_grad = _torch_prob_form(x, t)
    assert abs(sc.soft_ce_loss(x, t) - ref_loss) <= tol * (1 + abs(ref_loss))
    assert abs(sc.soft_ce_prob_form(x, t) - ref_loss) <= 1e-9 * (1 + abs(ref_loss))
    np.testing.assert_allclose(sc.soft_ce_grad(x, t), ref_grad, rtol=tol, atol=tol)
    # float64 against float64: the forms agree far below the reference's tolerance
    np.testing.assert_allclose(sc.soft_ce_grad(x, t), ref_grad, rtol=1e-9, atol=1e-12)


def test_gradient_finite_differences():
    rng = np.random.default_rng(1)
    x = rng.normal(size=(3, 17)) * 2
    t = rng.normal(size=(3, 17)) * 2
    g = sc.soft_ce_grad(x, t, grad_output=0.75)
    h = 1e-6
    num = np.zeros_like(x)
    for i in range(x.shape[0]):
        for j in range(x.shape[1]):
            xp, xm = x.copy(), x.copy()
            xp[i, j] += h
            xm[i, j] -= h
            num[i, j] = 0.75 * (sc.soft_ce_loss(xp, t) - sc.soft_ce_loss(xm, t)) / (2 * h)
    np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-9)


def test_one_hot_teacher_is_cross_entropy():
    rng = np.random.default_rng(2)
    x = rng.normal(size=(5, 300))
    labels = rng.integers(0, 300, size=5)
    t = np.full_like(x, -1e4)
    t[np.arange(5), labels] = 0.0
    ref = torch.nn.functional.cross_entropy(torch.as_tensor(x), torch.as_tensor(labels), reduction="sum").item()
    assert abs(sc.soft_ce_loss(x, t) - ref) <= 1e-9 * (1 + abs(ref))


def test_identical_logits():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(4, 1000)) * 3
    np.testing.assert_allclose(sc.soft_ce_grad(x, x), 0.0, atol=1e-15)
    p = np.exp(x - x.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    entropy = -(p * np.log(p)).sum()
    assert abs(sc.soft_ce_loss(x, x) - entropy) <= 1e-9 * entropy


def test_shift_invariance():
    rng = np.random.default_rng(4)
    x = rng.normal(size=(3, 500))
    t = rng.normal(size=(3, 500))
    cx = rng.normal(size=(3, 1)) * 50
    ct = rng.normal(size=(3, 1)) * 50
    assert abs(sc.soft_ce_loss(x + cx, t + ct) - sc.soft_ce_loss(x, t)) < 1e-8
    np.testing.assert_allclose(sc.soft_ce_grad(x + cx, t + ct), sc.soft_ce_grad(x, t), atol=1e-12)


def test_statistics():
    rng = np.random.default_rng(5)
    x = rng.normal(size=(2, 64))
    t = rng.normal(size=(2, 64))
    ce, (mx, dx, mt, dt) = sc.soft_ce_rows(x, t)
    np.testing.assert_allclose(mx + np.log(dx), np.log(np.exp(x).sum(axis=1)), rtol=1e-12)
    np.testing.assert_allclose(mt + np.log(dt), np.log(np.exp(t).sum(axis=1)), rtol=1e-12)
    assert ce.shape == (2,)
