"""CPU oracle for the stable soft cross-entropy of the MTP sampler loss (numpy,
float64).

TEST INFRASTRUCTURE. Only ``tests/`` and the ``cpu_baseline`` leg of
``bench.py`` import this module, and only as the checker. The product package
never imports it and has no CPU fallback.

What it restates (``mtp_glora/core/loss.py`` of the reference checkout):

* ``soft_ce_rows``  - per row of student logits x and teacher logits t,
      ce = -(sum_j e^{t_j - mt} x_j) / dt + mx + log dx,
      mx = max x, dx = max(sum_j e^{x_j - mx}, 1e-20),
      mt = max t, dt = max(sum_j e^{t_j - mt}, 1e-20),
  i.e. ``_compute_loss_logits_no_prob`` (loss.py:14-28) per row, which is what
  ``stable_soft_ce_forward_kernel_*`` (loss.py:63-124) store, together with the
  saved statistics (mx, dx, mt, dt) (loss.py:119-124).
* ``soft_ce_grad``  - the backward kernels (loss.py:188-222):
      grad_x = go * (e^{x - mx} / dx - e^{t - mt} / dt);
  the teacher gets no gradient (loss.py:330).
* ``soft_ce_prob_form`` - ``_compute_loss_prob`` (loss.py:8-12): the sum of
  -softmax(t) . log_softmax(x) over rows, the form the reference's own test
  (loss.py:335-385) compares against.

The loss is the sum over rows (loss.py:294). Parity pins live in
``tests/test_oracle_soft_ce.py``.
"""
from __future__ import annotations

import numpy as np

CLAMP = 1e-20   # loss.py:85, 112, 203-205


def _rows(a) -> np.ndarray:
    a = np.asarray(a, dtype=np.float64)
    return a.reshape(-1, a.shape[-1])


def soft_ce_rows(student, teacher):
    """Per-row loss and the (mx, dx, mt, dt) statistics, float64."""
    x, t = _rows(student), _rows(teacher)
    assert x.shape == t.shape
    mx = x.max(axis=1)
    dx = np.maximum(np.exp(x - mx[:, None]).sum(axis=1), CLAMP)
    mt = t.max(axis=1)
    et = np.exp(t - mt[:, None])
    dt = np.maximum(et.sum(axis=1), CLAMP)
    s = (et * x).sum(axis=1)
    ce = -(s / dt) + mx + np.log(dx)
    return ce, np.stack([mx, dx, mt, dt])


def soft_ce_loss(student, teacher) -> float:
    """The autograd Function's forward value: the sum of the row losses."""
    return float(soft_ce_rows(student, teacher)[0].sum())


def soft_ce_grad(student, teacher, grad_output: float = 1.0):
    """d loss / d student, shaped like ``student``."""
    x, t = _rows(student), _rows(teacher)
    _, (mx, dx, mt, dt) = soft_ce_rows(x, t)
    g = grad_output * (np.exp(x - mx[:, None]) / dx[:, None] - np.exp(t - mt[:, None]) / dt[:, None])
    return g.reshape(np.shape(student))


def soft_ce_prob_form(student, teacher) -> float:
    """sum over rows of -softmax(t) . log_softmax(x) (loss.py:8-12)."""
    x, t = _rows(student), _rows(teacher)
    lx = x - x.max(axis=1, keepdims=True)
    log_sm = lx - np.log(np.exp(lx).sum(axis=1, keepdims=True))
    lt = np.exp(t - t.max(axis=1, keepdims=True))
    p = lt / lt.sum(axis=1, keepdims=True)
    return float(-(p * log_sm).sum())
