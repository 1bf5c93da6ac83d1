"""Pins for the oracle's dense masked attention (forward and backward).

Checked against library routines: torch's eager ``flex_attention`` with the
reference BlockMask (the reference's own CPU path), torch autograd of a dense
float64 implementation, ``scaled_dot_product_attention`` where the MTP mask
reduces to plain causal attention, and closed-form special cases.
"""
import math

import numpy as np
import pytest
import torch

from oracle import flex_ref as fr
from oracle import mtp_oracle as mo


def make_case(seed, n_reg, n_anchor, D_draft, P, Hq, Hkv, D, pad=0, tail=False):
    rng = np.random.default_rng(seed)
    anchors = rng.choice(n_reg, size=n_anchor, replace=False)
    seq = mo.pad_to(mo.synth_sequence(n_reg, anchors, D_draft, tail_unlabelled=tail),
                    n_reg + n_anchor * D_draft + pad)
    S = len(seq.gate)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, Hq, S, D, generator=g, dtype=torch.float64) * 0.5
    k = torch.randn(1, Hkv, P + S, D, generator=g, dtype=torch.float64) * 0.5
    v = torch.randn(1, Hkv, P + S, D, generator=g, dtype=torch.float64) * 0.5
    do = torch.randn(1, Hq, S, D, generator=g, dtype=torch.float64)
    return seq, q, k, v, do


def dense_autograd(q, k, v, allowed, scale, do):
    """Textbook masked attention in float64 with torch autograd; fully masked
    rows produce 0 (torch._safe_softmax semantics)."""
    q = q.clone().requires_grad_()
    k = k.clone().requires_grad_()
    v = v.clone().requires_grad_()
    G = q.shape[1] // k.shape[1]
    kk = k.repeat_interleave(G, dim=1)
    vv = v.repeat_interleave(G, dim=1)
    s = scale * q @ kk.transpose(-1, -2)
    m = torch.tensor(allowed)[None, None]
    s = s.masked_fill(~m, float("-inf"))
    p = torch._safe_softmax(s, dim=-1)
    o = p @ vv
    o.backward(do)
    return o.detach(), q.grad, k.grad, v.grad


CASES = [
    dict(seed=0, n_reg=200, n_anchor=20, D_draft=4, P=0, Hq=4, Hkv=2, D=16),
    dict(seed=1, n_reg=150, n_anchor=30, D_draft=4, P=130, Hq=4, Hkv=1, D=8),
    dict(seed=2, n_reg=100, n_anchor=10, D_draft=3, P=64, Hq=2, Hkv=2, D=16, pad=40),
    dict(seed=3, n_reg=80, n_anchor=40, D_draft=8, P=200, Hq=8, Hkv=2, D=8, tail=True),
]


@pytest.mark.parametrize("c", CASES)
def test_forward_matches_flex_eager(c):
    seq, q, k, v, _ = make_case(**c)
    P = c["P"]
    scale = c["D"] ** -0.5
    gate = torch.tensor(seq.gate)[None]
    bm = fr.reference_block_mask(gate, P)
    o_ref, lse_ref = fr.reference_attention(q, k, v, bm, scale)
    o, lse = mo.attention_fwd(q[0].numpy(), k[0].numpy(), v[0].numpy(),
                              mo.mtp_mask_dense(seq.gate, P), scale)
    assert np.allclose(o, o_ref[0].numpy(), atol=1e-10)
    lr = lse_ref[0].numpy()
    assert np.array_equal(np.isneginf(lse), np.isneginf(lr))
    fin = np.isfinite(lse)
    assert np.allclose(lse[fin], lr[fin], atol=1e-10)


@pytest.mark.parametrize("c", CASES)
def test_backward_matches_autograd_and_flex(c):
    seq, q, k, v, do = make_case(**c)
    P = c["P"]
    scale = c["D"] ** -0.5
    allowed = mo.mtp_mask_dense(seq.gate, P)
    o_a, dq_a, dk_a, dv_a = dense_autograd(q, k, v, allowed, scale, do)
    o, lse = mo.attention_fwd(q[0].numpy(), k[0].numpy(), v[0].numpy(), allowed, scale)
    dq, dk, dv = mo.attention_bwd(q[0].numpy(), k[0].numpy(), v[0].numpy(), o, lse, do[0].numpy(),
                                  allowed, scale)
    assert np.allclose(o, o_a[0].numpy(), atol=1e-12)
    assert np.allclose(dq, dq_a[0].numpy(), atol=1e-10)
    assert np.allclose(dk, dk_a[0].numpy(), atol=1e-10)
    assert np.allclose(dv, dv_a[0].numpy(), atol=1e-10)
    # and against flex_attention's own backward (eager, library)
    bm = fr.reference_block_mask(torch.tensor(seq.gate)[None], P)
    _, _, dq_f, dk_f, dv_f = fr.reference_attention(q, k, v, bm, scale, do=do)
    assert np.allclose(dq, dq_f[0].numpy(), atol=1e-9)
    assert np.allclose(dk, dk_f[0].numpy(), atol=1e-9)
    assert np.allclose(dv, dv_f[0].numpy(), atol=1e-9)
    # the detached prefix: grad_start drops exactly the first P key rows
    dq2, dk2, dv2 = mo.attention_bwd(q[0].numpy(), k[0].numpy(), v[0].numpy(), o, lse,
                                     do[0].numpy(), allowed, scale, grad_start=P)
    assert np.array_equal(dk2, dk[:, P:]) and np.array_equal(dv2, dv[:, P:])


def test_reduces_to_causal_sdpa():
    """All-regular chunk, empty prefix: the MTP mask is the causal mask."""
    g = torch.Generator().manual_seed(5)
    S, Hq, Hkv, D = 150, 4, 2, 16
    q = torch.randn(1, Hq, S, D, generator=g, dtype=torch.float64)
    k = torch.randn(1, Hkv, S, D, generator=g, dtype=torch.float64)
    v = torch.randn(1, Hkv, S, D, generator=g, dtype=torch.float64)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
    o, _ = mo.attention_fwd(q[0].numpy(), k[0].numpy(), v[0].numpy(),
                            mo.mtp_mask_dense(np.zeros(S, np.int64), 0), D ** -0.5)
    assert np.allclose(o, ref[0].numpy(), atol=1e-12)


def test_special_rows():
    """A pad row is all zero with LSE -inf and no gradient; the first regular
    token (sees only itself) outputs its own V row with LSE = scale * q.k."""
    seq = mo.pad_to(mo.synth_sequence(20, [4, 9], 2), 30)
    S, D = len(seq.gate), 8
    rng = np.random.default_rng(0)
    q = rng.standard_normal((2, S, D))
    k = rng.standard_normal((1, S, D))
    v = rng.standard_normal((1, S, D))
    do = rng.standard_normal((2, S, D))
    allowed = mo.mtp_mask_dense(seq.gate, 0)
    o, lse = mo.attention_fwd(q, k, v, allowed, 0.3)
    pad = seq.gate == -1
    assert (o[:, pad] == 0).all() and np.isneginf(lse[:, pad]).all()
    assert np.allclose(o[:, 0], v[0, 0])
    assert np.allclose(lse[:, 0], 0.3 * (q[:, 0] @ k[0, 0]))
    dq, dk, dv = mo.attention_bwd(q, k, v, o, lse, do, allowed, 0.3)
    assert (dq[:, pad] == 0).all() and (dk[:, pad] == 0).all() and (dv[:, pad] == 0).all()


def test_mha_is_gqa_with_one_group():
    rng = np.random.default_rng(1)
    S, D = 40, 8
    q = rng.standard_normal((2, S, D))
    k = rng.standard_normal((2, S, D))
    v = rng.standard_normal((2, S, D))
    allowed = mo.mtp_mask_dense(mo.synth_sequence(32, [3, 7], 4).gate, 0)
    o, _ = mo.attention_fwd(q, k, v, allowed, 0.2)
    for h in range(2):
        oh, _ = mo.attention_fwd(q[h:h + 1], k[h:h + 1], v[h:h + 1], allowed, 0.2)
        assert np.allclose(o[h], oh[0])
