"""Shared builders for the GPU parity tests (seeded synthetic chunks and the
oracle comparisons with the stated bf16 tolerance)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import mtp_oracle as mo

# Tolerance for attention outputs and gradients against the reference:
# max-abs error <= 2e-2 and mean-abs error <= 2e-3.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def chunk_layout(n_reg, n_anchor, draft, P, seed=0, pad=0, tail=False, every=None):
    if every is not None:
        anchors = np.arange(0, n_reg, every)[:n_anchor]
    else:
        anchors = mo.sample_anchors(n_reg, n_anchor, seed)
    seq = mo.synth_sequence(n_reg, anchors, draft, pos0=P, tail_unlabelled=tail)
    return mo.pad_to(seq, len(seq.gate) + pad)


def qkv(S, P, Hq, Hkv, D, dtype, dev, seed=0, std=0.5):
    """q/k/v in the projection layout [1, S, H, D] viewed as [1, H, S, D];
    prefix K/V [1, Hkv, P, D]; dO ~ N(0, 1) in [1, S, Hq, D]."""
    gens = [torch.Generator(device=dev).manual_seed(seed * 16 + i) for i in range(6)]
    r = lambda shape, g, s: (torch.randn(*shape, generator=g, device=dev) * s).to(dtype)
    q = r((1, S, Hq, D), gens[0], std).transpose(1, 2)
    k = r((1, S, Hkv, D), gens[1], std).transpose(1, 2)
    v = r((1, S, Hkv, D), gens[2], std).transpose(1, 2)
    kp = r((1, Hkv, P, D), gens[3], std)
    vp = r((1, Hkv, P, D), gens[4], std)
    do = r((1, S, Hq, D), gens[5], 1.0)
    return q, k, v, kp, vp, do


def f64(t):
    return t.detach().double().cpu().numpy()


def check(name, got, ref, max_abs=MAX_ABS, mean_abs=MEAN_ABS, scale_above_one=False, tensor_scale=False):
    """max |got - ref| <= max_abs and mean |got - ref| <= mean_abs.

    scale_above_one: the max bound applies to |got - ref| / max(1, |ref|),
    i.e. absolute where |ref| <= 1 and relative above. For a bf16 output of
    magnitude 4..8 one rounding alone is up to 2^-6 = 0.0156, and the bf16
    probabilities the dV / dK products multiply add about as much again, so
    the absolute 2e-2 is then below what any bf16 implementation (the
    reference's flex path included) can meet; the mean bound stays absolute.

    tensor_scale: both bounds scale by max(1, max |ref|) of the whole tensor,
    for data whose outputs are sums of terms far larger than themselves (an
    element's error then follows the terms, not its own magnitude)."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    err = np.abs(g - r)
    mx, mn = float(err.max()) if err.size else 0.0, float(err.mean()) if err.size else 0.0
    lim = err / np.maximum(1.0, np.abs(r)) if scale_above_one else err
    mxs = float(lim.max()) if lim.size else 0.0
    big = float(np.abs(r).max()) if r.size else 0.0
    if tensor_scale:
        max_abs, mean_abs = max_abs * max(1.0, big), mean_abs * max(1.0, big)
        print(f"  {name}: bounds x max(1, max |ref|) = x{max(1.0, big):.2f}", flush=True)
    print(f"  {name}: max-abs {mx:.3e} mean-abs {mn:.3e}"
          + (f" max-abs/max(1,|ref|) {mxs:.3e} (max |ref| {big:.2f})" if scale_above_one else ""), flush=True)
    assert np.isfinite(got).all(), f"{name} has non-finite values"
    assert mxs <= max_abs and mn <= mean_abs, f"{name}: max-abs {mx:.3e} ({mxs:.3e}) mean-abs {mn:.3e}"


def torch_dense_reference(q, kfull, vfull, allowed, scale, do=None, grad_start=0):
    """fp32 dense masked attention on the GPU with autograd, one query head at
    a time (for shapes the float64 numpy oracle is too slow for). Inputs are
    the kernel's own bf16 values upcast to fp32; the prefix gets no gradient."""
    Hq, S, D = q.shape[1], q.shape[2], q.shape[3]
    Hkv = kfull.shape[1]
    G = Hq // Hkv
    m = torch.as_tensor(allowed, device=q.device)
    rowok = m.any(dim=1)
    o = torch.empty(Hq, S, D, device=q.device, dtype=torch.float32)
    lse = torch.empty(Hq, S, device=q.device, dtype=torch.float32)
    dq = torch.empty_like(o) if do is not None else None
    L = kfull.shape[2]
    dk = torch.zeros(Hkv, L - grad_start, D, device=q.device) if do is not None else None
    dv = torch.zeros_like(dk) if do is not None else None
    for h in range(Hq):
        g = h // G
        qh = q[0, h].float().detach().requires_grad_(do is not None)
        kh = kfull[0, g].float().detach().requires_grad_(do is not None)
        vh = vfull[0, g].float().detach().requires_grad_(do is not None)
        s = (qh @ kh.T) * scale
        s = s.masked_fill(~m, float("-inf"))
        lse[h] = torch.where(rowok, torch.logsumexp(s, dim=1), torch.full_like(lse[h], float("-inf"))).detach()
        p = torch.where(rowok[:, None], torch.softmax(s.masked_fill(~rowok[:, None], 0.0), dim=1), 0.0)
        oh = p @ vh
        o[h] = oh.detach()
        if do is not None:
            oh.backward(do[0, :, h].float())
            dq[h] = qh.grad
            dk[g] += kh.grad[grad_start:]
            dv[g] += vh.grad[grad_start:]
    return o, lse, dq, dk, dv


def round_to(dtype):
    """fp64 -> the values of a 16-bit torch dtype, as fp64 (round to nearest even)."""
    return lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dtype).double().numpy()


def rounding_model_grad_errors(q, k, v, do, allowed, scale, grad_start, rnd):
    """Error against float64 of attention gradients computed with only the
    reference's 16-bit rounding points, everything else in float64: the
    forward's output is stored in the operand dtype and delta = rowsum(out *
    grad_out) is formed from that stored output
    ([torch]_inductor/kernel/flex/flex_attention.py:750-751), and the compiled
    backward casts P to the operand dtype before dV = P^T dO and dS before dQ
    and dK (flex_backwards.py.jinja:570-618) and stores dQ, dK and dV in the
    operand dtype (:177, 273, 287). Returns {name: (max-abs, mean-abs)} for dq,
    dk, dv: the error floor of any implementation with those rounding points on
    these inputs."""
    o, lse = mo.attention_fwd(q, k, v, allowed, scale)
    exact = mo.attention_bwd(q, k, v, o, lse, do, allowed, scale, grad_start=grad_start)
    Hq, S, D = q.shape
    Hkv, L, _ = k.shape
    G = Hq // Hkv
    dq = np.zeros((Hq, S, D))
    dk = np.zeros((Hkv, L, D))
    dv = np.zeros((Hkv, L, D))
    for h in range(Hq):
        g = h // G
        s = scale * (q[h] @ k[g].T)
        rowok = np.isfinite(lse[h])
        p = np.where(allowed & rowok[:, None], np.exp(s - np.where(rowok, lse[h], 0.0)[:, None]), 0.0)
        dv[g] += rnd(p).T @ do[h]
        ds = rnd(p * (do[h] @ v[g].T - (rnd(o[h]) * do[h]).sum(axis=1)[:, None]))
        dq[h] = scale * (ds @ k[g])
        dk[g] += scale * (ds.T @ q[h])
    got = (rnd(dq), rnd(dk[:, grad_start:]), rnd(dv[:, grad_start:]))
    return {n: (float(np.abs(a - b).max()), float(np.abs(a - b).mean()))
            for n, a, b in zip(("dq", "dk", "dv"), got, exact)}


def torch_rounding_model_grads(q, kfull, vfull, allowed, scale, do, grad_start, dtype):
    """rounding_model_grad_errors' gradients computed on the GPU in fp32 (for the
    full-size stream shapes the float64 oracle is too slow for): the
    reference's 16-bit rounding points -- the stored output that delta is
    formed from, P before dV = P^T dO, dS before dQ and dK, and the 16-bit
    gradient stores -- and fp32 everywhere else, one query head at a time.
    Returns dq [Hq, S, D], dk, dv [Hkv, L - grad_start, D] as fp32 tensors."""
    rnd = lambda t: t.to(dtype).float()
    Hq, S, D = q.shape[1], q.shape[2], q.shape[3]
    Hkv, L = kfull.shape[1], kfull.shape[2]
    G = Hq // Hkv
    m = torch.as_tensor(allowed, device=q.device)
    rowok = m.any(dim=1)
    dq = torch.empty(Hq, S, D, device=q.device)
    dk = torch.zeros(Hkv, L, D, device=q.device)
    dv = torch.zeros(Hkv, L, D, device=q.device)
    for h in range(Hq):
        g = h // G
        qh, kh, vh = q[0, h].float(), kfull[0, g].float(), vfull[0, g].float()
        doh = do[0, :, h].float()
        s = ((qh @ kh.T) * scale).masked_fill(~m, float("-inf"))
        lse = torch.where(rowok, torch.logsumexp(s, dim=1), torch.zeros_like(s[:, 0]))
        p = torch.where(m & rowok[:, None], torch.exp(s - lse[:, None]), torch.zeros_like(s))
        del s
        o = rnd(p @ vh)
        dv[g] += rnd(p).T @ doh
        ds = rnd(p * (doh @ vh.T - (o * doh).sum(dim=1)[:, None]))
        del p
        dq[h] = scale * (ds @ kh)
        dk[g] += scale * (ds.T @ qh)
        del ds
    return rnd(dq), rnd(dk[:, grad_start:]), rnd(dv[:, grad_start:])


def check_grad(name, got, ref, model, k=2.0, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    """A gradient against the exact reference: within the absolute bound
    (max-abs max_abs, mean-abs mean_abs), or within k times the max- and
    mean-abs error of the reference's rounding model on the same inputs
    (model: its gradient, or its (max-abs, mean-abs) errors), whichever is
    larger. The model measures what the 16-bit rounding points alone cost: with
    |dV| near 7, one bf16 rounding is 1.6e-2, so an absolute 2e-2 is then below
    what the reference's own flex path can meet."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    if isinstance(model, tuple):
        mmx, mmn = model
    else:
        me = np.abs(np.asarray(model, np.float64) - r)
        mmx, mmn = float(me.max()), float(me.mean())
    err = np.abs(g - r)
    mx, mn = float(err.max()), float(err.mean())
    bmx, bmn = max(max_abs, k * mmx), max(mean_abs, k * mmn)
    print(f"  {name}: max-abs {mx:.3e} mean-abs {mn:.3e}; rounding model max-abs {mmx:.3e} "
          f"mean-abs {mmn:.3e}; bounds {bmx:.3e} / {bmn:.3e} (k = {k})", flush=True)
    assert np.isfinite(g).all(), f"{name} has non-finite values"
    assert mx <= bmx and mn <= bmn, f"{name}: max-abs {mx:.3e} mean-abs {mn:.3e} > bounds {bmx:.3e} / {bmn:.3e}"
