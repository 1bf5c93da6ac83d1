"""CPU oracle for the Qwen3 query/key normalisation + rotary embedding (numpy).

TEST INFRASTRUCTURE. Only ``tests/`` and the ``cpu_baseline`` leg of
``bench.py`` import this module, and only as the checker. The product package
never imports it and has no CPU fallback.

What it restates (``mtp_glora/models/modeling_qwen3.py`` of the reference
checkout), per row x of D elements (one head of one token) in the model dtype T:

* ``norm_rope``  - Qwen3RMSNorm.forward (:61-67) followed by
  apply_rotary_pos_emb (:125-149) with rotate_half (:118-122), as
  Qwen3Attention.forward calls them (:274-279):
      var = mean(x * x)  (fp32),  r = 1 / sqrt(var + eps)  (fp32),
      n   = T(w * T(x * r)),
      out = T(T(n * cos) + T(rotate_half(n) * sin)),
      rotate_half(n) = [-n[D/2:], n[:D/2]],
  where T rounds fp32 to the model dtype (round to nearest even) for bf16 and
  fp16 operands and is the identity for fp32 ones. Each torch op on bf16 tensors computes in fp32
  and rounds once, which is what T after every op restates. The mean is
  numpy's fp32 sum times fp32(1/D) (torch's mean reduction multiplies by the
  reciprocal of the count), and r is the correctly rounded fp32 of the
  float64 1/sqrt, so ``var`` and ``r`` may differ from a GPU's in the last
  fp32 bit (different summation order, approximate rsqrt).
* ``norm_rope_grad`` - the gradient of the same map with respect to x in
  float64 with every T taken as identity (the backward of the HIP kernel
  computes in fp32 on that model):
      dn = g * cos + [g[D/2:] * sin[D/2:], -g[:D/2] * sin[:D/2]],
      dy = w * dn,  dx = r * dy - (r^3 / D) * x * sum(dy * x).

Parity pins live in ``tests/test_oracle_qk_rope.py``.
"""
from __future__ import annotations

import numpy as np


def bf16_round(a) -> np.ndarray:
    """fp32 -> nearest bf16 (ties to even), returned as fp32. Finite inputs."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def f16_round(a) -> np.ndarray:
    """fp32 -> nearest fp16 (ties to even; past 65504 -> inf), returned as fp32."""
    with np.errstate(over="ignore"):
        return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def _rounder(rnd):
    if rnd is True or rnd == "bf16":
        return bf16_round
    if rnd == "f16":
        return f16_round
    if rnd is False or rnd == "f32":
        return lambda a: np.asarray(a, dtype=np.float32)
    raise ValueError(f"rounding mode {rnd!r}")


def norm_rope(x, w, cos, sin, eps: float, rnd):
    """x [S, H, D], w [D], cos / sin [S, D] (values already in the model dtype).
    rnd: the model dtype's rounding, "bf16" (or True), "f16", "f32" (or False).

    Returns (out [S, H, D] fp32 holding model-dtype values, r [S, H] fp32)."""
    T = _rounder(rnd)
    x = np.asarray(x, dtype=np.float32)
    S, H, D = x.shape
    half = D // 2
    var = (x * x).sum(axis=-1, dtype=np.float32) * np.float32(1.0 / D)
    r = (1.0 / np.sqrt(var.astype(np.float64) + np.float64(np.float32(eps)))).astype(np.float32)
    y = T(x * r[..., None])
    n = T(np.asarray(w, dtype=np.float32)[None, None, :] * y)
    c = np.asarray(cos, dtype=np.float32)[:, None, :]
    s = np.asarray(sin, dtype=np.float32)[:, None, :]
    rot = np.concatenate([-n[..., half:], n[..., :half]], axis=-1)
    out = T(T(n * c) + T(rot * s))
    return out, r


def norm_rope_grad(x, w, cos, sin, g, eps: float):
    """d(sum(out * g)) / dx in float64, roundings as identity; shapes as norm_rope."""
    x = np.asarray(x, dtype=np.float64)
    g = np.asarray(g, dtype=np.float64)
    S, H, D = x.shape
    half = D // 2
    c = np.asarray(cos, dtype=np.float64)[:, None, :]
    s = np.asarray(sin, dtype=np.float64)[:, None, :]
    gs = g * s
    dn = g * c + np.concatenate([gs[..., half:], -gs[..., :half]], axis=-1)
    dy = dn * np.asarray(w, dtype=np.float64)[None, None, :]
    r = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    dot = (dy * x).sum(axis=-1, keepdims=True)
    return r * dy - (r ** 3 / D) * x * dot


def rope_tables(positions, D: int, theta: float = 1_000_000.0):
    """cos / sin [S, D] of the rotary embedding at integer positions (float64):
    inv_freq = theta^(-2i/D), angles = pos * inv_freq, duplicated over both
    halves (Qwen3RotaryEmbedding.forward with the default rope,
    modeling_qwen3.py:401-412, before its cast to the model dtype)."""
    inv = theta ** (-np.arange(0, D, 2, dtype=np.float64) / D)
    ang = np.asarray(positions, dtype=np.float64)[:, None] * inv[None, :]
    emb = np.concatenate([ang, ang], axis=-1)
    return np.cos(emb), np.sin(emb)
