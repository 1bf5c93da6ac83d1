"""CPU oracle for the gated LoRA linear layer (numpy, float64).

TEST INFRASTRUCTURE. Only ``tests/`` and the ``cpu_baseline`` leg of
``bench.py`` import this module, and only as the checker. The product package
never imports it and has no CPU fallback.

What it restates (``mtp_glora/models/layers/gated_lora.py`` of the reference
checkout):

* ``forward`` - GatedLoRALinear.forward (:51-53) for a bias-free base layer:
      h = dropout(x) = x * keep / (1 - p),
      y = x W^T + s * ((h A^T) B^T) * gate[:, None],
  s = alpha / rank (alpha / sqrt(rank) with rs-LoRA, :35).
* ``backward`` - the autograd gradients of that map with the base weight
  frozen (only ``lora_`` parameters train, :56-58): given dY,
      d_lora = s * gate[:, None] * dY,   dB = d_lora^T (h A^T),
      d_a = d_lora B,   dA = d_a^T h,   dX = dY W + (d_a A) * keep / (1 - p).
* ``keep_mask`` - the dropout keep bits of the HIP kernels (their own
  design: the reference draws its mask from torch's generator): element i of
  the flattened [S, K] input belongs to pair j = i // 2, whose bits are
  fmix32(fmix32(lo(j) ^ lo(seed)) ^ hi(j) ^ hi(seed)) (fmix32: MurmurHash3's
  32-bit finaliser); the low 16 bits decide the even element, the high 16 the
  odd one, kept when >= round(65536 p).

Parity pins live in ``tests/test_oracle_gated_lora.py``.
"""
from __future__ import annotations

import numpy as np

_M32 = np.uint64(0xFFFFFFFF)


def _fmix32(h: np.ndarray) -> np.ndarray:
    h = h.astype(np.uint64) & _M32
    h ^= h >> np.uint64(16)
    h = (h * np.uint64(0x85EBCA6B)) & _M32
    h ^= h >> np.uint64(13)
    h = (h * np.uint64(0xC2B2AE35)) & _M32
    h ^= h >> np.uint64(16)
    return h


def drop_threshold(p: float) -> int:
    return int(round(p * 65536.0))


def keep_mask(seed: int, S: int, K: int, p: float) -> np.ndarray:
    """Boolean [S, K] keep mask (all True for p = 0)."""
    thr = drop_threshold(p)
    if thr == 0:
        return np.ones((S, K), dtype=bool)
    pair = np.arange(S * K // 2, dtype=np.uint64)
    s_lo, s_hi = np.uint64(seed & 0xFFFFFFFF), np.uint64((seed >> 32) & 0xFFFFFFFF)
    bits = _fmix32(_fmix32((pair & _M32) ^ s_lo) ^ (pair >> np.uint64(32)) ^ s_hi)
    keep = np.empty(S * K, dtype=bool)
    keep[0::2] = (bits & np.uint64(0xFFFF)) >= np.uint64(thr)
    keep[1::2] = (bits >> np.uint64(16)) >= np.uint64(thr)
    return keep.reshape(S, K)


def forward(x, W, A, B, gate, scaling: float, keep=None, p: float = 0.0):
    """y [S, N] in float64; gate [S] or None; keep [S, K] bool or None."""
    x = np.asarray(x, dtype=np.float64)
    h = x if keep is None else x * keep / (1.0 - p)
    g = np.ones(x.shape[0]) if gate is None else np.asarray(gate, dtype=np.float64)
    lora = (h @ np.asarray(A, np.float64).T) @ np.asarray(B, np.float64).T
    return x @ np.asarray(W, np.float64).T + scaling * lora * g[:, None]


def backward(dy, x, W, A, B, gate, scaling: float, keep=None, p: float = 0.0):
    """(dX, dA, dB) in float64."""
    dy = np.asarray(dy, np.float64)
    x = np.asarray(x, np.float64)
    A = np.asarray(A, np.float64)
    B = np.asarray(B, np.float64)
    h = x if keep is None else x * keep / (1.0 - p)
    g = np.ones(x.shape[0]) if gate is None else np.asarray(gate, dtype=np.float64)
    d_lora = scaling * g[:, None] * dy
    dB = d_lora.T @ (h @ A.T)
    d_a = d_lora @ B
    dA = d_a.T @ h
    dh = d_a @ A
    dx = dy @ np.asarray(W, np.float64) + (dh if keep is None else dh * keep / (1.0 - p))
    return dx, dA, dB
