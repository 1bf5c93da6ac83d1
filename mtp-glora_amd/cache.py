"""Streaming KV cache: preallocated per-layer K/V buffers behind the
transformers ``Cache`` API the reference's adapters and manager call.

Layout in HBM: per layer one ``[Hkv, capacity, D]`` buffer for K and one for V
(model dtype, row-major, a head's rows contiguous), all allocated once, before
the first chunk. The cached prefix of P regular tokens occupies rows ``[0, P)``
of every head. Each layer's buffers are separate allocations so that autograd's
version counters (bumped on every raw write) are per layer.

* ``update(k, v, layer)`` (``[tf]cache_utils.py:1349-1381``; called at
  mtp_glora/models/modeling_qwen3.py:281-284, modeling_llama.py:314-317)
  copies the chunk's S rows to ``[P, P+S)`` with one HIP kernel (O(S), not the
  O(P+S) ``torch.cat`` of ``DynamicLayer.update``, :144-146) and returns
  ``[1, Hkv, P+S, D]`` views equal to ``cat(prefix, new)``. The views carry the
  gradient back to the chunk's K/V (the prefix is detached, as in
  collator.py:279-280).
* ``commit_regular(idx, R)`` is the in-place form of collator.py:270-287: the
  chunk's regular rows are gathered into ``[P, P+R)`` and P grows by R.
* Legacy access used by the reference manager: ``cache[i]`` -> ``(K, V)``,
  iteration over 2-tuples, ``to_legacy_cache()``, ``from_legacy_cache()``.
"""
from __future__ import annotations

import os

import torch

from . import ops

DEFAULT_CAPACITY = int(os.environ.get("MGA_CACHE_CAPACITY", 131072 + 16384))


class _StageKV(torch.autograd.Function):
    """Identity on the staged buffer view whose backward routes the rows of the
    chunk (the last S) to the chunk's K or V and drops the detached prefix."""

    @staticmethod
    def forward(ctx, cur, full_view):
        ctx.P = full_view.shape[2] - cur.shape[2]
        return full_view.view_as(full_view)

    @staticmethod
    def backward(ctx, g):
        return g[:, :, ctx.P:], None


class StreamingKVCache:
    """Preallocated streaming KV cache (batch size 1)."""

    is_compileable = False

    def __init__(self, capacity: int = DEFAULT_CAPACITY, num_layers: int | None = None,
                 num_kv_heads: int | None = None, head_dim: int | None = None,
                 dtype: torch.dtype | None = None, device=None):
        if capacity <= 0:
            raise ValueError("capacity must be positive")
        self.capacity = int(capacity)
        self.num_layers = num_layers
        self._dims = None            # (Hkv, D, dtype, device)
        self._k = None               # per layer [Hkv, cap, D]
        self._v = None
        self.prefix_len = 0          # P: committed regular rows (all layers)
        self._len: list[int] = []    # rows visible per layer (P, or P + S after update)
        self._staged: list = []      # per layer: (k_cur, v_cur) of the last update
        if None not in (num_layers, num_kv_heads, head_dim, dtype, device):
            self._allocate(num_layers, num_kv_heads, head_dim, dtype, torch.device(device))

    # -- allocation ---------------------------------------------------------
    def _allocate(self, layers, hkv, d, dtype, device):
        if device.type != "cuda":
            raise RuntimeError(f"StreamingKVCache lives in GPU memory; got device {device}")
        ops.dtype_code(dtype)
        self.num_layers = layers
        self._dims = (hkv, d, dtype, device)
        self._k = [torch.empty(hkv, self.capacity, d, dtype=dtype, device=device) for _ in range(layers)]
        self._v = [torch.empty(hkv, self.capacity, d, dtype=dtype, device=device) for _ in range(layers)]
        self._len = [self.prefix_len] * layers
        self._staged = [None] * layers

    def _ensure(self, layer_idx: int, k: torch.Tensor):
        if self._k is None:
            if self.num_layers is None:
                raise RuntimeError("StreamingKVCache needs num_layers before the first update")
            self._allocate(self.num_layers, k.shape[1], k.shape[3], k.dtype, k.device)
        hkv, d, dtype, device = self._dims
        if k.dim() != 4 or k.shape[0] != 1:
            raise ValueError(f"expected [1, Hkv, S, D] key/value states, got {tuple(k.shape)}")
        if (k.shape[1], k.shape[3]) != (hkv, d) or k.dtype != dtype or k.device != device:
            raise ValueError(f"key/value states {tuple(k.shape)} {k.dtype} {k.device} do not match "
                             f"the cache ([1, {hkv}, S, {d}] {dtype} {device})")
        if not 0 <= layer_idx < self.num_layers:
            raise IndexError(f"layer_idx {layer_idx} outside [0, {self.num_layers})")

    @property
    def is_sliding(self):
        return [False] * (self.num_layers or 0)

    def key_buffer(self, layer_idx: int) -> torch.Tensor:
        return self._k[layer_idx]

    def value_buffer(self, layer_idx: int) -> torch.Tensor:
        return self._v[layer_idx]

    def _bump(self, layer_idx: int):
        # Writes through raw pointers: tell autograd the buffer changed so a
        # view saved for a backward that runs later fails loudly.
        torch.autograd.graph.increment_version(self._k[layer_idx])
        torch.autograd.graph.increment_version(self._v[layer_idx])

    def stage_rows(self, layer_idx: int, like: torch.Tensor):
        """``[1, Hkv, S, D]`` views of rows ``[P, P + S)`` of the layer's K and V
        buffers (S and the dims from ``like``), for a kernel that writes the
        chunk's K/V there itself; ``update`` given these views copies nothing."""
        self._ensure(layer_idx, like)
        P, S = self.prefix_len, like.shape[2]
        if P + S > self.capacity:
            raise RuntimeError(f"StreamingKVCache capacity {self.capacity} exceeded ({P} + {S} rows)")
        return self._k[layer_idx][None, :, P:P + S], self._v[layer_idx][None, :, P:P + S]

    @staticmethod
    def _in_place(t: torch.Tensor, buf: torch.Tensor, P: int) -> bool:
        # a full buffer has no row P: the append then raises its capacity error
        if P >= buf.shape[1]:
            return False
        return (t.data_ptr() == buf[:, P].data_ptr() and t.stride()[1:] == buf.stride()
                and t.shape[1] == buf.shape[0])

    # -- Cache API ------------------------------------------------------------
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs=None):
        """Stage the chunk's K/V after the cached prefix and return the full
        ``[1, Hkv, P + S, D]`` K and V. K/V that already are the views of
        ``stage_rows`` are not copied."""
        self._ensure(layer_idx, key_states)
        if value_states.shape != key_states.shape:
            raise ValueError("key and value states must have the same shape")
        P = self.prefix_len
        S = key_states.shape[2]
        kb, vb = self._k[layer_idx], self._v[layer_idx]
        in_place = self._in_place(key_states, kb, P), self._in_place(value_states, vb, P)
        if in_place == (True, True):
            restage = getattr(key_states, "_mga_restage", None)
            if restage is None:
                raise ValueError("key / value states sit in the cache rows without a way to re-stage their "
                                 "regular rows (stage them with rope.qk_norm_rope_stage)")
            self._staged[layer_idx] = restage
        elif any(in_place):
            raise ValueError("only one of key / value states sits in the cache rows")
        else:
            ops.kv_append(key_states, value_states, kb, vb, dst_offset=P)   # raises on capacity
            self._staged[layer_idx] = (key_states, value_states)
        self._bump(layer_idx)
        self._len[layer_idx] = P + S
        kf = kb[None, :, :P + S]
        vf = vb[None, :, :P + S]
        if key_states.requires_grad:
            kf = _StageKV.apply(key_states, kf)
        if value_states.requires_grad:
            vf = _StageKV.apply(value_states, vf)
        # read by the HIP attention to send dK/dV straight to the chunk's K/V
        kf._mga_stage = (key_states, P)
        vf._mga_stage = (value_states, P)
        return kf, vf

    def get_seq_length(self, layer_idx: int = 0) -> int:
        if not self._len:
            return self.prefix_len
        return self._len[layer_idx]

    def get_max_cache_shape(self, layer_idx: int = 0) -> int:
        return self.capacity

    def get_mask_sizes(self, query_length: int, layer_idx: int = 0):
        return self.get_seq_length(layer_idx) + query_length, 0

    def get_query_offset(self, layer_idx: int = 0) -> int:
        return self.get_seq_length(layer_idx)

    def __len__(self) -> int:
        return self.num_layers or 0

    def __getitem__(self, layer_idx: int):
        n = self._len[layer_idx]
        return self._k[layer_idx][None, :, :n], self._v[layer_idx][None, :, :n]

    def __iter__(self):
        for i in range(len(self)):
            yield self[i]

    def to_legacy_cache(self):
        return tuple(self[i] for i in range(len(self)))

    # -- streaming ------------------------------------------------------------
    def reset(self) -> None:
        """Forget every cached token (buffers stay allocated)."""
        self.prefix_len = 0
        self._len = [0] * (self.num_layers or 0) if self._k is not None else []
        self._staged = [None] * (self.num_layers or 0) if self._k is not None else []

    def commit_regular(self, idx: torch.Tensor, n_regular: int) -> None:
        """Append the staged chunk's regular tokens (``idx[:n_regular]``, chunk
        positions ascending) to the prefix of every layer, then P += n_regular."""
        if self._k is None:
            raise RuntimeError("commit_regular before any update")
        P = self.prefix_len
        for layer in range(self.num_layers):
            st = self._staged[layer]
            if st is None:
                raise RuntimeError(f"layer {layer} has no staged chunk to commit")
            if callable(st):   # staged in place: re-staged from the projections
                st(idx, n_regular, self._k[layer], self._v[layer], P)
            else:
                k_cur, v_cur = st
                ops.kv_append(k_cur.detach(), v_cur.detach(), self._k[layer], self._v[layer],
                              dst_offset=P, idx=idx, n_rows=n_regular)
            self._bump(layer)
        self.prefix_len = P + n_regular
        self._len = [self.prefix_len] * self.num_layers
        self._staged = [None] * self.num_layers

    def crop(self, max_length: int) -> None:
        """Keep only the first ``max_length`` cached prefix tokens (negative:
        drop that many from the end), as transformers' ``Cache.crop``; a
        staged chunk is discarded. The buffers stay allocated."""
        if max_length < 0:
            max_length = self.prefix_len + max_length
        if max_length < 0:
            raise ValueError("crop would leave a negative length")
        self.prefix_len = min(self.prefix_len, int(max_length))
        n = self.num_layers or 0
        self._len = [self.prefix_len] * n if self._k is not None else []
        self._staged = [None] * n if self._k is not None else []

    def append_prefix(self, keys, values) -> None:
        """Append already-filtered prefix rows (``[1, Hkv, n, D]`` per layer) for
        every layer, e.g. when taking over a legacy cache."""
        n = keys[0].shape[2]
        for layer, (k, v) in enumerate(zip(keys, values)):
            self._ensure(layer, k)
            ops.kv_append(k.detach(), v.detach(), self._k[layer], self._v[layer],
                          dst_offset=self.prefix_len)
            self._bump(layer)
        self.prefix_len += n
        self._len = [self.prefix_len] * self.num_layers
        self._staged = [None] * self.num_layers

    @classmethod
    def from_legacy_cache(cls, past_key_values, capacity: int = DEFAULT_CAPACITY) -> "StreamingKVCache":
        """Build a cache from ``((K, V), ...)`` tuples of ``[1, Hkv, P, D]``
        (the call of collator.py:287)."""
        keys = [kv[0] for kv in past_key_values]
        values = [kv[1] for kv in past_key_values]
        c = cls(capacity=capacity, num_layers=len(keys))
        c.append_prefix(keys, values)
        return c
