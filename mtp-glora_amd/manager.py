"""``StreamingKVCacheManager`` with the reference's three public methods
(mtp_glora/data_utils/collator.py:178-287), driven by the trainer's chunk loop
(mtp_glora/trainer/trainer.py:95-136):

* ``reset_cache()``                              (collator.py:188-190)
* ``prepare_data_with_kv_cache(chunk)``          (collator.py:193-217)
* ``extract_regular_kv_cache_for_next_chunk(chunk, past_key_values)`` (collator.py:220-287)

The BlockMask is built on the GPU from the unclamped gate (pad = -1), and only
then is the gate clamped and unsqueezed for the LoRA gating (collator.py:208-215).
The carry-over keeps the chunk's regular-token K/V in the preallocated cache
in place instead of re-concatenating the prefix.

The reference's ``regular_token_mask.nonzero()`` waits for everything queued
before it, i.e. the whole forward and backward of the chunk. Here the
regular-token index is built when the chunk is prepared, before any of the
chunk's attention work is queued, and its count is copied to pinned host
memory behind an event; the carry-over waits on that event only, so the host
goes on queueing the next chunk's kernels while the backward still runs. The
position sanity check (collator.py:251-258) is queued at the same point: a
mismatch flag formed on the device travels with the count, and the carry-over
prints the reference's message from it (reading the positions back only when
the flag is set).
"""
from __future__ import annotations

import warnings

import torch

from . import ops
from .block_mask import build_mtp_block_mask
from .cache import DEFAULT_CAPACITY, StreamingKVCache


class StreamingKVCacheManager:
    """KV cache manager for streaming/sequential chunk processing."""

    def __init__(self, capacity: int = DEFAULT_CAPACITY, sanity_check: bool = True):
        self.past_seen_tokens = 0
        self.capacity = int(capacity)
        self.sanity_check = sanity_check
        self.cache: StreamingKVCache | None = None
        self._host: torch.Tensor | None = None   # pinned [count, position mismatch]
        self._pending = None   # (mask tensor, its version, idx, event, position check or None)

    def reset_cache(self) -> None:
        """Reset KV cache for a new sequence (buffers stay allocated)."""
        self.past_seen_tokens = 0
        if self.cache is not None:
            self.cache.reset()

    def new_cache(self, num_layers: int) -> StreamingKVCache:
        """The manager's cache, reset, for a model with ``num_layers`` layers;
        pass it as ``past_key_values`` of the first chunk to skip the model's
        own DynamicCache."""
        if self.cache is None or self.cache.num_layers != num_layers:
            self.cache = StreamingKVCache(capacity=self.capacity, num_layers=num_layers)
        self.cache.reset()
        self.past_seen_tokens = 0
        return self.cache

    def prepare_data_with_kv_cache(self, chunk_data: dict) -> dict:
        """Attach the chunk's MTP BlockMask (against ``past_seen_tokens`` cached
        tokens) as ``attention_mask``, then clamp the gate to >= 0 and unsqueeze
        it for the LoRA gating."""
        gate = chunk_data["gate_mask"]
        if gate.shape[0] > 1:
            warnings.warn("`prepare_data_with_kv_cache` expects batch size to be 1, "
                          f"but got batch size: {gate.shape[0]}")
        bm = build_mtp_block_mask(gate[:1], self.past_seen_tokens)
        chunk_data["attention_mask"] = bm.to(chunk_data["input_ids"].device)
        chunk_data["gate_mask"] = torch.clamp(chunk_data["gate_mask"], min=0)[:, :, None]
        self._pending = None
        reg = chunk_data.get("regular_token_mask")
        if isinstance(reg, torch.Tensor) and reg.is_cuda:
            idx, cnt = ops.regular_index(reg[0])
            if self._host is None:
                self._host = torch.empty(2, dtype=torch.int32, pin_memory=True)
            pos = chunk_data.get("position_ids") if self.sanity_check else None
            check = None
            if isinstance(pos, torch.Tensor) and pos.is_cuda and pos.dim() == 2 and pos.shape[1] == idx.numel():
                check = (pos, pos._version, self.past_seen_tokens)
                src = torch.cat([cnt, self._position_mismatch(pos[0], idx, cnt, self.past_seen_tokens)])
            else:
                src = cnt
            self._host[:src.numel()].copy_(src, non_blocking=True)
            event = torch.cuda.Event()
            event.record()
            self._pending = (reg, reg._version, idx, event, check)
        return chunk_data

    @staticmethod
    def _position_mismatch(pos: torch.Tensor, idx: torch.Tensor, cnt: torch.Tensor, P: int) -> torch.Tensor:
        """[1] int32 on the device: 1 when the positions of the regular rows are
        not P, P + 1, ..., P + R - 1 (the check of collator.py:251-258), queued
        without a host wait."""
        i = torch.arange(idx.numel(), device=idx.device)
        valid = i < cnt
        got = pos[torch.where(valid, idx.long(), 0)]
        return ((got != i + P) & valid).any().to(torch.int32).reshape(1)

    def _regular_rows(self, reg: torch.Tensor, pos):
        """(idx, R, mismatch) of the chunk's regular tokens: from the index
        built by ``prepare_data_with_kv_cache`` when it was built for this same,
        unmodified mask (waiting on its event only), else built now with one
        stream sync, as the reference's nonzero(). ``mismatch`` is the queued
        position check's flag when it was formed for these same, unmodified
        positions and prefix length, else None."""
        pend, self._pending = self._pending, None
        if pend is not None and pend[0] is reg and pend[1] == reg._version:
            _, _, idx, event, check = pend
            event.synchronize()
            mismatch = None
            if check is not None and check[0] is pos and check[1] == pos._version \
                    and check[2] == self.past_seen_tokens:
                mismatch = bool(self._host[1])
            return idx, int(self._host[0]), mismatch
        idx, cnt = ops.regular_index(reg[0])
        return idx, int(cnt.item()), None

    def extract_regular_kv_cache_for_next_chunk(self, chunk_data: dict, past_key_values=None):
        """Keep only the chunk's regular-token K/V (detached) behind the cached
        prefix and advance ``past_seen_tokens``. Returns the cache to pass as
        ``past_key_values`` of the next chunk."""
        bsz = chunk_data["input_ids"].shape[0]
        if bsz > 1:
            warnings.warn("`extract_regular_kv_cache_for_next_chunk` expects batch size to be 1, "
                          f"but got batch size: {bsz}")
        if past_key_values is None:
            return None
        pos_ids = chunk_data.get("position_ids")
        idx, R, mismatch = self._regular_rows(chunk_data["regular_token_mask"], pos_ids)

        if self.sanity_check and pos_ids is not None:
            pos = pos_ids[0]
            got = expected = None
            if mismatch is None:   # no queued flag for these positions: the reference's comparison (waits)
                got = pos[idx[:R].long()]
                expected = torch.arange(self.past_seen_tokens, self.past_seen_tokens + R, device=pos.device)
                mismatch = not torch.equal(got, expected.to(got.dtype))
            if mismatch:
                if got is None:
                    got = pos[idx[:R].long()]
                    expected = torch.arange(self.past_seen_tokens, self.past_seen_tokens + R, device=pos.device)
                print("extract_regular_kv_cache_for_next_chunk: Sanity check failed. Position IDs mismatch. "
                      f"Expected: {expected}, Actual: {got}")
                print(f"self.past_seen_tokens: {self.past_seen_tokens}, num_new_regular_tokens: {R}")

        if isinstance(past_key_values, StreamingKVCache):
            cache = past_key_values
            if cache.prefix_len != self.past_seen_tokens:
                raise RuntimeError(f"cache holds {cache.prefix_len} prefix tokens but the manager "
                                   f"has seen {self.past_seen_tokens}")
            cache.commit_regular(idx, R)
        else:
            cache = self._take_over(past_key_values, chunk_data["input_ids"].shape[1], idx, R)
        self.cache = cache
        self.past_seen_tokens += R
        return cache

    def _take_over(self, past_key_values, chunk_len: int, idx: torch.Tensor, R: int) -> StreamingKVCache:
        """Move a transformers DynamicCache / legacy tuple (the model builds one
        when the first chunk gets ``past_key_values=None``) into the streaming
        cache: its prefix rows, then the chunk's regular rows."""
        layers = [(kv[0], kv[1]) for kv in past_key_values]
        n = len(layers)
        if self.cache is None or self.cache.num_layers != n:
            self.cache = StreamingKVCache(capacity=self.capacity, num_layers=n)
        cache = self.cache
        cache.reset()
        P = self.past_seen_tokens
        for li, (k, v) in enumerate(layers):
            if k.shape[2] != P + chunk_len:
                raise RuntimeError(f"layer {li} holds {k.shape[2]} tokens, expected {P} + {chunk_len}")
        if P > 0:
            cache.append_prefix([k[:, :, :P] for k, _ in layers], [v[:, :, :P] for _, v in layers])
        for li, (k, v) in enumerate(layers):
            cache._ensure(li, k)
            cache._staged[li] = (k[:, :, P:], v[:, :, P:])
        cache.commit_regular(idx, R)
        return cache
