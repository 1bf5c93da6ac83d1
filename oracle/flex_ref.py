"""The reference's own operator path, restated on torch's CPU kernels.

TEST INFRASTRUCTURE. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it. It never runs on the product path.

* ``mtp_mask_mod``: the ``mask_mod`` of ``mtp_glora/data_utils/collator.py:311-355``,
  composed with torch's own ``and_masks`` / ``or_masks`` exactly as there.
* ``reference_block_mask``: ``create_block_mask(mask_mod, B=None, H=None,
  Q_LEN=S, KV_LEN=P+S)`` (collator.py:357-363) on the CPU.
* ``reference_attention``: ``flex_attention`` eager (the dense math path),
  GQA enabled, fwd with LSE, autograd bwd -- the arithmetic of
  ``[tf]integrations/flex_attention.py:262-368`` on CPU.
* ``reference_cache_ops``: ``DynamicLayer.update``'s ``torch.cat``
  (``[tf]cache_utils.py:144-146``) and the regular-token gather + cat of
  collator.py:273-282.
"""
from __future__ import annotations

import torch
from torch.nn.attention.flex_attention import (
    and_masks, create_block_mask, flex_attention, or_masks)


def mtp_mask_mod(gate: torch.Tensor, P: int):
    """collator.py:311-355; ``gate`` is the chunk's ``[1, S]`` int64 gate mask."""
    bsz = gate.shape[0]
    if P > 0:
        g = torch.cat([torch.zeros(bsz, P, dtype=gate.dtype, device=gate.device), gate], dim=1)
    else:
        g = gate
    npx = (g == 0).long().cumsum(dim=1)

    def is_causal(b, h, q_idx, kv_idx): return q_idx + P >= kv_idx
    def is_query_not_pad(b, h, q_idx, kv_idx): return g[b, q_idx + P] != -1
    def is_key_not_pad(b, h, q_idx, kv_idx): return g[b, kv_idx] != -1
    def is_query_x(b, h, q_idx, kv_idx): return g[b, q_idx + P] == 0
    def is_query_m(b, h, q_idx, kv_idx): return g[b, q_idx + P] == 1
    def is_key_x(b, h, q_idx, kv_idx): return g[b, kv_idx] == 0
    def is_key_m(b, h, q_idx, kv_idx): return g[b, kv_idx] == 1
    def is_same_m_block(b, h, q_idx, kv_idx): return npx[b, q_idx + P] == npx[b, kv_idx]

    x_rule = and_masks(is_query_x, is_key_x)
    m_rule = and_masks(is_query_m, or_masks(is_key_x, and_masks(is_key_m, is_same_m_block)))
    return and_masks(is_causal, is_query_not_pad, is_key_not_pad, or_masks(x_rule, m_rule))


def reference_block_mask(gate: torch.Tensor, P: int, device="cpu"):
    S = gate.shape[1]
    return create_block_mask(mtp_mask_mod(gate.to(device), P), B=None, H=None,
                             Q_LEN=S, KV_LEN=P + S, device=device)


def block_mask_tensors(bm) -> dict:
    """The eight int32 tensors of a BlockMask as numpy arrays."""
    names = ["kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
             "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices"]
    return {n: getattr(bm, n).cpu().numpy() for n in names}


def reference_attention(q, k, v, block_mask, scale, do=None):
    """flex_attention eager on CPU. q [1,Hq,S,D], k/v [1,Hkv,L,D].
    Returns (o [1,Hq,S,D], lse [1,Hq,S]) and, with ``do`` ([1,Hq,S,D]),
    also (dq, dk, dv) from autograd."""
    q = q.detach().clone().requires_grad_(do is not None)
    k = k.detach().clone().requires_grad_(do is not None)
    v = v.detach().clone().requires_grad_(do is not None)
    enable_gqa = q.shape[1] != k.shape[1]
    o, aux = flex_attention(q, k, v, block_mask=block_mask, scale=scale,
                            enable_gqa=enable_gqa, return_aux=_aux_request())
    lse = aux.lse if hasattr(aux, "lse") else aux
    if do is None:
        return o.detach(), lse.detach()
    o.backward(do)
    return o.detach(), lse.detach(), q.grad, k.grad, v.grad


def _aux_request():
    from torch.nn.attention.flex_attention import AuxRequest
    return AuxRequest(lse=True)


def reference_cache_ops(prefix_k, cur_k, regular_mask):
    """One layer of the reference's cache traffic for K (V is identical):
    update's cat (cache_utils.py:144-146), then collator.py:273-280's split,
    regular gather, cat and detach. Tensors are [1, H, seq, D]."""
    P = prefix_k.shape[2]
    S = cur_k.shape[2]
    full = torch.cat([prefix_k, cur_k], dim=-2)
    idx = regular_mask[0].nonzero(as_tuple=True)[0]
    past, cur = full.split([P, S], dim=2)
    return full, torch.cat([past, cur[:, :, idx, :]], dim=2).detach()
