"""MTP block-masked attention as a transformers attention function.

``mtp_attention_forward`` has the signature and return convention of
``flex_attention_forward`` ([tf]integrations/flex_attention.py:262-368): it is
looked up through ``ALL_ATTENTION_FUNCTIONS[config._attn_implementation]`` by
the adapters (mtp_glora/models/modeling_qwen3.py:286-300,
modeling_llama.py:320-332) and returns ``(attn_output [B, S, Hq, D]
contiguous, lse)``. ``register()`` installs it under ``"mtp_hip"`` and, with
``replace_flex=True``, under ``"flex_attention"`` so the reference's
``attn_implementation="flex_attention"`` (trainer/utils.py:68) picks it up
unchanged.

Gradients: dQ for every visited tile; dK/dV only for keys that carry
gradient. When the keys come from ``StreamingKVCache.update`` the gradient
goes straight to the chunk's K/V (the cached prefix is detached,
collator.py:279-280) and the prefix costs no dK/dV work; for a plain key tensor
every key gets its gradient.
"""
from __future__ import annotations

import torch

from . import _lib, ops
from .block_mask import MTPBlockMask


class _MTPAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k_grad, v_grad, k_full, v_full, mask: MTPBlockMask, scale: float,
                grad_start: int):
        bm = mask.kernel_tensors()
        code = mask.mtp_code
        P = mask.prefix_len
        o, lse = ops.attn_fwd(q, k_full, v_full, code, bm, P, scale)
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(q, k_full, v_full, o, lse)
        ctx.mask = mask
        ctx.scale = scale
        ctx.grad_start = grad_start
        return o, lse

    @staticmethod
    def backward(ctx, do, dlse):
        if dlse is not None:
            raise NotImplementedError("gradient through the attention LSE is not supported "
                                      "(the decoder layers discard it)")
        q, k_full, v_full, o, lse = ctx.saved_tensors
        if do is None:
            return (None,) * 8
        mask = ctx.mask
        L = k_full.shape[2]
        need_kv = ctx.needs_input_grad[1] or ctx.needs_input_grad[2]
        grad_start = ctx.grad_start if need_kv else L
        passes = _lib.BWD_DQ | (_lib.BWD_DKDV if need_kv else 0)
        dq, dk, dv = ops.attn_bwd(q, k_full, v_full, o, lse, do, mask.mtp_code,
                                  mask.kernel_tensors(), mask.prefix_len, ctx.scale, grad_start,
                                  passes=passes)
        dq = dq if ctx.needs_input_grad[0] else None
        dk = dk if ctx.needs_input_grad[1] else None
        dv = dv if ctx.needs_input_grad[2] else None
        return dq, dk, dv, None, None, None, None, None


def _grad_source(t: torch.Tensor):
    """(tensor that receives the gradient, first key row that has one)."""
    st = getattr(t, "_mga_stage", None)
    if st is not None:
        cur, P = st
        if t.shape[2] - cur.shape[2] != P:
            raise RuntimeError("staged key/value views do not match their chunk")
        return cur, P
    return t, 0


def mtp_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                  mask: MTPBlockMask, scale: float | None = None):
    """Core op: query [1, Hq, S, D], key/value [1, Hkv, P+S, D] -> (o [1, S, Hq, D], lse [1, Hq, S])."""
    if not isinstance(mask, MTPBlockMask):
        raise TypeError("mtp_attention needs the MTPBlockMask built by StreamingKVCacheManager "
                        f"(got {type(mask).__name__})")
    S = query.shape[2]
    L = key.shape[2]
    if mask.seq_lengths != (S, L) or mask.prefix_len + S != L:
        raise ValueError(f"mask covers {mask.seq_lengths} with prefix {mask.prefix_len}, "
                         f"but query/key lengths are ({S}, {L})")
    if scale is None:
        scale = query.shape[-1] ** -0.5
    k_src, k0 = _grad_source(key)
    v_src, v0 = _grad_source(value)
    if k0 != v0:
        raise RuntimeError("key and value have different gradient starts")
    # the kernels read K/V from the full views; gradients go to k_src / v_src
    return _MTPAttention.apply(query, k_src, v_src, key.detach(), value.detach(), mask,
                               float(scale), k0)


def mtp_attention_forward(module: torch.nn.Module, query: torch.Tensor, key: torch.Tensor,
                          value: torch.Tensor, attention_mask, scaling: float | None = None,
                          softcap: float | None = None, s_aux=None, position_bias=None,
                          **kwargs):
    """Drop-in for ``flex_attention_forward`` with an MTP BlockMask."""
    if kwargs.get("dropout", 0.0) > 0:
        raise ValueError("mtp_attention does not support dropout "
                         "(as flex_attention_forward, [tf]integrations/flex_attention.py:274-278)")
    if softcap is not None or s_aux is not None or position_bias is not None:
        raise NotImplementedError("mtp_attention supports neither softcap, attention sinks nor position bias")
    if kwargs.get("sliding_window") is not None:
        raise NotImplementedError("mtp_attention does not implement sliding-window layers")
    if query.shape[0] != 1:
        raise ValueError(f"mtp_attention assumes batch size 1 (got {query.shape[0]})")
    o, lse = mtp_attention(query, key, value, attention_mask, scaling)
    return o, lse.to(value.dtype)


def register(name: str = "mtp_hip", replace_flex: bool = False) -> None:
    """Register with transformers' ``AttentionInterface``."""
    from transformers import AttentionInterface
    AttentionInterface.register(name, mtp_attention_forward)
    if replace_flex:
        AttentionInterface.register("flex_attention", mtp_attention_forward)
