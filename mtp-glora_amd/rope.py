"""Qwen3 query / key normalisation + rotary embedding, fused, on the HIP
kernels of libmtp_glora_amd.so.

The reference's Qwen3Attention.forward (mtp_glora/models/modeling_qwen3.py:
254-305) runs, per layer and chunk,

    q = q_norm(q_proj(x).view(B, S, Hq, D)).transpose(1, 2)      # :274
    k = k_norm(k_proj(x).view(B, S, Hkv, D)).transpose(1, 2)     # :275
    q, k = apply_rotary_pos_emb(q, k, cos, sin)                  # :278-279

as about a dozen torch ops that each read and write the whole of q or k.
``qk_norm_rope`` does the same in one kernel launch that reads q, k, the norm
weights and the cos / sin rows once and writes the two embeddings once, with
the reference's rounding after every op. It returns the embeddings as
[B, H, S, D] views of [B, S, H, D] storage, which is the layout the reference's
elementwise ops produce from their transposed inputs.

Backward: dq and dk in fp32 inside the kernel (the norm weights, cos and sin
get no gradient; in the reference they are frozen base-model tensors, and
asking for a norm-weight gradient here is an error).

``qwen3_attention_forward`` is Qwen3Attention.forward with those lines replaced
by ``qk_norm_rope``; everything else (projections, the cache update, the
attention function looked up in ALL_ATTENTION_FUNCTIONS, o_proj) is called as
the reference calls it. With a ``StreamingKVCache`` the same launch also
writes the post-RoPE keys and the values into the cache rows the update would
fill (``qk_norm_rope_stage``), so the update copies nothing; committing the
chunk's regular rows then re-runs the kernel on the projections' regular rows
(the staged rows are the gather's destination, so they cannot be its source).
"""
from __future__ import annotations

import sys

import torch

from . import _lib
from .cache import StreamingKVCache
from .ops import _dev, _stream, dtype_code


def _heads(name: str, t: torch.Tensor):
    """A [S, H, D] view with unit stride on D of a [1, S, H, D] operand."""
    _dev(name, t)
    if t.dim() != 4 or t.shape[0] != 1:
        raise ValueError(f"{name}: expected [1, S, heads, head_dim], got {tuple(t.shape)}")
    t3 = t[0]
    if t3.stride(2) != 1:
        t3 = t3.contiguous()
    return t3


def _table(name: str, t: torch.Tensor, S: int, D: int):
    """A [S, D] view with unit stride on D of cos / sin ([1, S, D] or [S, D])."""
    _dev(name, t)
    if t.dim() == 3:
        if t.shape[0] != 1:
            raise ValueError(f"{name}: batch size must be 1 (got {t.shape[0]})")
        t = t[0]
    if tuple(t.shape) != (S, D):
        raise ValueError(f"{name}: expected [{S}, {D}], got {tuple(t.shape)}")
    if t.stride(1) != 1:
        t = t.contiguous()
    return t


def _check_dtypes(q, *others):
    for name, t in others:
        if t.dtype != q.dtype:
            raise TypeError(f"{name} dtype {t.dtype} != query dtype {q.dtype}")


def norm_rope_forward(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
                      cos: torch.Tensor, sin: torch.Tensor, eps: float):
    """q [1, S, Hq, D], k [1, S, Hkv, D] -> (q_embed [1, S, Hq, D], k_embed
    [1, S, Hkv, D], rstd [S, Hq + Hkv] fp32)."""
    q3, k3 = _heads("query_states", q), _heads("key_states", k)
    S, Hq, D = q3.shape
    if k3.shape[0] != S or k3.shape[2] != D:
        raise ValueError(f"key_states {tuple(k.shape)} does not match query_states {tuple(q.shape)}")
    Hkv = k3.shape[1]
    for name, w in (("q_weight", q_weight), ("k_weight", k_weight)):
        _dev(name, w)
        if w.dim() != 1 or w.shape[0] != D or w.stride(0) != 1:
            raise ValueError(f"{name}: expected a contiguous [{D}] weight, got {tuple(w.shape)}")
    c, s = _table("cos", cos, S, D), _table("sin", sin, S, D)
    if c.stride(0) != s.stride(0):
        c, s = c.contiguous(), s.contiguous()
    _check_dtypes(q3, ("key_states", k3), ("q_weight", q_weight), ("k_weight", k_weight), ("cos", c), ("sin", s))
    dev = q3.device
    qo = torch.empty(1, S, Hq, D, device=dev, dtype=q3.dtype)
    ko = torch.empty(1, S, Hkv, D, device=dev, dtype=q3.dtype)
    rstd = torch.empty(S, Hq + Hkv, device=dev, dtype=torch.float32)
    _lib.call("mga_qk_norm_rope_fwd", q3.data_ptr(), q3.stride(0), q3.stride(1), k3.data_ptr(), k3.stride(0),
              k3.stride(1), q_weight.data_ptr(), k_weight.data_ptr(), c.data_ptr(), s.data_ptr(), c.stride(0),
              float(eps), S, Hq, Hkv, D, dtype_code(q3.dtype), qo.data_ptr(), qo.stride(1), qo.stride(2),
              ko.data_ptr(), ko.stride(1), ko.stride(2), rstd.data_ptr(), _stream(q3))
    return qo, ko, rstd


def norm_rope_backward(q, k, q_weight, k_weight, cos, sin, rstd, grad_q, grad_k):
    """Gradients [1, S, H, D] of q and k given those of the embeddings
    (grad_q [1, S, Hq, D], grad_k [1, S, Hkv, D], any strides)."""
    q3, k3 = _heads("query_states", q), _heads("key_states", k)
    S, Hq, D = q3.shape
    Hkv = k3.shape[1]
    c, s = _table("cos", cos, S, D), _table("sin", sin, S, D)
    if c.stride(0) != s.stride(0):
        c, s = c.contiguous(), s.contiguous()
    gq, gk = _heads("grad_q", grad_q.to(q3.dtype)), _heads("grad_k", grad_k.to(q3.dtype))
    dq = torch.empty(1, S, Hq, D, device=q3.device, dtype=q3.dtype)
    dk = torch.empty(1, S, Hkv, D, device=q3.device, dtype=q3.dtype)
    _lib.call("mga_qk_norm_rope_bwd", q3.data_ptr(), q3.stride(0), q3.stride(1), k3.data_ptr(), k3.stride(0),
              k3.stride(1), q_weight.data_ptr(), k_weight.data_ptr(), c.data_ptr(), s.data_ptr(), c.stride(0),
              rstd.data_ptr(), S, Hq, Hkv, D, dtype_code(q3.dtype), gq.data_ptr(), gq.stride(0), gq.stride(1),
              gk.data_ptr(), gk.stride(0), gk.stride(1), dq.data_ptr(), dq.stride(1), dq.stride(2),
              dk.data_ptr(), dk.stride(1), dk.stride(2), _stream(q3))
    return dq, dk


def _dst(name: str, t: torch.Tensor, S: int, H: int, D: int, dtype):
    """(token stride, head stride) of a [1, H, S, D] destination view."""
    _dev(name, t)
    if tuple(t.shape) != (1, H, S, D) or t.stride(3) != 1 or t.dtype != dtype:
        raise ValueError(f"{name}: expected a [1, {H}, {S}, {D}] {dtype} view with unit stride on D, got "
                         f"{tuple(t.shape)} {t.dtype} strides {t.stride()}")
    return t.stride(2), t.stride(1)


def norm_rope_stage_forward(q, k, v, q_weight, k_weight, cos, sin, eps: float, k_dst, v_dst,
                            rows: torch.Tensor | None = None):
    """One launch: q / k norm + RoPE as ``norm_rope_forward``, with the key
    embeddings written into ``k_dst`` and v copied into ``v_dst`` ([1, Hkv, S,
    D] views, e.g. KV-cache rows). q may be None (keys and values only). With
    ``rows`` (int32 [n]) output row s takes input row rows[s] (gather; n rows
    written). Returns (q_embed [1, S, Hq, D] or None, rstd or None)."""
    k3, v3 = _heads("key_states", k), _heads("value_states", v)
    S_in, Hkv, D = k3.shape
    if tuple(v3.shape) != (S_in, Hkv, D):
        raise ValueError(f"value_states {tuple(v.shape)} does not match key_states {tuple(k.shape)}")
    c, s = _table("cos", cos, S_in, D), _table("sin", sin, S_in, D)
    if c.stride(0) != s.stride(0):
        c, s = c.contiguous(), s.contiguous()
    _check_dtypes(k3, ("value_states", v3), ("k_weight", k_weight), ("cos", c), ("sin", s))
    if rows is not None:
        _dev("rows", rows)
        if rows.dtype != torch.int32 or rows.dim() != 1 or not rows.is_contiguous():
            raise TypeError("rows: expected a contiguous int32 vector")
        S = rows.numel()
    else:
        S = S_in
    kss, khs = _dst("k_dst", k_dst, S, Hkv, D, k3.dtype)
    vss, vhs = _dst("v_dst", v_dst, S, Hkv, D, k3.dtype)
    qo = rstd = None
    qp = qss = qhs = qop = qoss = qohs = 0
    Hq = 0
    if q is not None:
        q3 = _heads("query_states", q)
        if q3.shape[0] != S_in or q3.shape[2] != D:
            raise ValueError(f"query_states {tuple(q.shape)} does not match key_states {tuple(k.shape)}")
        _check_dtypes(k3, ("query_states", q3), ("q_weight", q_weight))
        Hq = q3.shape[1]
        qo = torch.empty(1, S, Hq, D, device=k3.device, dtype=k3.dtype)
        rstd = torch.empty(S, Hq + Hkv, device=k3.device, dtype=torch.float32)
        qp, qss, qhs, qop, qoss, qohs = q3.data_ptr(), q3.stride(0), q3.stride(1), qo.data_ptr(), qo.stride(1), \
            qo.stride(2)
    for name, w in (("q_weight", q_weight), ("k_weight", k_weight)):
        if w is None and name == "q_weight" and q is None:
            continue
        _dev(name, w)
        if w.dim() != 1 or w.shape[0] != D or w.stride(0) != 1:
            raise ValueError(f"{name}: expected a contiguous [{D}] weight, got {tuple(w.shape)}")
    _lib.call("mga_qk_norm_rope_stage_fwd", qp or None, qss, qhs, k3.data_ptr(), k3.stride(0), k3.stride(1),
              v3.data_ptr(), v3.stride(0), v3.stride(1), q_weight.data_ptr() if q is not None else None,
              k_weight.data_ptr(), c.data_ptr(), s.data_ptr(), c.stride(0), float(eps),
              rows.data_ptr() if rows is not None else None, S_in if rows is not None else 0, S, Hq, Hkv, D,
              dtype_code(k3.dtype), qop or None, qoss, qohs, k_dst.data_ptr(), kss, khs, v_dst.data_ptr(), vss,
              vhs, rstd.data_ptr() if rstd is not None else None, _stream(k3))
    return qo, rstd


class _Restage:
    """Re-stages a chunk's regular rows into the cache prefix from the
    projections (the rows staged in place are overwritten by the gather, so
    they cannot be its source): the same kernel, keys and values only."""

    def __init__(self, k, v, k_weight, cos, sin, eps):
        self.args = (k.detach(), v.detach(), k_weight.detach(), cos.detach(), sin.detach(), eps)

    def __call__(self, idx: torch.Tensor, n: int, k_buf: torch.Tensor, v_buf: torch.Tensor, P: int):
        k, v, kw, cos, sin, eps = self.args
        if n == 0:
            return
        norm_rope_stage_forward(None, k, v, None, kw, cos, sin, eps, k_buf[None, :, P:P + n],
                                v_buf[None, :, P:P + n], rows=idx[:n])


def _alias(t: torch.Tensor) -> torch.Tensor:
    """A tensor on t's memory (same storage, offset, sizes, strides) that is
    not an autograd view of it: the cache buffer it lives in is written again
    through raw pointers (and its version bumped) while the alias is in use."""
    return torch.empty(0, dtype=t.dtype, device=t.device).set_(t.untyped_storage(), t.storage_offset(),
                                                               t.size(), t.stride())


class _QKNormRopeStage(torch.autograd.Function):
    """q embed, and the key embeddings / values written straight into the
    destination rows; returns aliases of those rows whose gradients go back to
    k / v."""

    @staticmethod
    def forward(ctx, q, k, v, q_weight, k_weight, cos, sin, eps, k_dst, v_dst):
        qo, rstd = norm_rope_stage_forward(q, k, v, q_weight, k_weight, cos, sin, eps, k_dst, v_dst)
        ctx.save_for_backward(q, k, q_weight, k_weight, cos, sin, rstd)
        return qo.transpose(1, 2), _alias(k_dst), _alias(v_dst)

    @staticmethod
    def backward(ctx, gq, gk, gv):
        q, k, q_weight, k_weight, cos, sin, rstd = ctx.saved_tensors
        dq, dk = norm_rope_backward(q, k, q_weight, k_weight, cos, sin, rstd, gq.transpose(1, 2),
                                    gk.transpose(1, 2))
        return (dq if ctx.needs_input_grad[0] else None, dk if ctx.needs_input_grad[1] else None,
                gv.transpose(1, 2) if ctx.needs_input_grad[2] else None, None, None, None, None, None, None, None)


def qk_norm_rope_stage(query_states, key_states, value_states, q_weight, k_weight, cos, sin, eps, cache,
                       layer_idx: int):
    """``qk_norm_rope`` for a ``StreamingKVCache`` layer: one kernel writes
    the post-RoPE keys and the values into the cache rows [P, P + S) and
    returns (q_embed [1, Hq, S, D], k, v [1, Hkv, S, D] views of those rows);
    ``cache.update`` given these views copies nothing."""
    if torch.is_grad_enabled():
        for name, w in (("q_norm.weight", q_weight), ("k_norm.weight", k_weight)):
            if w.requires_grad:
                raise NotImplementedError(f"{name} requires grad; the fused q/k norm computes no weight "
                                          "gradient (freeze the base model's norm weights)")
        if cos.requires_grad or sin.requires_grad:
            raise NotImplementedError("cos / sin require grad; the fused rope computes no gradient for them")
    k_dst, v_dst = cache.stage_rows(layer_idx, key_states.transpose(1, 2))
    qe, ke, ve = _QKNormRopeStage.apply(query_states, key_states, value_states, q_weight, k_weight, cos, sin,
                                        eps, k_dst, v_dst)
    ke._mga_restage = _Restage(key_states, value_states, k_weight, cos, sin, eps)
    return qe, ke, ve


class _QKNormRope(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, q_weight, k_weight, cos, sin, eps):
        qo, ko, rstd = norm_rope_forward(q, k, q_weight, k_weight, cos, sin, eps)
        ctx.save_for_backward(q, k, q_weight, k_weight, cos, sin, rstd)
        return qo.transpose(1, 2), ko.transpose(1, 2)

    @staticmethod
    def backward(ctx, gq, gk):
        q, k, q_weight, k_weight, cos, sin, rstd = ctx.saved_tensors
        dq, dk = norm_rope_backward(q, k, q_weight, k_weight, cos, sin, rstd, gq.transpose(1, 2),
                                    gk.transpose(1, 2))
        return (dq if ctx.needs_input_grad[0] else None, dk if ctx.needs_input_grad[1] else None,
                None, None, None, None, None)


def qk_norm_rope(query_states: torch.Tensor, key_states: torch.Tensor, q_weight: torch.Tensor,
                 k_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, eps: float = 1e-6):
    """(q_embed [1, Hq, S, D], k_embed [1, Hkv, S, D]) of the projections
    query_states [1, S, Hq, D] and key_states [1, S, Hkv, D]; equals
    apply_rotary_pos_emb(q_norm(q).transpose(1, 2), k_norm(k).transpose(1, 2),
    cos, sin) of modeling_qwen3.py:274-279 with eps the norms' epsilon."""
    if torch.is_grad_enabled():
        for name, w in (("q_norm.weight", q_weight), ("k_norm.weight", k_weight)):
            if w.requires_grad:
                raise NotImplementedError(f"{name} requires grad; the fused q/k norm computes no weight "
                                          "gradient (freeze the base model's norm weights)")
        if cos.requires_grad or sin.requires_grad:
            raise NotImplementedError("cos / sin require grad; the fused rope computes no gradient for them")
    return _QKNormRope.apply(query_states, key_states, q_weight, k_weight, cos, sin, eps)


def _attention_interface(module):
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    impl = module.config._attn_implementation
    if impl == "eager":
        return sys.modules[type(module).__module__].eager_attention_forward
    return ALL_ATTENTION_FUNCTIONS[impl]


def qwen3_attention_forward(self, hidden_states: torch.Tensor, position_embeddings, attention_mask,
                            gate_mask: torch.Tensor | None = None, past_key_value=None, cache_position=None,
                            **kwargs):
    """Qwen3Attention.forward (modeling_qwen3.py:254-305) with q_norm / k_norm /
    apply_rotary_pos_emb fused into ``qk_norm_rope``. Install with
    ``Qwen3Attention.forward = qwen3_attention_forward``. Takes the reference's
    arguments (gate_mask, past_key_value, cache_position) and transformers'
    ``past_key_values`` keyword; modules without the reference's fused
    ``forward_qkv_proj`` use q_proj / k_proj / v_proj."""
    if past_key_value is None:
        past_key_value = kwargs.pop("past_key_values", None)
    else:
        kwargs.pop("past_key_values", None)
    input_shape = hidden_states.shape[:-1]
    hidden_shape = (*input_shape, -1, self.head_dim)

    if hasattr(self, "forward_qkv_proj"):
        q, k, v = self.forward_qkv_proj(hidden_states, gate_mask)
    else:
        q, k, v = self.q_proj(hidden_states), self.k_proj(hidden_states), self.v_proj(hidden_states)
    if self.q_norm.variance_epsilon != self.k_norm.variance_epsilon:
        raise ValueError("q_norm and k_norm epsilons differ")
    cos, sin = position_embeddings
    if isinstance(past_key_value, StreamingKVCache):
        # keys and values go straight into the cache rows [P, P + S): the
        # update below finds them in place and copies nothing
        query_states, key_states, value_states = qk_norm_rope_stage(
            q.view(hidden_shape), k.view(hidden_shape), v.view(hidden_shape), self.q_norm.weight,
            self.k_norm.weight, cos, sin, self.q_norm.variance_epsilon, past_key_value, self.layer_idx)
    else:
        query_states, key_states = qk_norm_rope(q.view(hidden_shape), k.view(hidden_shape), self.q_norm.weight,
                                                self.k_norm.weight, cos, sin, self.q_norm.variance_epsilon)
        value_states = v.view(hidden_shape).transpose(1, 2)

    if past_key_value is not None:
        cache_kwargs = {"sin": sin, "cos": cos, "cache_position": cache_position}
        key_states, value_states = past_key_value.update(key_states, value_states, self.layer_idx, cache_kwargs)

    attn_output, attn_weights = _attention_interface(self)(
        self, query_states, key_states, value_states, attention_mask,
        dropout=0.0 if not self.training else self.attention_dropout,
        scaling=self.scaling, sliding_window=self.sliding_window, **kwargs)

    attn_output = attn_output.reshape(*input_shape, -1).contiguous()
    attn_output = self.o_proj(attn_output, gate_mask) if gate_mask is not None else self.o_proj(attn_output)
    return attn_output, attn_weights
