"""Gated LoRA linear layers on libmtp_glora_amd.so.

``GatedLoRALinear`` mirrors the reference's module
(mtp_glora/models/layers/gated_lora.py:10-53): same constructor arguments,
same parameters (``base_layer``, ``lora_A``, ``lora_B``; state-dict keys
unchanged), same initialisation, and ``forward(x, gate_mask)`` returning

    base_layer(x) + lora_scaling * lora_B(lora_A(dropout(x))) * gate_mask

in one call of ``mga_gated_lora_fwd`` (a HIP kernel for the down-projection
with dropout fused in, hipBLASLt for the rank-r up-projection and the base
GEMM accumulated onto it); the backward is one call of
``mga_gated_lora_bwd``. ``apply_lora_to_model`` mirrors the reference's
function of the same name (:61-100): it wraps the matching ``nn.Linear``
children (rank and alpha x3 for ``qkv_proj``, x2 for ``gate_up_proj``) and
leaves only ``lora_`` parameters trainable.

Differences from the reference, none of which changes what is learned:
the dropout mask comes from a counter hash of a per-call seed (drawn from
torch's default generator) rather than torch's dropout generator; the scaling
and gate are applied to the rank-r activations before lora_B rather than to
lora_B's output (the same value when the scaling is a power of two and the
gate is 0 / 1, as in the reference's configurations), and the base product
is accumulated in fp32 onto the rounded LoRA term before one final rounding
(in the backward likewise for dX). bf16, fp16 and fp32 layers (the
reference's model dtypes, args.py:15): bf16 runs the HIP down-projection and
streaming backward kernels; fp16 and fp32 run every product in hipBLASLt in
the layer's dtype with HIP kernels for the dropout (the same mask) and the
row scaling, and keep the dropout output for grad_A. Other dtypes raise
TypeError (before apply_lora_to_model changes anything); no biases (Qwen3
and Llama projections have none), base weights frozen.
"""
from __future__ import annotations

import math
import warnings
from typing import List

import torch
import torch.nn as nn

from . import _lib
from .ops import _dev, _stream


def _rpad(rank: int) -> int:
    return (rank + 31) // 32 * 32


DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16, torch.float32: _lib.DTYPE_F32}


def _rows(name: str, t: torch.Tensor, cols: int, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """A [rows, cols] view of ``dtype`` whose rows suit 16-byte vector access."""
    _dev(name, t)
    if t.dtype != dtype:
        raise TypeError(f"{name}: {dtype} required (got {t.dtype})")
    if t.shape[-1] != cols:
        raise ValueError(f"{name}: last dimension {t.shape[-1]} != {cols}")
    v = t.reshape(-1, cols)
    if v.stride(1) != 1 or v.stride(0) % 8 or v.data_ptr() % 16:
        v = v.contiguous()
    return v


def _gate(gate_mask, rows: int, device):
    if gate_mask is None:
        return None
    g = gate_mask.reshape(-1)
    if g.numel() != rows:
        raise ValueError(f"gate_mask has {g.numel()} entries for {rows} rows")
    return g.to(device=device, dtype=torch.float32).contiguous()


def _workspace(S: int, K: int, N: int, rank: int, device) -> torch.Tensor:
    n = int(_lib.load().mga_gated_lora_workspace_bytes(S, K, N, rank))
    return torch.empty(n, dtype=torch.uint8, device=device)


def gated_lora_forward(x2, weight, lora_a, lora_b, gate, scaling: float, p: float, seed: int,
                       keep_h: bool = False):
    """y [S, N], t [S, rpad] and h [S, K] = dropout(x2) for x2 [S, K]. h is
    None unless dropout is on and either ``keep_h`` asks for it or K is not a
    multiple of 128 (the backward otherwise draws the mask again from x2)."""
    S, K = x2.shape
    N, rank = weight.shape[0], lora_a.shape[0]
    dev, dt = x2.device, x2.dtype
    y = torch.empty(S, N, device=dev, dtype=dt)
    t = torch.empty(S, _rpad(rank), device=dev, dtype=dt)
    # the general path (fp16 / fp32) always keeps h: its grad_A reads it
    h = torch.empty(S, K, device=dev, dtype=dt) if p > 0 and (keep_h or K % 128 or dt != torch.bfloat16) else None
    ws = _workspace(S, K, N, rank, dev)
    _lib.call("mga_gated_lora_fwd", x2.data_ptr(), x2.stride(0), weight.data_ptr(), weight.stride(0),
              lora_a.data_ptr(), lora_a.stride(0), lora_b.data_ptr(), lora_b.stride(0),
              gate.data_ptr() if gate is not None else None, float(scaling), float(p), seed,
              S, K, N, rank, y.data_ptr(), y.stride(0), t.data_ptr(), t.stride(0),
              h.data_ptr() if h is not None else None, h.stride(0) if h is not None else 0,
              ws.data_ptr(), ws.numel(), DTYPES[dt], _stream(x2))
    return y, t, h


def gated_lora_backward(gy2, x2, h, t, weight, lora_a, lora_b, gate, scaling: float, p: float, seed: int,
                        need_x: bool, need_a: bool, need_b: bool):
    S, K = x2.shape
    N, rank = weight.shape[0], lora_a.shape[0]
    dev, dt = x2.device, x2.dtype
    gx = torch.empty(S, K, device=dev, dtype=dt) if need_x else None
    ga = torch.empty(rank, K, device=dev, dtype=dt) if need_a else None
    gb = torch.empty(N, rank, device=dev, dtype=dt) if need_b else None
    ws = _workspace(S, K, N, rank, dev)
    ptr = lambda v: v.data_ptr() if v is not None else None   # noqa: E731
    rs = lambda v: v.stride(0) if v is not None else 0         # noqa: E731
    _lib.call("mga_gated_lora_bwd", gy2.data_ptr(), gy2.stride(0), x2.data_ptr(), x2.stride(0), ptr(h), rs(h),
              weight.data_ptr(), weight.stride(0), lora_a.data_ptr(), lora_a.stride(0), lora_b.data_ptr(),
              lora_b.stride(0), t.data_ptr(), t.stride(0), ptr(gate), float(scaling), float(p), seed,
              S, K, N, rank, ptr(gx), rs(gx), ptr(ga), rs(ga), ptr(gb), rs(gb),
              ws.data_ptr(), ws.numel(), DTYPES[dt], _stream(x2))
    return gx, ga, gb


class _GatedLoRA(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, lora_a, lora_b, gate_mask, scaling, p, seed):
        K = weight.shape[1]
        dt = weight.dtype
        if dt not in DTYPES:
            raise TypeError(f"weight: bfloat16, float16 or float32 required (got {dt})")
        x2 = _rows("x", x, K, dt)
        for name, w in (("weight", weight), ("lora_A.weight", lora_a), ("lora_B.weight", lora_b)):
            _dev(name, w)
            if w.dtype != dt:
                raise TypeError(f"{name}: {dt} required (got {w.dtype})")
        weight, lora_a, lora_b = weight.contiguous(), lora_a.contiguous(), lora_b.contiguous()
        if lora_a.shape[1] != K or lora_b.shape != (weight.shape[0], lora_a.shape[0]):
            raise ValueError(f"shapes: weight {tuple(weight.shape)}, lora_A {tuple(lora_a.shape)}, "
                             f"lora_B {tuple(lora_b.shape)}")
        gate = _gate(gate_mask, x2.shape[0], x2.device)
        y, t, h = gated_lora_forward(x2, weight, lora_a, lora_b, gate, scaling, p, seed)
        ctx.save_for_backward(x2, h, t, weight, lora_a, lora_b, gate)
        ctx.meta = (scaling, p, seed, x.shape)
        return y.view(*x.shape[:-1], weight.shape[0])

    @staticmethod
    def backward(ctx, gy):
        x2, h, t, weight, lora_a, lora_b, gate = ctx.saved_tensors
        scaling, p, seed, xshape = ctx.meta
        gy2 = _rows("grad_output", gy.to(weight.dtype), weight.shape[0], weight.dtype)
        gx, ga, gb = gated_lora_backward(gy2, x2, h, t, weight, lora_a, lora_b, gate, scaling, p, seed,
                                         ctx.needs_input_grad[0], ctx.needs_input_grad[2],
                                         ctx.needs_input_grad[3])
        return (gx.view(xshape) if gx is not None else None, None, ga, gb, None, None, None, None)


def gated_lora_linear(x, weight, lora_a, lora_b, gate_mask, scaling: float, dropout_p: float = 0.0,
                      seed: int | None = None):
    """Functional form: ``x W^T + scaling * lora_B(lora_A(dropout(x))) * gate_mask``."""
    if torch.is_grad_enabled() and weight.requires_grad:
        raise NotImplementedError("the base weight must be frozen (the fused layer computes no gradient for it)")
    if seed is None:
        seed = int(torch.randint(0, 2 ** 62, (), dtype=torch.int64).item()) if dropout_p > 0 else 0
    return _GatedLoRA.apply(x, weight, lora_a, lora_b, gate_mask, float(scaling), float(dropout_p), int(seed))


class GatedLoRALinear(nn.Module):
    """Drop-in for mtp_glora/models/layers/gated_lora.py:10-53."""

    def __init__(self, base_layer: nn.Linear, rank: int, alpha: float, dropout: float, lora_bias: bool,
                 use_rslora: bool):
        super().__init__()
        _check_base_dtype("base_layer", base_layer)
        self.base_layer = base_layer
        self.rank = rank
        self.alpha = alpha
        self.lora_scaling = alpha / math.sqrt(rank) if use_rslora else alpha / rank
        if lora_bias and base_layer.bias is None:
            warnings.warn("lora_bias is True but base_linear.bias is None")
        self.dropout = nn.Dropout(p=dropout) if dropout > 0 else nn.Identity()
        w = base_layer.weight
        self.lora_A = nn.Linear(base_layer.in_features, rank, bias=False, dtype=w.dtype, device=w.device)
        self.lora_B = nn.Linear(rank, base_layer.out_features, bias=lora_bias, dtype=w.dtype, device=w.device)
        nn.init.kaiming_uniform_(self.lora_A.weight, a=math.sqrt(5))
        nn.init.zeros_(self.lora_B.weight)

    def forward(self, x: torch.Tensor, gate_mask: torch.Tensor | None = None):
        if self.base_layer.bias is not None or self.lora_B.bias is not None:
            raise NotImplementedError("biases are not supported by the fused gated LoRA layer")
        p = self.dropout.p if (self.training and isinstance(self.dropout, nn.Dropout)) else 0.0
        return gated_lora_linear(x, self.base_layer.weight, self.lora_A.weight, self.lora_B.weight, gate_mask,
                                 self.lora_scaling, p)


def _check_base_dtype(name: str, layer: nn.Linear) -> None:
    if layer.weight.dtype not in DTYPES:
        raise TypeError(f"{name}: the fused gated LoRA layer supports bfloat16, float16 and float32 base "
                        f"layers (got {layer.weight.dtype})")


def _freeze_base_and_enable_lora(model: nn.Module) -> None:
    for name, param in model.named_parameters():
        param.requires_grad = "lora_" in name


def apply_lora_to_model(model: nn.Module, target_modules: List[str] = None, rank: int = 16, alpha: float = 32,
                        dropout: float = 0.1, lora_bias: bool = False, use_rslora: bool = False) -> None:
    """Wrap every ``nn.Linear`` whose child name contains a target in
    ``GatedLoRALinear`` (the reference's rule, gated_lora.py:61-100)."""
    targets = target_modules or ["qkv_proj", "o_proj", "gate_up_proj", "down_proj"]

    def matches(module: nn.Module, prefix: str = ""):
        for name, child in module.named_children():
            if isinstance(child, nn.Linear):
                if any(t in name for t in targets):
                    yield module, name, child, prefix + name
            else:
                yield from matches(child, prefix + name + ".")

    found = list(matches(model))
    for _, _, child, path in found:   # every target checked before the model changes
        _check_base_dtype(path, child)
    for module, name, child, _ in found:
        mult = 3 if "qkv_proj" in name else (2 if "gate_up_proj" in name else 1)
        setattr(module, name, GatedLoRALinear(child, mult * rank, mult * alpha, dropout, lora_bias, use_rslora))
    _freeze_base_and_enable_lora(model)
