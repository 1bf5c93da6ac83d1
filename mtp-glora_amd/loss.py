"""Stable soft cross-entropy of the MTP sampler loss, on the HIP kernels of
libmtp_glora_amd.so.

``StableSoftCrossEntropy`` mirrors the reference's autograd Function
(mtp_glora/core/loss.py:259-330): ``apply(student_logits, teacher_logits)``
with two [B, T, V] tensors of the same shape returns the sum over rows of

    -(sum_j e^{t_j - mt} x_j) / dt + mx + log dx

(the cross-entropy of softmax(student) against softmax(teacher)), and its
backward returns the student's gradient in the student's dtype and None for
the teacher. Differences from the reference that do not change results: rows
are read through their strides (the reference makes both operands
contiguous first; the teacher it is called with, ``core/mtp.py:124``, is a
strided view), the student and teacher rows are read once each in the
forward (the reference reads the student twice), and the gradient is written
in the student's dtype directly (the reference writes fp32 and casts).
"""
from __future__ import annotations

import torch

from . import _lib
from .ops import _dev, _stream, dtype_code


def _row_view(name: str, t: torch.Tensor, rows: int, cols: int):
    """A [rows, cols] view with contiguous columns (a copy only if needed)."""
    _dev(name, t)
    if t.dim() != 3:
        raise ValueError(f"{name}: expected [B, T, V], got {tuple(t.shape)}")
    v = t.reshape(rows, cols) if t.stride(2) == 1 else None
    if v is None or v.stride(1) != 1:
        v = t.contiguous().view(rows, cols)
    return v


def soft_ce_forward(student: torch.Tensor, teacher: torch.Tensor):
    """Row losses [B*T] and the saved statistics [4, B*T] (mx, dx, mt, dt)."""
    if student.shape != teacher.shape:
        raise ValueError(f"student {tuple(student.shape)} and teacher {tuple(teacher.shape)} differ")
    if student.dtype != teacher.dtype:
        raise TypeError(f"student dtype {student.dtype} != teacher dtype {teacher.dtype}")
    B, T, V = student.shape
    N = B * T
    x = _row_view("student", student, N, V)
    t = _row_view("teacher", teacher, N, V)
    dev = x.device
    loss = torch.empty(N, device=dev, dtype=torch.float32)
    stats = torch.empty(4, N, device=dev, dtype=torch.float32)
    ws = torch.empty(int(_lib.load().mga_soft_ce_workspace_floats(N, V)), device=dev, dtype=torch.float32)
    _lib.call("mga_soft_ce_fwd", x.data_ptr(), x.stride(0), t.data_ptr(), t.stride(0), N, V,
              dtype_code(x.dtype), loss.data_ptr(), stats.data_ptr(), ws.data_ptr(), _stream(x))
    return loss, stats


def soft_ce_backward(student: torch.Tensor, teacher: torch.Tensor, stats: torch.Tensor,
                     grad_output: torch.Tensor) -> torch.Tensor:
    """Gradient of the summed loss with respect to the student, [B, T, V]."""
    B, T, V = student.shape
    N = B * T
    x = _row_view("student", student, N, V)
    t = _row_view("teacher", teacher, N, V)
    go = grad_output.detach().reshape(1).to(device=x.device, dtype=torch.float32).contiguous()
    grad = torch.empty(N, V, device=x.device, dtype=student.dtype)
    _lib.call("mga_soft_ce_bwd", x.data_ptr(), x.stride(0), t.data_ptr(), t.stride(0), N, V,
              dtype_code(x.dtype), go.data_ptr(), stats.data_ptr(), grad.data_ptr(), grad.stride(0), _stream(x))
    return grad.view(B, T, V)


class StableSoftCrossEntropy(torch.autograd.Function):
    """Drop-in for mtp_glora/core/loss.py:259-330 (called at core/mtp.py:126)."""

    @staticmethod
    def forward(ctx, student_logits: torch.Tensor, teacher_logits: torch.Tensor):
        if student_logits.ndim != 3 or teacher_logits.ndim != 3:
            raise ValueError("student and teacher logits must be [B, T, V]")
        loss, stats = soft_ce_forward(student_logits.detach(), teacher_logits.detach())
        ctx.save_for_backward(student_logits.detach(), teacher_logits.detach(), stats)
        return loss.sum()

    @staticmethod
    def backward(ctx, grad_output):
        student, teacher, stats = ctx.saved_tensors
        return soft_ce_backward(student, teacher, stats, grad_output), None
