"""Tensor-level wrappers over the C ABI.

PyTorch supplies device memory and the current HIP stream; every computation
runs in libmtp_glora_amd.so. Inputs must be device tensors: a CPU tensor is an
error, never a reason to compute elsewhere.
"""
from __future__ import annotations

import math

import torch

from . import _lib

BLOCK = 128


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _dev(name: str, t: torch.Tensor) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name}: expected a GPU tensor, got device {t.device}; "
                           "libmtp_glora_amd has no CPU path")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return _lib.DTYPE_BF16
    if dt == torch.float16:
        return _lib.DTYPE_F16
    if dt == torch.float32:
        return _lib.DTYPE_F32
    raise TypeError(f"unsupported dtype {dt}; expected bfloat16, float16 or float32")


def _rows(name: str, t: torch.Tensor):
    """(ptr, stride_h, stride_s) of a [1, H, seq, D] or [H, seq, D] operand;
    copies only if the last dim is not contiguous or rows are misaligned."""
    _dev(name, t)
    if t.dim() == 4:
        if t.shape[0] != 1:
            raise ValueError(f"{name}: batch size must be 1 (got {t.shape[0]})")
        t3 = t[0]
    elif t.dim() == 3:
        t3 = t
    else:
        raise ValueError(f"{name}: expected [1, H, seq, D] or [H, seq, D], got {tuple(t.shape)}")
    eb = t3.element_size()
    ok = (t3.stride(2) == 1 and (t3.stride(0) * eb) % 16 == 0 and (t3.stride(1) * eb) % 16 == 0
          and t3.data_ptr() % 16 == 0)
    if not ok:
        t3 = t3.contiguous()
    return t3, t3.stride(0), t3.stride(1)


# ----------------------------------------------------------------------------
# Cache
# ----------------------------------------------------------------------------

def kv_append(src_k: torch.Tensor, src_v: torch.Tensor, dst_k: torch.Tensor, dst_v: torch.Tensor,
              dst_offset: int, idx: torch.Tensor | None = None, n_rows: int | None = None) -> None:
    """dst[:, dst_offset + r] = src[:, idx[r] if idx is not None else r] for K and V.

    src: [1, H, S, D] or [H, S, D] views; dst: [H, capacity, D] buffers.
    """
    sk, ssh, sss = _rows("src_k", src_k)
    sv, vsh, vss = _rows("src_v", src_v)
    if (vsh, vss) != (ssh, sss) or sv.shape != sk.shape:
        sk, sv = sk.contiguous(), sv.contiguous()
        ssh, sss = sk.stride(0), sk.stride(1)
    _dev("dst_k", dst_k)
    _dev("dst_v", dst_v)
    if dst_k.dim() != 3 or dst_k.shape != dst_v.shape or dst_k.stride() != dst_v.stride():
        raise ValueError("dst_k/dst_v must be matching [H, capacity, D] buffers")
    if dst_k.dtype != sk.dtype or dst_v.dtype != sv.dtype:
        raise TypeError(f"cache dtype {dst_k.dtype} != source dtype {sk.dtype}")
    H, cap, D = dst_k.shape
    if sk.shape[0] != H or sk.shape[2] != D:
        raise ValueError(f"source heads/head_dim {tuple(sk.shape)} do not match cache {tuple(dst_k.shape)}")
    if idx is not None:
        _dev("idx", idx)
        if idx.dtype != torch.int32 or not idx.is_contiguous():
            raise TypeError("idx must be a contiguous int32 tensor")
        rows = int(idx.numel()) if n_rows is None else int(n_rows)
    else:
        rows = sk.shape[1] if n_rows is None else int(n_rows)
    _lib.call("mga_kv_append", sk.data_ptr(), sv.data_ptr(), ssh, sss, sk.shape[1],
              idx.data_ptr() if idx is not None else None, rows,
              dst_k.data_ptr(), dst_v.data_ptr(), dst_k.stride(0), dst_k.stride(1),
              int(dst_offset), cap, H, D, dtype_code(dst_k.dtype), _stream(dst_k))


def regular_index(regular_mask: torch.Tensor):
    """int32 indices of the nonzero entries of a [1, S] (or [S]) int64 mask,
    plus the device count. Returns (idx[S], count[1])."""
    _dev("regular_token_mask", regular_mask)
    m = regular_mask.reshape(-1) if regular_mask.dim() == 2 and regular_mask.shape[0] == 1 else regular_mask
    if m.dim() != 1:
        raise ValueError("regular_token_mask must be [1, S] or [S]")
    if m.dtype != torch.int64:
        m = m.to(torch.int64)
    n = m.numel()
    idx = torch.empty(n, dtype=torch.int32, device=m.device)
    cnt = torch.empty(1, dtype=torch.int32, device=m.device)
    _lib.call("mga_regular_index", m.data_ptr(), m.stride(0), n, idx.data_ptr(), cnt.data_ptr(),
              _stream(m))
    return idx, cnt


# ----------------------------------------------------------------------------
# Block mask
# ----------------------------------------------------------------------------

def mtp_block_mask_tensors(gate: torch.Tensor, P: int) -> dict:
    """Codes and the eight BlockMask tensors ([1, 1, ...] int32) of the MTP
    mask of a chunk with gate ``gate`` ([1, S] int64) against a P-token prefix."""
    _dev("gate_mask", gate)
    g = gate.reshape(-1) if gate.dim() == 2 and gate.shape[0] == 1 else gate
    if g.dim() != 1:
        raise ValueError("gate_mask must be [1, S] or [S]")
    if g.dtype != torch.int64:
        g = g.to(torch.int64)
    S = g.numel()
    L = P + S
    nQ = -(-S // BLOCK)
    nKV = -(-L // BLOCK)
    dev = g.device
    # one int32 allocation carved into the nine outputs (each 16-byte aligned)
    shapes = dict(code=(S,), kv_num_blocks=(1, 1, nQ), kv_indices=(1, 1, nQ, nKV),
                  full_kv_num_blocks=(1, 1, nQ), full_kv_indices=(1, 1, nQ, nKV),
                  q_num_blocks=(1, 1, nKV), q_indices=(1, 1, nKV, nQ),
                  full_q_num_blocks=(1, 1, nKV), full_q_indices=(1, 1, nKV, nQ))
    sizes = {n: math.prod(sh) for n, sh in shapes.items()}
    total = sum((n_ + 3) // 4 * 4 for n_ in sizes.values())
    buf = torch.empty(total, dtype=torch.int32, device=dev)
    out, off = {}, 0
    for n, sh in shapes.items():
        out[n] = buf[off:off + sizes[n]].view(sh)
        off += (sizes[n] + 3) // 4 * 4
    out["tile_class"] = torch.empty(nQ * nKV, dtype=torch.int8, device=dev)
    _lib.call("mga_mtp_block_mask", g.data_ptr(), g.stride(0), S, int(P),
              out["code"].data_ptr(), out["tile_class"].data_ptr(),
              out["kv_num_blocks"].data_ptr(), out["kv_indices"].data_ptr(),
              out["full_kv_num_blocks"].data_ptr(), out["full_kv_indices"].data_ptr(),
              out["q_num_blocks"].data_ptr(), out["q_indices"].data_ptr(),
              out["full_q_num_blocks"].data_ptr(), out["full_q_indices"].data_ptr(), _stream(g))
    return out


# ----------------------------------------------------------------------------
# Attention
# ----------------------------------------------------------------------------

def attn_fwd(q, k, v, code, bm: dict, P: int, scale: float):
    """q [1, Hq, S, D]; k/v [1, Hkv, L, D] with L = P + S.
    Returns o [1, S, Hq, D] (contiguous) and lse [1, Hq, S] fp32 (natural log)."""
    qq, q_sh, q_ss = _rows("query", q)
    kk, k_sh, k_ss = _rows("key", k)
    vv, v_sh, v_ss = _rows("value", v)
    Hq, S, D = qq.shape
    Hkv, L, _ = kk.shape
    if vv.shape != kk.shape:
        raise ValueError(f"key {tuple(kk.shape)} and value {tuple(vv.shape)} shapes differ")
    if L != P + S:
        raise ValueError(f"key length {L} != prefix {P} + queries {S}")
    if kk.dtype != qq.dtype or vv.dtype != qq.dtype:
        raise TypeError("query, key and value must share one dtype")
    o = torch.empty(1, S, Hq, D, dtype=qq.dtype, device=qq.device)
    lse = torch.empty(1, Hq, S, dtype=torch.float32, device=qq.device)
    _lib.call("mga_attn_fwd", qq.data_ptr(), q_sh, q_ss, kk.data_ptr(), k_sh, k_ss,
              vv.data_ptr(), v_sh, v_ss, o.data_ptr(), D, Hq * D, lse.data_ptr(), code.data_ptr(),
              bm["kv_num_blocks"].data_ptr(), bm["kv_indices"].data_ptr(),
              bm["full_kv_num_blocks"].data_ptr(), bm["full_kv_indices"].data_ptr(),
              S, L, P, Hq, Hkv, D, dtype_code(qq.dtype), float(scale), _stream(qq))
    return o, lse


def bwd_buffers(q, k, grad_start: int) -> dict:
    """Output and workspace buffers of ``attn_bwd``: dq [1, S, Hq, D], dk/dv
    [1, L - grad_start, Hkv, D] (None when grad_start == L) and delta, the
    backward's row-data workspace of ``BWD_WS_WORDS_PER_ROW * Hq * S`` 32-bit
    words (fp32 storage)."""
    _, Hq, S, D = q.shape
    _, Hkv, L, _ = k.shape
    dev, dt = q.device, q.dtype
    Lg = L - grad_start
    return dict(dq=torch.empty(1, S, Hq, D, dtype=dt, device=dev),
                dk=torch.empty(1, Lg, Hkv, D, dtype=dt, device=dev) if Lg > 0 else None,
                dv=torch.empty(1, Lg, Hkv, D, dtype=dt, device=dev) if Lg > 0 else None,
                delta=torch.empty(_lib.BWD_WS_WORDS_PER_ROW * Hq * S, dtype=torch.float32, device=dev))


def attn_bwd(q, k, v, o, lse, dout, code, bm: dict, P: int, scale: float, grad_start: int,
             passes: int = _lib.BWD_DQ | _lib.BWD_DKDV, buffers: dict | None = None,
             no_alloc: bool = False):
    """Gradients of ``attn_fwd``. Returns dq [1, Hq, S, D] (a transposed view of
    an [1, S, Hq, D] buffer), and dk, dv [1, Hkv, L - grad_start, D] (views of
    [1, L - grad_start, Hkv, D] buffers) or None when grad_start == L.

    ``passes`` selects the dQ pass (which also writes delta = rowsum(o * dout))
    and/or the dK/dV pass; to issue them as two calls in stream order, pass the
    same ``buffers`` (from ``bwd_buffers``) to both, the dQ pass first.

    ``no_alloc`` calls ``mga_attn_bwd_noalloc``: delta lives in the library's
    fixed per-GPU workspace instead of ``buffers["delta"]``."""
    qq, q_sh, q_ss = _rows("query", q)
    kk, k_sh, k_ss = _rows("key", k)
    vv, v_sh, v_ss = _rows("value", v)
    Hq, S, D = qq.shape
    Hkv, L, _ = kk.shape
    o3 = o[0] if o.dim() == 4 else o             # [S, Hq, D]
    d3 = dout[0] if dout.dim() == 4 else dout
    _dev("grad_output", d3)
    if d3.shape != o3.shape:
        raise ValueError(f"grad_output shape {tuple(d3.shape)} != output shape {tuple(o3.shape)}")
    if d3.dtype != qq.dtype:
        d3 = d3.to(qq.dtype)
    if d3.stride(2) != 1 or (d3.stride(0) * d3.element_size()) % 16 or (d3.stride(1) * d3.element_size()) % 16 \
            or d3.data_ptr() % 16:
        d3 = d3.contiguous()
    b = buffers if buffers is not None else bwd_buffers(q, k, grad_start)
    dq, dk, dv, delta = b["dq"], b["dk"], b["dv"], b["delta"]
    if dq.shape != (1, S, Hq, D) or delta.numel() != _lib.BWD_WS_WORDS_PER_ROW * Hq * S:
        raise ValueError("backward buffers do not match the operands")
    dk_ptr = dk.data_ptr() if dk is not None else None
    dv_ptr = dv.data_ptr() if dv is not None else None
    # o3 is [S, Hq, D]: element (h, s, d) at h * D + s * Hq * D + d
    head = (["mga_attn_bwd_noalloc", qq.data_ptr(), q_sh, q_ss, kk.data_ptr(), k_sh, k_ss,
             vv.data_ptr(), v_sh, v_ss, o3.data_ptr(), o3.stride(1), o3.stride(0),
             d3.data_ptr(), d3.stride(1), d3.stride(0), lse.data_ptr()] if no_alloc else
            ["mga_attn_bwd", qq.data_ptr(), q_sh, q_ss, kk.data_ptr(), k_sh, k_ss,
             vv.data_ptr(), v_sh, v_ss, o3.data_ptr(), o3.stride(1), o3.stride(0),
             d3.data_ptr(), d3.stride(1), d3.stride(0), lse.data_ptr(), delta.data_ptr()])
    _lib.call(*head,
              dq.data_ptr(), D, Hq * D, dk_ptr, D, Hkv * D, dv_ptr, D, Hkv * D,
              int(grad_start), code.data_ptr(),
              bm["kv_num_blocks"].data_ptr(), bm["kv_indices"].data_ptr(),
              bm["full_kv_num_blocks"].data_ptr(), bm["full_kv_indices"].data_ptr(),
              bm["q_num_blocks"].data_ptr(), bm["q_indices"].data_ptr(),
              bm["full_q_num_blocks"].data_ptr(), bm["full_q_indices"].data_ptr(),
              S, L, P, Hq, Hkv, D, dtype_code(qq.dtype), float(scale), int(passes), _stream(qq))
    dq_t = dq.transpose(1, 2)
    if dk is None:
        return dq_t, None, None
    return dq_t, dk.transpose(1, 2), dv.transpose(1, 2)
