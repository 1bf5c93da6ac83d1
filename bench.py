#!/usr/bin/env python3
"""Benchmark of the chunked-training hot path on one MI355X.

Metric: masked-attention fwd+bwd TFLOP/s and KV-append GB/s
per chunk at Qwen3-8B attention geometry. Workload: config 2 (one layer,
32 query / 8 KV heads, head_dim 128, bf16; a 8192-token cached prefix; a chunk
of 4096 regular tokens + 256 anchors x 4 mask tokens = 5120 query rows).

One step is one layer-chunk through the drop-in boundary, exactly as the
trainer's chunk loop drives it (mtp_glora/trainer/trainer.py:95-136):
  prepare_data_with_kv_cache (MTP block mask on the GPU) -> cache.update (stage
  the chunk's K/V after the prefix) -> attention forward -> backward (dQ, and
  dK/dV of the chunk's keys) -> extract_regular_kv_cache_for_next_chunk
  (regular-token index + gather-append of the 4096 regular rows),
then the cache is cropped back to the same prefix so every step is identical.
Inputs are resident in HBM before the timed region.

``value`` = credited attention FLOPs per step / measured step time (the whole
step: mask build, appends and attention). The credited FLOPs count only the
non-empty 128x128 tiles of the reference BlockMask and no dK/dV for the
detached prefix: Hq*D*[4(A_pre+A_cur) + 6 A_pre + 10 A_cur]. Per-kernel
durations (HIP events on the launch stream) give the roofline fractions.

``cpu_baseline``: the reference's CPU path (torch flex_attention eager -- the
dense math path -- fwd + autograd bwd on the restated MTP mask_mod) over the
whole layer-chunk, one KV-head group (4 query heads, full S and P+S) after
another; beside it, ``compiled_fwd_only``: torch.compile(flex_attention)
forward on the first group, which on the CPU serves inference only (no LSE,
no backward).

``north_star``, ``config3_stream`` and ``config5_step``: the north-star point
(config 3's last chunk as one layer-chunk step), the whole config-3 stream (36
layers x 8 chunks) and the config-5 step, timed in the same run.
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "masked-attn fwd+bwd TFLOP/s + KV append GB/s per chunk, Qwen3-8B shape, 1 GPU"
PEAK_MFMA_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0           # MI355X HBM3E

CONFIGS = {
    2: dict(workload="config2: Qwen3-8B single layer, 4096 regular + 256x4 mask rows vs 8192-token prefix",
            Hq=32, Hkv=8, D=128, P=8192, n_reg=4096, n_anchor=256, draft=4, every=None),
    5: dict(workload="config5: Qwen3-4B dense MTP, 2048 regular + 512x8 mask rows vs 16384-token prefix",
            Hq=32, Hkv=8, D=128, P=16384, n_reg=2048, n_anchor=512, draft=8, every=4),
}
SEED = 1234

# Chunk streams: per chunk (regular rows, anchors, draft length); every layer
# runs update -> attention fwd -> bwd, then the regular rows are committed
# (except after the last chunk, trainer.py:133).
STREAMS = {
    3: dict(workload="config3: Qwen3-8B, 36 layers, 8 chunks of 4096 regular + 512x4 mask rows, "
                     "prefix 0 -> 28672",
            Hq=32, Hkv=8, D=128, layers=36, chunks=[(4096, 512, 4)] * 8),
    4: dict(workload="config4: Llama-3.1-8B, 32 layers, 32 chunks of 4096 regular + 256x4 mask rows "
                     "to a 131072-token prefix, then a 768 regular + 64x4 mask (1024-row) remainder chunk",
            Hq=32, Hkv=8, D=128, layers=32, chunks=[(4096, 256, 4)] * 32 + [(768, 64, 4)]),
}


def tile_areas(bm, S: int, L: int, P: int, block: int = 128):
    """(A_pre, A_cur): clipped areas of the non-empty tiles of the block mask,
    split at the prefix boundary P."""
    kv_num = bm.kv_num_blocks[0, 0].tolist()
    kv_idx = bm.kv_indices[0, 0].tolist()
    fkv_num = bm.full_kv_num_blocks[0, 0].tolist()
    fkv_idx = bm.full_kv_indices[0, 0].tolist()
    a_pre = a_cur = 0
    for qt in range(len(kv_num)):
        rows = min(block, S - qt * block)
        for kt in kv_idx[qt][:kv_num[qt]] + fkv_idx[qt][:fkv_num[qt]]:
            k0, k1 = kt * block, min(L, kt * block + block)
            npre = max(0, min(k1, P) - k0)
            a_pre += rows * npre
            a_cur += rows * (k1 - k0 - npre)
    return a_pre, a_cur


class EventTimer:
    """Average duration of a callable's GPU work over ``n`` back-to-back runs,
    from HIP events recorded on the stream the kernels are launched on."""

    def __init__(self, torch):
        self.torch = torch

    def __call__(self, fn, n: int) -> float:
        torch = self.torch
        st = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        fn()
        torch.cuda.synchronize()
        e0.record(st)
        for _ in range(n):
            fn()
        e1.record(st)
        e1.synchronize()
        return e0.elapsed_time(e1) / n


QWEN3_VOCAB = 151936


def soft_ce_phase(torch, mga, timer, rows: int, vocab: int, n: int, cpu_rows: int) -> dict:
    """The sampler's soft cross-entropy (StableSoftCrossEntropy) at [1, rows,
    vocab] bf16: forward and backward kernel time (HIP events), bytes moved
    against the HBM peak, and the reference's math as torch eager on the CPU
    for ``cpu_rows`` rows (the reference's kernel is Triton, GPU-only)."""
    from importlib import import_module
    lossmod = import_module("mtp-glora_amd.loss")
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(SEED + 7)
    x = (torch.randn(1, rows, vocab, generator=g, device=dev) * 3).bfloat16()
    t = (torch.randn(1, rows, vocab, generator=g, device=dev) * 3).bfloat16()
    go = torch.ones((), device=dev)
    loss, stats = lossmod.soft_ce_forward(x, t)
    t_f = timer(lambda: lossmod.soft_ce_forward(x, t), n)
    t_b = timer(lambda: lossmod.soft_ce_backward(x, t, stats, go), n)
    elems = rows * vocab
    fwd_bytes = 2 * elems * 2                 # student and teacher read once
    bwd_bytes = 3 * elems * 2                 # both read, the bf16 gradient written
    fwd_gbps = fwd_bytes / (t_f * 1e-3) / 1e9
    bwd_gbps = bwd_bytes / (t_b * 1e-3) / 1e9
    # CPU: the reference's formulas (loss.py:14-28 forward, autograd backward)
    xc = x[0, :cpu_rows].float().cpu()
    tc = t[0, :cpu_rows].float().cpu()
    secs = []
    for _ in range(4):
        xr = xc.clone().requires_grad_()
        t0 = time.perf_counter()
        mx = xr.amax(dim=-1, keepdim=True)
        dx = (xr - mx).exp().sum(dim=-1, keepdim=True).clamp_min(1e-20)
        mt = tc.amax(dim=-1, keepdim=True)
        dt = (tc - mt).exp().sum(dim=-1, keepdim=True).clamp_min(1e-20)
        ce = (-(((tc - mt).exp() * xr).sum(dim=-1, keepdim=True) / dt) + mx + dx.log()).sum()
        ce.backward()
        secs.append(time.perf_counter() - t0)
    cpu_s = sorted(secs[1:])[1]
    return {"rows": rows, "vocab": vocab, "dtype": "bf16",
            "fwd_ms": round(t_f, 4), "bwd_ms": round(t_b, 4),
            "fwd_GBps": round(fwd_gbps, 1), "bwd_GBps": round(bwd_gbps, 1),
            "fwd_frac": round(fwd_gbps / PEAK_HBM_GBPS, 4), "bwd_frac": round(bwd_gbps / PEAK_HBM_GBPS, 4),
            "peak": PEAK_HBM_GBPS, "bytes": {"fwd": fwd_bytes, "bwd": bwd_bytes},
            "cpu_rows_per_s": round(cpu_rows / cpu_s, 1), "gpu_rows_per_s": round(rows / ((t_f + t_b) * 1e-3), 1),
            "cpu_sample": f"torch eager fp32 on the CPU, the reference's formulas, {cpu_rows} rows, fwd + bwd, "
                          f"median of 3 after a warm-up, {torch.get_num_threads()} threads"}


def qk_rope_phase(torch, timer, S: int, Hq: int, Hkv: int, D: int, n: int, cpu_tokens: int) -> dict:
    """Qwen3 q_norm / k_norm + rotary embedding (qk_norm_rope) at the chunk's
    [1, S, H, D] bf16 projections: forward and backward kernel time (HIP
    events around a graph of 20 launches), bytes against the HBM peak; the
    reference's ops
    (Qwen3RMSNorm + apply_rotary_pos_emb, modeling_qwen3.py:274-279) as torch
    eager on the same GPU for comparison, and on the CPU for ``cpu_tokens``."""
    from importlib import import_module
    rope = import_module("mtp-glora_amd.rope")
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(SEED + 9)
    bf = torch.bfloat16
    q = torch.randn(1, S, Hq, D, generator=g, device=dev).to(bf)
    k = torch.randn(1, S, Hkv, D, generator=g, device=dev).to(bf)
    qw = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(bf)
    kw = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(bf)
    pos = torch.arange(S, device=dev, dtype=torch.float32)[:, None]
    inv = 1e6 ** (-torch.arange(0, D, 2, device=dev, dtype=torch.float32) / D)
    emb = torch.cat([pos * inv, pos * inv], dim=-1)
    cos, sin = emb.cos().to(bf)[None], emb.sin().to(bf)[None]
    gq = torch.randn(1, S, Hq, D, generator=g, device=dev).to(bf)
    gk = torch.randn(1, S, Hkv, D, generator=g, device=dev).to(bf)
    _, _, rstd = rope.norm_rope_forward(q, k, qw, kw, cos, sin, 1e-6)
    # one launch of tens of microseconds: time it inside a HIP graph, so the
    # host's argument checks and allocations between launches are not counted
    t_f = graph_time(torch, lambda: rope.norm_rope_forward(q, k, qw, kw, cos, sin, 1e-6), 20)
    t_b = graph_time(torch, lambda: rope.norm_rope_backward(q, k, qw, kw, cos, sin, rstd, gq, gk), 20)
    t_f_eager = timer(lambda: rope.norm_rope_forward(q, k, qw, kw, cos, sin, 1e-6), n)
    rows = S * (Hq + Hkv)
    table = 2 * S * D * 2                       # cos and sin rows
    fwd_bytes = 2 * rows * D * 2 + rows * 4 + table
    bwd_bytes = 3 * rows * D * 2 + rows * 4 + table
    fwd_gbps = fwd_bytes / (t_f * 1e-3) / 1e9
    bwd_gbps = bwd_bytes / (t_b * 1e-3) / 1e9

    def reference_ops(qx, kx, c, s_, wq, wk):
        def norm(x, w):
            xf = x.float()
            xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
            return w * xf.to(x.dtype)

        def rot(x):
            return torch.cat((-x[..., D // 2:], x[..., :D // 2]), dim=-1)
        qn, kn = norm(qx, wq).transpose(1, 2), norm(kx, wk).transpose(1, 2)
        c, s_ = c.unsqueeze(1), s_.unsqueeze(1)
        return qn * c + rot(qn) * s_, kn * c + rot(kn) * s_

    def eager_step(qx, kx, c, s_, wq, wk, go_q, go_k):
        qx = qx.detach().requires_grad_()
        kx = kx.detach().requires_grad_()
        eq, ek = reference_ops(qx, kx, c, s_, wq, wk)
        torch.autograd.backward([eq, ek], [go_q.transpose(1, 2), go_k.transpose(1, 2)])

    t_eager = timer(lambda: eager_step(q, k, cos, sin, qw, kw, gq, gk), n)

    # the chunk's keys and values into the KV cache rows [P, P + S) of a
    # layer: norm / RoPE, then the cache update's copy of K and V, against the
    # one launch that writes the post-RoPE keys and the values into the rows
    ops = import_module("mtp-glora_amd.ops")
    v = torch.randn(1, S, Hkv, D, generator=g, device=dev).to(bf)
    Pc = 8192
    kbuf = torch.empty(Hkv, Pc + S, D, device=dev, dtype=bf)
    vbuf = torch.empty(Hkv, Pc + S, D, device=dev, dtype=bf)

    def copy_path():
        _, ko, _ = rope.norm_rope_forward(q, k, qw, kw, cos, sin, 1e-6)
        ops.kv_append(ko.transpose(1, 2), v.transpose(1, 2), kbuf, vbuf, dst_offset=Pc)

    def fused_path():
        rope.norm_rope_stage_forward(q, k, v, qw, kw, cos, sin, 1e-6, kbuf[None, :, Pc:], vbuf[None, :, Pc:])

    t_copy = graph_time(torch, copy_path, 20)
    t_fused = graph_time(torch, fused_path, 20)
    kv_rows = S * Hkv * D * 2
    stage = {"prefix": Pc, "copy_path_ms": round(t_copy, 5), "fused_ms": round(t_fused, 5),
             "bytes_copy_path": fwd_bytes + 4 * kv_rows, "bytes_fused": fwd_bytes + 2 * kv_rows,
             "launches_copy_path": 2, "launches_fused": 1,
             "what": "norm/RoPE of q and k with the chunk's K and V staged into the cache rows [P, P+S): "
                     "norm_rope_forward + kv_append (post-RoPE K written, read back and written again, V "
                     "read and written) against mga_qk_norm_rope_stage_fwd (K written once into the rows, "
                     "V copied in the same launch)"}
    args_cpu = [t_[:, :cpu_tokens].cpu() if t_.dim() == 4 else t_.cpu() for t_ in (q, k)]
    c_cpu, s_cpu = cos[:, :cpu_tokens].cpu(), sin[:, :cpu_tokens].cpu()
    secs = []
    for _ in range(4):
        t0 = time.perf_counter()
        eager_step(args_cpu[0], args_cpu[1], c_cpu, s_cpu, qw.cpu(), kw.cpu(), gq[:, :cpu_tokens].cpu(),
                   gk[:, :cpu_tokens].cpu())
        secs.append(time.perf_counter() - t0)
    cpu_s = sorted(secs[1:])[1]
    return {"tokens": S, "Hq": Hq, "Hkv": Hkv, "head_dim": D, "dtype": "bf16",
            "fwd_ms": round(t_f, 5), "bwd_ms": round(t_b, 5),
            "fwd_GBps": round(fwd_gbps, 1), "bwd_GBps": round(bwd_gbps, 1),
            "fwd_frac": round(fwd_gbps / PEAK_HBM_GBPS, 4), "bwd_frac": round(bwd_gbps / PEAK_HBM_GBPS, 4),
            "peak": PEAK_HBM_GBPS, "bytes": {"fwd": fwd_bytes, "bwd": bwd_bytes},
            "fwd_ms_eager_launches": round(t_f_eager, 5), "cache_stage": stage,
            "torch_eager_gpu_fwd_bwd_ms": round(t_eager, 4),
            "cpu_tokens_per_s": round(cpu_tokens / cpu_s, 1),
            "gpu_tokens_per_s": round(S / ((t_f + t_b) * 1e-3), 1),
            "cpu_sample": f"the reference's ops as torch eager bf16 on the CPU, fwd + bwd, {cpu_tokens} tokens, "
                          f"median of 3 after a warm-up, {torch.get_num_threads()} threads"}


def gated_lora_phase(torch, timer, S: int, K: int, N: int, rank: int, p: float, n: int, cpu_rows: int) -> dict:
    """The gated LoRA layer (GatedLoRALinear, gated_lora.py:51-53) at Qwen3-8B's
    fused qkv_proj with the reference's training ranks and dropout: forward and
    backward of the fused layer, the base GEMM alone (the floor any layout
    pays), and the reference's torch ops on the same GPU and on the CPU."""
    from importlib import import_module
    lm = import_module("mtp-glora_amd.lora")
    F = torch.nn.functional
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(SEED + 11)
    bf = torch.bfloat16
    x = torch.randn(S, K, generator=g, device=dev).to(bf)
    W = (torch.randn(N, K, generator=g, device=dev) / K ** 0.5).to(bf)
    A = (torch.randn(rank, K, generator=g, device=dev) / K ** 0.5).to(bf)
    B = (torch.randn(N, rank, generator=g, device=dev) * 0.05).to(bf)
    gate = (torch.rand(S, generator=g, device=dev) < 0.8).float()
    dy = torch.randn(S, N, generator=g, device=dev).to(bf)
    scaling = 2.0
    y, t, h = lm.gated_lora_forward(x, W, A, B, gate, scaling, p, 7)
    t_f = timer(lambda: lm.gated_lora_forward(x, W, A, B, gate, scaling, p, 7), n)
    t_b = timer(lambda: lm.gated_lora_backward(dy, x, h, t, W, A, B, gate, scaling, p, 7, True, True, True), n)
    t_gemm = timer(lambda: F.linear(x, W), n)

    def reference(xx, go):
        # GatedLoRALinear.forward as the reference runs it, then autograd
        xr = xx.detach().requires_grad_()
        Ar, Br = A.detach().requires_grad_(), B.detach().requires_grad_()
        out = F.linear(xr, W) + scaling * F.linear(F.linear(F.dropout(xr, p, True), Ar), Br) * gate[:xx.shape[0], None]
        out.backward(go)

    t_ref = timer(lambda: reference(x, dy), n)
    fl_fwd = 2.0 * S * K * N + 2.0 * S * rank * (K + N)
    fl_bwd = 2.0 * S * K * N + 4.0 * S * rank * (K + N)
    xc, dyc = x[:cpu_rows].cpu(), dy[:cpu_rows].cpu()
    W_c, A_c, B_c, g_c = W.cpu(), A.cpu(), B.cpu(), gate.cpu()
    secs = []
    for _ in range(3):
        t0 = time.perf_counter()
        xr = xc.detach().requires_grad_()
        Ar, Br = A_c.detach().requires_grad_(), B_c.detach().requires_grad_()
        out = F.linear(xr, W_c) + scaling * F.linear(F.linear(F.dropout(xr, p, True), Ar), Br) * g_c[:cpu_rows, None]
        out.backward(dyc)
        secs.append(time.perf_counter() - t0)
    cpu_s = sorted(secs[1:])[0]
    # HIP kernels' algorithmic bytes: the down-projection reads x and writes t
    # (no dropout output is kept); the dX term is written once; grad_A reads x
    # again (and d_a) to draw the mask
    rp = (rank + 31) // 32 * 32
    down_bytes = S * K * 2 + S * rp * 2
    dx_bytes = S * K * 2 if p > 0 else 0
    da_bytes = S * K * 2 + S * rp * 2 + rank * K * 2 if p > 0 else 0
    return {"S": S, "in": K, "out": N, "rank": rank, "dropout": p, "dtype": "bf16",
            "fwd_ms": round(t_f, 4), "bwd_ms": round(t_b, 4), "base_gemm_ms": round(t_gemm, 4),
            "fwd_tflops": round(fl_fwd / (t_f * 1e-3) / 1e12, 1), "bwd_tflops": round(fl_bwd / (t_b * 1e-3) / 1e12, 1),
            "base_gemm_tflops": round(2.0 * S * K * N / (t_gemm * 1e-3) / 1e12, 1),
            "fwd_over_base_gemm": round(t_f / t_gemm, 3),
            "torch_eager_gpu_fwd_bwd_ms": round(t_ref, 4),
            "kernel_bytes": {"lora_down_kernel": down_bytes, "lora_dx_kernel": dx_bytes, "lora_da_kernel": da_bytes},
            "cpu_rows_per_s": round(cpu_rows / cpu_s, 1), "gpu_rows_per_s": round(S / ((t_f + t_b) * 1e-3), 1),
            "cpu_sample": f"the reference's ops as torch eager bf16 on the CPU, fwd + bwd, {cpu_rows} rows, "
                          f"best of 2 after a warm-up, {torch.get_num_threads()} threads"}


def graph_time(torch, fn, n: int, reps: int = 5) -> float:
    """Average duration of ``fn`` captured ``n`` times into one HIP graph
    (removes host launch gaps from microsecond kernels)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(n):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st = torch.cuda.current_stream()
    e0.record(st)
    for _ in range(reps):
        g.replay()
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) / (n * reps)


def cpu_compiled_fwd(torch, fr, q, k, v, bm, scale: float, reps: int) -> dict:
    """torch.compile(flex_attention) on the CPU, forward only: Inductor's CPU
    flex kernel serves inference only (it refuses the LSE output and the
    backward, [torch]_inductor/kernel/flex/flex_cpu.py:71-74), so this figure
    is an inference-only forward, not the reference's training path. Compiled
    in this process (compile_threads = 1: no worker pool is started)."""
    import torch._inductor.config as icfg
    from torch.nn.attention.flex_attention import flex_attention
    icfg.compile_threads = 1
    fn = torch.compile(flex_attention)
    with torch.no_grad():
        t0 = time.perf_counter()
        fn(q, k, v, block_mask=bm, scale=scale, enable_gqa=True)   # compile + first run
        compile_s = time.perf_counter() - t0
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn(q, k, v, block_mask=bm, scale=scale, enable_gqa=True)
            times.append(time.perf_counter() - t0)
    return dict(seconds=statistics.median(times), compile_s=compile_s)


def cpu_baseline(cfg: dict, gate_cpu, reps: int, heads: int, compiled: bool, groups: int = 1) -> dict:
    """The reference's CPU attention path over ``groups`` KV-head groups of
    ``heads`` query heads each, one after another (the eager dense path
    materialises fp32 [heads, S, P+S] scores, so one group at a time), each
    with its own inputs: ``reps`` passes over the groups after a warm-up call,
    ``seconds`` = the median pass's total. With ``compiled``, the compiled
    inference-only forward on the first group's inputs."""
    import torch
    from oracle import flex_ref as fr
    threads = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(threads)
    P, D = cfg["P"], cfg["D"]
    S = gate_cpu.shape[1]
    L = P + S
    t0 = time.perf_counter()
    bm = fr.reference_block_mask(gate_cpu, P)
    mask_s = time.perf_counter() - t0
    data = []
    for grp in range(groups):
        g = torch.Generator().manual_seed(SEED + 100 * grp)
        data.append(((torch.randn(1, heads, S, D, generator=g) * 0.5).bfloat16(),
                     (torch.randn(1, 1, L, D, generator=g) * 0.5).bfloat16(),
                     (torch.randn(1, 1, L, D, generator=g) * 0.5).bfloat16(),
                     torch.randn(1, heads, S, D, generator=g).bfloat16()))
    q, k, v, do = data[0]
    import warnings
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        fr.reference_attention(q, k, v, bm, D ** -0.5, do=do)          # warm-up
        times = []
        for _ in range(reps):
            total = 0.0
            for qg, kg, vg, dog in data:
                t0 = time.perf_counter()
                fr.reference_attention(qg, kg, vg, bm, D ** -0.5, do=dog)
                total += time.perf_counter() - t0
            times.append(total)
    comp = None
    if compiled:
        try:
            comp = cpu_compiled_fwd(torch, fr, q, k, v, bm, D ** -0.5, reps)
        except Exception as e:   # an Inductor CPU toolchain problem leaves the eager figure standing
            comp = dict(error=f"{type(e).__name__}: {str(e)[:200]}")
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return dict(seconds=statistics.median(times), times=times, mask_build_s=mask_s, compiled=comp,
                threads=torch.get_num_threads(), cpu_count=os.cpu_count(), cpu_model=model)


# bench phase -> kernel whose counters stand for it in the traffic summary
PHASE_KERNEL = {"fwd": "attn_fwd_kernel", "bwd_dq_pass": "attn_bwd_dq_kernel",
                "bwd_dkdv_pass": "attn_bwd_dkdv_kernel", "append_commit": "kv_copy_rows_kernel"}
CALIB_ROWS = 65536   # rows per head of the calibration copy (8 heads x 256 B x 2 tensors = 268 MB)


def load_mfma(path: str) -> dict:
    """Per attention kernel: MFMA-busy fraction and the MFMA work the counters
    saw over the credited work, from a committed counter summary
    (rocprof_summary.py mfma), or {}."""
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return {}
    out = {}
    for k, e in t.get("kernels", {}).items():
        out[k] = {n: round(e[n], 4) for n in ("mfma_busy_frac", "mfma_flop_over_credited", "valu_per_mfma",
                                             "salu_per_mfma", "lds_per_mfma") if n in e}
    return out


def layer_step_phase(torch, mga, syn, geo: dict, steps: int, warmup: int, seed: int) -> dict:
    """One layer-chunk step at geometry ``geo`` (a CONFIGS entry), timed as the
    main step is: block mask, staging append, attention forward and backward,
    regular-row commit, the cache cropped back to the same prefix."""
    dev = torch.device("cuda:0")
    Hq, Hkv, D, P = geo["Hq"], geo["Hkv"], geo["D"], geo["P"]
    n_reg, n_anchor, draft = geo["n_reg"], geo["n_anchor"], geo["draft"]
    if geo["every"]:
        anchors = syn.every_kth_anchor(n_reg, geo["every"], n_anchor)
    else:
        anchors = syn.sample_anchors(n_reg, n_anchor, seed)
    chunk0 = syn.mtp_chunk(n_reg, anchors, draft, pos0=P, device=dev, seed=seed)
    S = chunk0["gate_mask"].shape[1]
    L = P + S
    scale = D ** -0.5
    gens = [torch.Generator(device=dev).manual_seed(seed * 10 + i) for i in range(6)]
    rnd = lambda shape, g, sd: (torch.randn(*shape, generator=g, device=dev) * sd).bfloat16()
    q = rnd((1, S, Hq, D), gens[0], 0.5).transpose(1, 2).requires_grad_()
    k = rnd((1, S, Hkv, D), gens[1], 0.5).transpose(1, 2).requires_grad_()
    v = rnd((1, S, Hkv, D), gens[2], 0.5).transpose(1, 2).requires_grad_()
    do = rnd((1, S, Hq, D), gens[5], 1.0)
    mgr = mga.StreamingKVCacheManager(capacity=L + 256, sanity_check=False)
    cache = mgr.new_cache(num_layers=1)
    cache.append_prefix([rnd((1, Hkv, P, D), gens[3], 0.5)], [rnd((1, Hkv, P, D), gens[4], 0.5)])
    mgr.past_seen_tokens = P
    module = torch.nn.Module()

    def step():
        chunk = mgr.prepare_data_with_kv_cache(dict(chunk0))
        kf, vf = cache.update(k, v, 0)
        o, _ = mga.mtp_attention_forward(module, q, kf, vf, chunk["attention_mask"], scaling=scale)
        grads = torch.autograd.grad(o, (q, k, v), do)
        mgr.extract_regular_kv_cache_for_next_chunk(chunk, cache)
        cache.crop(P)
        mgr.past_seen_tokens = P
        return grads

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    bm = mga.build_mtp_block_mask(chunk0["gate_mask"], P)
    a_pre, a_cur = tile_areas(bm, S, L, P)
    fl = Hq * D * (4 * (a_pre + a_cur) + 6 * a_pre + 10 * a_cur)
    tf = fl / (ms * 1e-3) / 1e12

    # the three attention passes on their own (HIP events on the launch stream)
    lib_ops = mga.ops
    libc = importlib.import_module("mtp-glora_amd._lib")
    kbuf, vbuf = cache.key_buffer(0), cache.value_buffer(0)
    code, bmt = bm.mtp_code, bm.kernel_tensors()
    kf, vf = kbuf[None, :, :L], vbuf[None, :, :L]
    lib_ops.kv_append(k.detach(), v.detach(), kbuf, vbuf, dst_offset=P)
    qd = q.detach()
    o, lse = lib_ops.attn_fwd(qd, kf, vf, code, bmt, P, scale)
    bufs = lib_ops.bwd_buffers(qd, kf, P)
    timer = EventTimer(torch)
    n = max(steps, 5)
    t_fwd = timer(lambda: lib_ops.attn_fwd(qd, kf, vf, code, bmt, P, scale), n)
    t_dq = timer(lambda: lib_ops.attn_bwd(qd, kf, vf, o, lse, do, code, bmt, P, scale, P,
                                          passes=libc.BWD_DQ, buffers=bufs), n)
    t_dkdv = timer(lambda: lib_ops.attn_bwd(qd, kf, vf, o, lse, do, code, bmt, P, scale, P,
                                            passes=libc.BWD_DKDV, buffers=bufs), n)
    passes = {}
    for name, t, f in (("fwd", t_fwd, 4 * (a_pre + a_cur)), ("bwd_dq_pass", t_dq, 6 * (a_pre + a_cur)),
                       ("bwd_dkdv_pass", t_dkdv, 4 * a_cur)):
        pt = Hq * D * f / (t * 1e-3) / 1e12
        passes[name] = {"ms": round(t, 4), "tflops": round(pt, 1), "frac": round(pt / PEAK_MFMA_BF16_TFLOPS, 4)}
    return {"chunk_rows": S, "prefix": P, "credited_gflop": round(fl / 1e9, 1), "ms_per_step": round(ms, 4),
            "tflops": round(tf, 2), "frac": round(tf / PEAK_MFMA_BF16_TFLOPS, 4), "steps": steps,
            "passes": passes}


# config 3's last chunk: the north-star point
NORTH_STAR = dict(Hq=32, Hkv=8, D=128, P=28672, n_reg=4096, n_anchor=512, draft=4, every=None)


def north_star_phase(torch, mga, syn, steps: int, warmup: int) -> dict:
    """The north-star point: one Qwen3-8B layer-chunk of 4096 regular rows plus
    512 anchors x 4 mask rows (S = 6144) against a 28 672-token cached prefix
    (config 3's last chunk)."""
    out = {"workload": "north-star point: Qwen3-8B layer-chunk, 4096 regular + 512x4 mask rows vs a "
                       "28672-token prefix (config 3, last chunk)"}
    out.update(layer_step_phase(torch, mga, syn, NORTH_STAR, steps, warmup, SEED + 7))
    out["target_frac"] = 0.5
    return out


def load_traffic(path: str, config: int):
    """HBM bytes per launch per kernel from a committed counter summary
    (FETCH_SIZE + WRITE_SIZE scaled by the calibration copy), or None."""
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("config") != config:
        return None
    return {k: v["traffic_bytes"] for k, v in t.get("kernels", {}).items()}


def pmc_pass(torch, mga, libc, q, k, v, do, kp, cache, chunk0, P, S, R, Hkv, D, scale) -> int:
    """One launch of each kernel for a hardware-counter run, preceded by a
    calibration copy of known size (the append kernel, contiguous rows)."""
    ops = mga.ops
    dev = q.device
    src = torch.randn(Hkv, CALIB_ROWS, D, device=dev).bfloat16()
    dst_k = torch.empty_like(src)
    dst_v = torch.empty_like(src)
    torch.cuda.synchronize()
    ops.kv_append(src, src, dst_k, dst_v, dst_offset=0)            # calibration copy
    torch.cuda.synchronize()
    L = P + S
    kbuf, vbuf = cache.key_buffer(0), cache.value_buffer(0)
    bm = mga.build_mtp_block_mask(chunk0["gate_mask"], P)
    kbuf[:, P:L].copy_(k.detach()[0])     # torch copies: the append kernel runs only as
    vbuf[:, P:L].copy_(v.detach()[0])     # the calibration copy and the commit below
    kf, vf = kbuf[None, :, :L], vbuf[None, :, :L]
    code, bmt = bm.mtp_code, bm.kernel_tensors()
    qd = q.detach()
    o, lse = ops.attn_fwd(qd, kf, vf, code, bmt, P, scale)
    bufs = ops.bwd_buffers(qd, kf, P)
    ops.attn_bwd(qd, kf, vf, o, lse, do, code, bmt, P, scale, P, passes=libc.BWD_DQ, buffers=bufs)
    ops.attn_bwd(qd, kf, vf, o, lse, do, code, bmt, P, scale, P, passes=libc.BWD_DKDV, buffers=bufs)
    idx, cnt = ops.regular_index(chunk0["regular_token_mask"])
    app_k = torch.empty(Hkv, R + 16, D, dtype=torch.bfloat16, device=dev)
    app_v = torch.empty_like(app_k)
    ops.kv_append(k.detach(), v.detach(), app_k, app_v, dst_offset=0, idx=idx, n_rows=R)
    lossmod = importlib.import_module("mtp-glora_amd.loss")
    xs = torch.randn(1, 256, QWEN3_VOCAB, device=dev).bfloat16()
    ts = torch.randn(1, 256, QWEN3_VOCAB, device=dev).bfloat16()
    _, st = lossmod.soft_ce_forward(xs, ts)
    lossmod.soft_ce_backward(xs, ts, st, torch.ones((), device=dev))
    rope = importlib.import_module("mtp-glora_amd.rope")
    Hq = q.shape[1]
    qr_ = torch.randn(1, S, Hq, D, device=dev).bfloat16()
    kr_ = torch.randn(1, S, Hkv, D, device=dev).bfloat16()
    wr_ = torch.ones(D, device=dev).bfloat16()
    cr_ = torch.ones(1, S, D, device=dev).bfloat16()
    _, _, rs_ = rope.norm_rope_forward(qr_, kr_, wr_, wr_, cr_, cr_, 1e-6)
    gq_, gk_ = torch.randn_like(qr_), torch.randn_like(kr_)   # gradients: their own memory
    rope.norm_rope_backward(qr_, kr_, wr_, wr_, cr_, cr_, rs_, gq_, gk_)
    lm = importlib.import_module("mtp-glora_amd.lora")
    Kl, Nl = Hq * D, (Hq + 2 * Hkv) * D
    xl = torch.randn(S, Kl, device=dev).bfloat16()
    Wl = torch.randn(Nl, Kl, device=dev).bfloat16()
    Al = torch.randn(96, Kl, device=dev).bfloat16()
    Bl = torch.randn(Nl, 96, device=dev).bfloat16()
    gl_ = torch.ones(S, device=dev)
    _, tl, hl = lm.gated_lora_forward(xl, Wl, Al, Bl, gl_, 2.0, 0.05, 7)
    lm.gated_lora_backward(torch.randn(S, Nl, device=dev).bfloat16(), xl, hl, tl, Wl, Al, Bl, gl_, 2.0, 0.05, 7,
                           True, True, True)
    torch.cuda.synchronize()
    calib = Hkv * CALIB_ROWS * D * 2 * 2
    a_pre, a_cur = tile_areas(bm, S, L, P)
    credited = {"attn_fwd_kernel": Hq * D * 4 * (a_pre + a_cur),
                "attn_bwd_dq_kernel": Hq * D * 6 * (a_pre + a_cur),
                "attn_bwd_dkdv_kernel": Hq * D * 4 * a_cur}
    print(json.dumps({"pmc_pass": True, "calibration": {"kernel": "kv_copy_rows_kernel",
                                                        "read_bytes": calib, "write_bytes": calib,
                                                        "grid_rows": CALIB_ROWS},
                      "credited_flop": credited}), flush=True)
    return 0


def stream_measure(torch, mga, syn, cfg: dict) -> dict:
    """Time one whole chunk stream (all layers, all chunks) through the
    drop-in API after a one-chunk warm-up; credited FLOPs per chunk from that
    chunk's block mask, times the layer count."""
    dev = torch.device("cuda:0")
    Hq, Hkv, D, nl = cfg["Hq"], cfg["Hkv"], cfg["D"], cfg["layers"]
    scale = D ** -0.5
    chunks, P = [], 0
    for c, (n_reg, n_anchor, draft) in enumerate(cfg["chunks"]):
        anchors = syn.sample_anchors(n_reg, n_anchor, SEED + c)
        chunks.append(syn.mtp_chunk(n_reg, anchors, draft, pos0=P, device=dev, seed=SEED + c))
        P += n_reg
    Smax = max(ch["gate_mask"].shape[1] for ch in chunks)
    cap = P + Smax + 256
    g = torch.Generator(device=dev).manual_seed(SEED)
    rnd = lambda shape, sd: (torch.randn(*shape, generator=g, device=dev) * sd).bfloat16()
    # one set of projections per chunk length, shared by the layers (values do not affect time)
    tens = {}
    for ch in chunks:
        S = ch["gate_mask"].shape[1]
        if S not in tens:
            tens[S] = (rnd((1, S, Hq, D), 0.5).transpose(1, 2).requires_grad_(),
                       rnd((1, S, Hkv, D), 0.5).transpose(1, 2).requires_grad_(),
                       rnd((1, S, Hkv, D), 0.5).transpose(1, 2).requires_grad_(),
                       rnd((1, S, Hq, D), 1.0))
    mgr = mga.StreamingKVCacheManager(capacity=cap, sanity_check=False)
    module = torch.nn.Module()

    def run(nchunks):
        mgr.reset_cache()
        cache = mgr.new_cache(num_layers=nl)
        for c in range(nchunks):
            chunk = mgr.prepare_data_with_kv_cache(dict(chunks[c]))
            q, k, v, do = tens[chunk["input_ids"].shape[1]]
            for layer in range(nl):
                kf, vf = cache.update(k, v, layer)
                o, _ = mga.mtp_attention_forward(module, q, kf, vf, chunk["attention_mask"], scaling=scale)
                torch.autograd.grad(o, (q, k, v), do)
            if c + 1 < len(chunks):
                cache = mgr.extract_regular_kv_cache_for_next_chunk(chunk, cache)

    run(1)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    run(len(chunks))
    e1.record()
    torch.cuda.synchronize()
    host_s = time.perf_counter() - t0
    seconds = e0.elapsed_time(e1) / 1e3

    credited, append_bytes, P = 0, 0, 0
    for c, ch in enumerate(chunks):
        S = ch["gate_mask"].shape[1]
        bm = mga.build_mtp_block_mask(ch["gate_mask"], P)
        a_pre, a_cur = tile_areas(bm, S, P + S, P)
        credited += nl * Hq * D * (4 * (a_pre + a_cur) + 6 * a_pre + 10 * a_cur)
        R = int(ch["regular_token_mask"].sum())
        if c + 1 < len(chunks):
            append_bytes += nl * 2 * R * Hkv * D * 2 * 2
        P += R
    tflops = credited / seconds / 1e12
    return dict(chunks=chunks, credited=credited, seconds=seconds, host_s=host_s, append_bytes=append_bytes,
                final_prefix=P, tflops=tflops)


def stream_bench(torch, mga, syn, config: int, cfg: dict, cpu_reps: int = 0) -> int:
    """The stream of ``cfg`` as the bench line (``--config 3`` / ``4``), with
    the CPU baseline sampled at three of its chunks."""
    Hq, Hkv, D, nl = cfg["Hq"], cfg["Hkv"], cfg["D"], cfg["layers"]
    m = stream_measure(torch, mga, syn, cfg)
    chunks, credited, seconds, tflops, P = m["chunks"], m["credited"], m["seconds"], m["tflops"], m["final_prefix"]
    host_s, append_bytes = m["host_s"], m["append_bytes"]
    cpu = None
    if cpu_reps > 0:
        # the reference's CPU path at the stream's first, middle and last chunk
        # of one layer, one query head (of one KV-head group), extrapolated
        samples, P_c = [], 0
        picks = sorted({0, len(chunks) // 2, len(chunks) - 1})
        for c, ch in enumerate(chunks):
            S_c = ch["gate_mask"].shape[1]
            if c in picks:
                bm_c = mga.build_mtp_block_mask(ch["gate_mask"], P_c)
                a_pre, a_cur = tile_areas(bm_c, S_c, P_c + S_c, P_c)
                fl_layer = Hq * D * (4 * (a_pre + a_cur) + 6 * a_pre + 10 * a_cur)
                cb = cpu_baseline(dict(P=P_c, D=D), ch["gate_mask"].cpu(), cpu_reps, 1, False)
                samples.append({"chunk": c, "prefix": P_c, "rows": S_c, "seconds_one_head": round(cb["seconds"], 3),
                                "tflops": round(fl_layer / Hq / cb["seconds"] / 1e12, 4)})
                threads = cb["threads"]
            P_c += int(ch["regular_token_mask"].sum())
        rate = statistics.mean(x["tflops"] for x in samples)
        cpu = {"value": round(rate, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
               "sample": (f"torch flex_attention eager fwd+bwd on CPU (restated MTP mask_mod), one query head of "
                          f"one layer at chunks {picks} of the stream, median of {cpu_reps} runs each; value = the "
                          f"mean of their credited-FLOP rates"),
               "extrapolated": (f"x{Hq} heads, x{nl} layers, all {len(chunks)} chunks at the mean rate: "
                                f"{credited / (rate * 1e12):.0f} s for the stream"),
               "chunks": samples}
    out = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": 1,
        "warmup": 1, "ms_per_step": round(seconds * 1e3, 2), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": cfg["workload"], "Hq": Hq, "Hkv": Hkv, "head_dim": D, "layers": nl,
                   "chunks": len(chunks), "final_prefix": P, "seed": SEED},
        "stream": {"credited_tflop": round(credited / 1e12, 2), "seconds": round(seconds, 4),
                   "host_seconds": round(host_s, 4), "append_bytes": append_bytes,
                   "roofline_frac": round(tflops / PEAK_MFMA_BF16_TFLOPS, 4),
                   "step": "per chunk: block mask; per layer: cache update, attention fwd, bwd; "
                           "then the regular-row commit of every layer (not after the last chunk)"},
    }
    if cpu is not None:
        out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2, choices=sorted(set(CONFIGS) | set(STREAMS)))
    ap.add_argument("--cpu-reps", type=int, default=1,
                    help="timed passes of the CPU baseline over the layer's KV-head groups (0 = skip)")
    ap.add_argument("--cpu-compiled", type=int, default=1,
                    help="also time the compiled (inference-only) CPU forward on the same sample (0 = skip)")
    ap.add_argument("--phase-iters", type=int, default=20)
    ap.add_argument("--pmc-pass", action="store_true",
                    help="for hardware-counter runs: one known-size calibration copy, then one launch "
                         "of each hot-path kernel; prints their byte counts and exits")
    ap.add_argument("--traffic", default=str(ROOT / "profiles" / "config2_traffic.json"),
                    help="counter summary (from rocprof_summary.py) that fills roofline.traffic")
    ap.add_argument("--mfma", default=str(ROOT / "profiles" / "config2_mfma.json"),
                    help="counter summary (rocprof_summary.py mfma) that fills roofline.mfma_busy")
    ap.add_argument("--north-star-steps", type=int, default=10,
                    help="timed steps of the north-star point (0 = skip)")
    ap.add_argument("--north-star-only", action="store_true",
                    help="time the north-star point alone (for a kernel trace of that workload); with "
                         "--pmc-pass, run the counter pass at that point")
    ap.add_argument("--extra", type=int, default=1,
                    help="also time the config-3 stream (36 layers x 8 chunks) and the config-5 step (0 = skip)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build's hot path (streaming KV cache + MTP "
              "attention) runs per GPU with no collectives; multi-GPU runs are not part of it.",
              file=sys.stderr)
        return 2

    import torch
    mga = importlib.import_module("mtp-glora_amd")
    from importlib import import_module
    syn = import_module("mtp-glora_amd.synthetic")
    lib_ops = mga.ops
    libc = import_module("mtp-glora_amd._lib")
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    mga.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.config in STREAMS:
        return stream_bench(torch, mga, syn, args.config, STREAMS[args.config], args.cpu_reps)
    if args.north_star_only and not args.pmc_pass:
        print(json.dumps({"north_star": north_star_phase(torch, mga, syn, max(args.north_star_steps, 1), 3)}))
        return 0

    # (--pmc-pass --north-star-only: the counter pass at the north-star point)
    cfg = NORTH_STAR if args.north_star_only else CONFIGS[args.config]
    Hq, Hkv, D, P = cfg["Hq"], cfg["Hkv"], cfg["D"], cfg["P"]
    n_reg = cfg["n_reg"]
    if cfg["every"]:
        anchors = syn.every_kth_anchor(n_reg, cfg["every"], cfg["n_anchor"])
    else:
        anchors = syn.sample_anchors(n_reg, cfg["n_anchor"], SEED)
    chunk0 = syn.mtp_chunk(n_reg, anchors, cfg["draft"], pos0=P, device=dev, seed=SEED)
    S = chunk0["gate_mask"].shape[1]
    L = P + S
    R = int(chunk0["regular_token_mask"].sum())
    scale = D ** -0.5

    gens = [torch.Generator(device=dev).manual_seed(SEED + i) for i in range(6)]
    rnd = lambda shape, g, s: (torch.randn(*shape, generator=g, device=dev) * s).bfloat16()
    # projection layout [1, S, H, D] seen as [1, H, S, D], as the adapters pass them
    q = rnd((1, S, Hq, D), gens[0], 0.5).transpose(1, 2).requires_grad_()
    k = rnd((1, S, Hkv, D), gens[1], 0.5).transpose(1, 2).requires_grad_()
    v = rnd((1, S, Hkv, D), gens[2], 0.5).transpose(1, 2).requires_grad_()
    kp = rnd((1, Hkv, P, D), gens[3], 0.5)
    vp = rnd((1, Hkv, P, D), gens[4], 0.5)
    do = rnd((1, S, Hq, D), gens[5], 1.0)

    mgr = mga.StreamingKVCacheManager(capacity=L + 256, sanity_check=False)
    cache = mgr.new_cache(num_layers=1)
    cache.append_prefix([kp], [vp])
    mgr.past_seen_tokens = P
    module = torch.nn.Module()

    def step():
        chunk = dict(chunk0)
        chunk = mgr.prepare_data_with_kv_cache(chunk)
        kf, vf = cache.update(k, v, 0)
        o, _ = mga.mtp_attention_forward(module, q, kf, vf, chunk["attention_mask"], scaling=scale)
        grads = torch.autograd.grad(o, (q, k, v), do)
        mgr.extract_regular_kv_cache_for_next_chunk(chunk, cache)
        cache.crop(P)
        mgr.past_seen_tokens = P
        return grads

    if args.pmc_pass:
        return pmc_pass(torch, mga, libc, q, k, v, do, kp, cache, chunk0, P, S, R, Hkv, D, scale)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_host = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    host_ms = (time.perf_counter() - t_host) * 1e3 / args.steps
    ms_per_step = e0.elapsed_time(e1) / args.steps

    # ---- credited work ------------------------------------------------------
    bm = mga.build_mtp_block_mask(chunk0["gate_mask"], P)
    a_pre, a_cur = tile_areas(bm, S, L, P)
    fl_fwd = Hq * D * 4 * (a_pre + a_cur)
    fl_dq = Hq * D * 6 * (a_pre + a_cur)
    fl_dkdv = Hq * D * 4 * a_cur
    fl_total = fl_fwd + fl_dq + fl_dkdv
    append_bytes = 2 * R * Hkv * D * 2 * 2        # read + write, K and V, bf16
    stage_bytes = 2 * S * Hkv * D * 2 * 2

    # ---- per-phase kernel timing (HIP events on the launch stream) ----------
    timer = EventTimer(torch)
    n = args.phase_iters
    kbuf, vbuf = cache.key_buffer(0), cache.value_buffer(0)
    code, bmt = bm.mtp_code, bm.kernel_tensors()
    kf = kbuf[None, :, :L]
    vf = vbuf[None, :, :L]
    lib_ops.kv_append(k.detach(), v.detach(), kbuf, vbuf, dst_offset=P)
    qd = q.detach()
    o, lse = lib_ops.attn_fwd(qd, kf, vf, code, bmt, P, scale)
    bufs = lib_ops.bwd_buffers(qd, kf, P)
    idx, cnt = lib_ops.regular_index(chunk0["regular_token_mask"])
    torch.cuda.synchronize()

    t_mask = timer(lambda: mga.build_mtp_block_mask(chunk0["gate_mask"], P), n)
    t_fwd = timer(lambda: lib_ops.attn_fwd(qd, kf, vf, code, bmt, P, scale), n)
    t_dq = timer(lambda: lib_ops.attn_bwd(qd, kf, vf, o, lse, do, code, bmt, P, scale, P,
                                          passes=libc.BWD_DQ, buffers=bufs), n)
    t_dkdv = timer(lambda: lib_ops.attn_bwd(qd, kf, vf, o, lse, do, code, bmt, P, scale, P,
                                            passes=libc.BWD_DKDV, buffers=bufs), n)
    app_dst = torch.empty(Hkv, R + 16, D, dtype=torch.bfloat16, device=dev)
    app_dst_v = torch.empty_like(app_dst)
    t_commit = graph_time(torch, lambda: lib_ops.kv_append(k.detach(), v.detach(), app_dst, app_dst_v,
                                                           dst_offset=0, idx=idx, n_rows=R), 50)
    t_stage = graph_time(torch, lambda: lib_ops.kv_append(k.detach(), v.detach(), kbuf, vbuf,
                                                          dst_offset=P), 50)
    torch.cuda.synchronize()

    phases = {"mask_build": t_mask, "fwd": t_fwd, "bwd_dq_pass": t_dq, "bwd_dkdv_pass": t_dkdv,
              "append_commit": t_commit, "append_stage": t_stage}
    soft_ce = soft_ce_phase(torch, mga, timer, int(anchors.numel()), QWEN3_VOCAB, n, cpu_rows=16)
    qk_rope = qk_rope_phase(torch, timer, S, Hq, Hkv, D, n, cpu_tokens=256)
    lora = gated_lora_phase(torch, timer, S, Hq * D, (Hq + 2 * Hkv) * D, 96, 0.05, n, cpu_rows=32)
    traffic = load_traffic(args.traffic, args.config)
    mfma = load_mfma(args.mfma) if args.config == 2 else {}
    credited = {"fwd": fl_fwd, "bwd_dq_pass": fl_dq, "bwd_dkdv_pass": fl_dkdv}
    dom = max(credited, key=lambda kname: phases[kname])
    attn_ms = t_fwd + t_dq + t_dkdv
    dom_tflops = credited[dom] / (phases[dom] * 1e-3) / 1e12
    commit_gbps = append_bytes / (t_commit * 1e-3) / 1e9

    out = {
        "metric": METRIC,
        "value": round(fl_total / (ms_per_step * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": cfg["workload"], "Hq": Hq, "Hkv": Hkv, "head_dim": D, "prefix": P,
                   "chunk_rows": S, "regular_rows": R, "anchors": int(anchors.numel()),
                   "draft_length": cfg["draft"], "seed": SEED},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(dom_tflops, 2),
                     "peak": PEAK_MFMA_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(dom_tflops / PEAK_MFMA_BF16_TFLOPS, 4),
                     "traffic": traffic.get(PHASE_KERNEL[dom]) if traffic else None,
                     "mfma_busy": mfma.get(PHASE_KERNEL[dom], {}).get("mfma_busy_frac")},
        "attention": {"credited_gflop": {"fwd": fl_fwd / 1e9, "bwd": (fl_dq + fl_dkdv) / 1e9,
                                         "total": fl_total / 1e9},
                      "tiles_area": {"prefix": a_pre, "chunk": a_cur},
                      "fwd_bwd_ms": round(attn_ms, 4),
                      "fwd_bwd_tflops": round(fl_total / (attn_ms * 1e-3) / 1e12, 2),
                      "fwd_bwd_frac": round(fl_total / (attn_ms * 1e-3) / 1e12 / PEAK_MFMA_BF16_TFLOPS, 4),
                      "fwd_tflops": round(fl_fwd / (t_fwd * 1e-3) / 1e12, 2),
                      "mfma_counters": ({PHASE_KERNEL[k_]: mfma.get(PHASE_KERNEL[k_]) for k_ in credited}
                                        if mfma else None),
                      "bwd_tflops": round((fl_dq + fl_dkdv) / ((t_dq + t_dkdv) * 1e-3) / 1e12, 2)},
        "append": {"bytes": append_bytes, "ms": round(t_commit, 5), "GBps": round(commit_gbps, 1),
                   "frac": round(commit_gbps / PEAK_HBM_GBPS, 4), "peak": PEAK_HBM_GBPS,
                   "stage_GBps": round(stage_bytes / (t_stage * 1e-3) / 1e9, 1)},
        "phases_ms": {kname: round(t, 5) for kname, t in phases.items()},
        "hbm_traffic_bytes": ({PHASE_KERNEL[k_]: traffic.get(PHASE_KERNEL[k_]) for k_ in PHASE_KERNEL}
                              if traffic else None),
        "soft_ce": soft_ce,
        "qk_norm_rope": qk_rope,
        "gated_lora_qkv": lora,
        "host_ms_per_step": round(host_ms, 4),
    }
    if args.north_star_steps > 0:
        out["north_star"] = north_star_phase(torch, mga, syn, args.north_star_steps, 3)
    if args.extra and args.config == 2:
        # config 3's whole stream and config 5's step, measured in the same run
        st = STREAMS[3]
        m = stream_measure(torch, mga, syn, st)
        out["config3_stream"] = {"workload": st["workload"], "credited_tflop": round(m["credited"] / 1e12, 2),
                                 "seconds": round(m["seconds"], 4), "tflops": round(m["tflops"], 2),
                                 "frac": round(m["tflops"] / PEAK_MFMA_BF16_TFLOPS, 4),
                                 "append_bytes": m["append_bytes"], "final_prefix": m["final_prefix"]}
        del m
        c5 = {"workload": CONFIGS[5]["workload"]}
        c5.update(layer_step_phase(torch, mga, syn, CONFIGS[5], 10, 3, SEED))
        out["config5_step"] = c5

    if args.cpu_reps > 0:
        G = Hq // Hkv
        cb = cpu_baseline(cfg, chunk0["gate_mask"].cpu(), args.cpu_reps, G, args.cpu_compiled, groups=Hkv)
        cpu_tflops = fl_total / cb["seconds"] / 1e12
        out["cpu_baseline"] = {
            "value": round(cpu_tflops, 4), "unit": "TFLOP/s", "cores": cb["threads"], "kind": "port",
            "sample": (f"the whole layer-chunk: torch flex_attention eager (dense math path) fwd+bwd on CPU "
                       f"with the restated MTP mask_mod, all {Hkv} KV-head groups of {G} query heads at the "
                       f"full S={S}, P+S={L}, one group after another (each its own inputs), summed; "
                       f"median of {args.cpu_reps} pass(es) after a warm-up call; no extrapolation"),
            "seconds": round(cb["seconds"], 3), "group_seconds": [round(t / Hkv, 3) for t in cb["times"]],
            "mask_build_s": round(cb["mask_build_s"], 3),
            "cpu_count": cb["cpu_count"], "cpu_model": cb["cpu_model"],
        }
        comp = cb["compiled"]
        if comp is not None:
            entry = {"label": ("inference-only: torch.compile(flex_attention) forward on the CPU, no LSE "
                               "and no backward (Inductor's CPU flex kernel refuses both), the first "
                               f"KV-head group's inputs and block mask, extrapolated x{Hkv} to the layer")}
            if "error" in comp:
                entry["error"] = comp["error"]
            else:
                entry.update({"value": round(fl_fwd / Hkv / comp["seconds"] / 1e12, 4), "unit": "TFLOP/s",
                              "seconds": round(comp["seconds"], 4), "compile_s": round(comp["compile_s"], 1),
                              "gpu_fwd_tflops": out["attention"]["fwd_tflops"]})
            out["cpu_baseline"]["compiled_fwd_only"] = entry
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
