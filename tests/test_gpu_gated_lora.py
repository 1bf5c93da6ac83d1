"""HIP / hipBLASLt gated LoRA layer (mga_gated_lora_*) against the float64
oracle (oracle/gated_lora.py, pinned by tests/test_oracle_gated_lora.py) on the
same bf16 inputs, the mask included.

Tolerances follow the bf16 roundings on each path (u = 2^-8 covers two
roundings of 2^-9):
* y: the rank-r term (whose activations t are rounded) is rounded, the base
  product accumulated onto it and the sum rounded:
  |y - y*| <= u (|y*| + |x W^T| + s g |h A^T| |B|^T) + 1e-5 max|y*|,
  plus, with dropout, the rounding of the dropout output h = T(x / (1 - p))
  carried through both products without cancellation: u/2 s g (|h| |A|^T) |B|^T
  (at rank 8 a few terms carry it and it alone exceeds the first bound);
* dX: the LoRA term goes through three roundings (u = dY B, d_a A, the
  dropout scaling), the base gradient dY W is accumulated onto it and the sum
  is rounded:
  |dX - dX*| <= u (|dX*| + |dY W| + 2 |d_a| |A| / (1 - p)) + 1e-5 max|dX*|;
* dA = d_a^T h and dB = dY^T t (sums over the S rows of rounded factors):
  |d - d*| <= u (|d*| + |a|^T |b|) with |a|^T |b| the sum of absolute products;
* the dropout output h equals the oracle's keep mask times T(x / (1 - p)) bit
  for bit.
The full Qwen3-8B qkv shape (S = 5120) is compared with an fp32 torch
reference on the GPU under the same bounds.

fp16 and fp32 layers (the reference's other model dtypes, args.py:15) run the
general path (hipBLASLt products in the layer's dtype, HIP dropout and row
scaling): the same bounds with u = 2^-10 for fp16; for fp32, u = 2^-18 and
the same u on the sums of absolute products, which covers fp32 accumulation
over K = 4096 terms.
"""
import importlib

import numpy as np
import pytest
import torch

from oracle import gated_lora as gl

pytestmark = pytest.mark.gpu
U = 2.0 ** -8
# rounding unit per dtype; ACC: the bound's factor on sums of absolute
# products (fp32 accumulation error), 0 where the roundings dominate
UNIT = {torch.bfloat16: (2.0 ** -8, 0.0), torch.float16: (2.0 ** -10, 0.0), torch.float32: (2.0 ** -18, 2.0 ** -18)}


def lora_mod():
    return importlib.import_module("mtp-glora_amd.lora")


def make(S, K, N, r, dev, seed=0, gate="mixed", dtype=torch.bfloat16):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(S, K, generator=g, device=dev).to(dtype)
    W = (torch.randn(N, K, generator=g, device=dev) / K ** 0.5).to(dtype)
    A = (torch.randn(r, K, generator=g, device=dev) / K ** 0.5).to(dtype)
    B = (torch.randn(N, r, generator=g, device=dev) * (0.5 / r ** 0.5)).to(dtype)
    gt = None if gate is None else (torch.rand(S, generator=g, device=dev) < 0.7).float()
    return x, W, A, B, gt


def f64(t):
    return None if t is None else t.detach().double().cpu().numpy()


def check(name, got, ref, bound):
    err = np.abs(got - ref)
    worst = (err / bound).max()
    print(f"  {name}: max-abs {err.max():.3e}, worst err/bound {worst:.3f}", flush=True)
    assert worst <= 1.0, name


def run_case(dev, S, K, N, r, p, gate="mixed", seed=0, scaling=2.0, dtype=torch.bfloat16):
    """The layer's own path (bf16: no dropout output kept when K is a multiple
    of 128, grad_A draws the mask again from x), checked against the oracle;
    with dropout on, also the path that keeps h: h bit for bit, the same y,
    and a grad_A over h that meets the same bound."""
    lm = lora_mod()
    U, ACC = UNIT[dtype]
    x, W, A, B, gt = make(S, K, N, r, dev, seed, gate, dtype)
    sd = 1234567 + seed
    y, t, h = lm.gated_lora_forward(x, W, A, B, gt, scaling, p, sd)
    assert h is None or K % 128 or p == 0 or dtype != torch.bfloat16
    assert (h is not None) == (p > 0) or dtype == torch.bfloat16
    dy = torch.randn(S, N, generator=torch.Generator(device=dev).manual_seed(seed + 7), device=dev).to(dtype)
    gx, ga, gb = lm.gated_lora_backward(dy, x, h, t, W, A, B, gt, scaling, p, sd, True, True, True)
    if p > 0:
        yk, tk, hk = lm.gated_lora_forward(x, W, A, B, gt, scaling, p, sd, keep_h=True)
        _, gak, _ = lm.gated_lora_backward(dy, x, hk, tk, W, A, B, gt, scaling, p, sd, False, True, False)
    torch.cuda.synchronize()
    X, Wn, An, Bn, G, DY = f64(x), f64(W), f64(A), f64(B), f64(gt), f64(dy)
    keep = gl.keep_mask(sd, S, K, p) if p > 0 else None
    if p > 0:   # the kernel's dropout output, bit for bit, and the same forward with or without it
        want = (keep * f64(x.float().mul(1.0 / (1.0 - p)).to(dtype)))
        np.testing.assert_array_equal(f64(hk), want)
        assert torch.equal(yk, y) and torch.equal(tk, t)
    Gv = np.ones(S) if G is None else G
    H = X if keep is None else X * keep / (1 - p)
    ks = 1.0 if p == 0 else 1.0 / (1 - p)
    y_ref = gl.forward(X, Wn, An, Bn, G, scaling, keep, p)
    lora_abs = scaling * Gv[:, None] * (np.abs(H @ An.T) @ np.abs(Bn).T)
    lora_sum = scaling * Gv[:, None] * ((np.abs(H) @ np.abs(An).T) @ np.abs(Bn).T)
    h_round = 0.0 if p == 0 else (U / 2) * lora_sum
    acc_y = ACC * (np.abs(X) @ np.abs(Wn).T + lora_sum)
    check("y", f64(y), y_ref,
          U * (np.abs(y_ref) + np.abs(X @ Wn.T) + lora_abs) + h_round + acc_y + 1e-5 * np.abs(y_ref).max())
    dx_ref, dA_ref, dB_ref = gl.backward(DY, X, Wn, An, Bn, G, scaling, keep, p)
    d_a = scaling * Gv[:, None] * (DY @ Bn)
    acc_x = ACC * (np.abs(DY) @ np.abs(Wn) + 2 * ks * ((Gv[:, None] * scaling * (np.abs(DY) @ np.abs(Bn))) @ np.abs(An)))
    bx = U * (np.abs(dx_ref) + np.abs(DY @ Wn) + 2 * ks * (np.abs(d_a) @ np.abs(An))) + acc_x \
        + 1e-5 * np.abs(dx_ref).max()
    check("dX", f64(gx), dx_ref, bx)
    check("dA", f64(ga), dA_ref, U * (np.abs(dA_ref) + np.abs(d_a).T @ np.abs(H)) + 1e-30)
    if p > 0:
        check("dA (kept h)", f64(gak), dA_ref, U * (np.abs(dA_ref) + np.abs(d_a).T @ np.abs(H)) + 1e-30)
    T = scaling * Gv[:, None] * (H @ An.T)
    check("dB", f64(gb), dB_ref, U * (np.abs(dB_ref) + np.abs(DY).T @ np.abs(T)) + 1e-30)
    return y, t, h


@pytest.mark.parametrize("p", [0.0, 0.05])
def test_qwen3_qkv_shape(dev, p):
    """Qwen3-8B fused qkv_proj with the reference's training ranks (3 x 32)."""
    run_case(dev, S=512, K=4096, N=6144, r=96, p=p)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("S,K,N,r,p,gate", [
    (512, 4096, 6144, 96, 0.05, "mixed"),   # Qwen3-8B qkv_proj, dropout on
    (512, 4096, 6144, 96, 0.0, "mixed"),
    (333, 4096, 4096, 32, 0.05, None),      # o_proj-like, ragged rows, no gate
    (40, 1024, 200, 64, 0.5, "mixed"),      # heavy dropout, odd N
    (31, 128, 64, 1, 0.0, "mixed"),         # rank 1
    (50, 272, 100, 24, 0.05, "mixed"),      # in_features not a multiple of 128
])
def test_fp16_fp32_layers(dev, dtype, S, K, N, r, p, gate):
    """fp16 and fp32 layers through the general path against the float64
    oracle, the dropout mask identical to the bf16 path's."""
    print(f"case {dtype} S={S} K={K} N={N} r={r} p={p}", flush=True)
    run_case(dev, S, K, N, r, p, gate=gate, seed=S + 1, dtype=dtype)


@pytest.mark.parametrize("S,K,N,r,p,gate", [
    (333, 4096, 4096, 32, 0.05, None),      # o_proj-like, ragged rows, no gate
    (100, 256, 256, 8, 0.0, "mixed"),       # config-1 sizes
    (64, 512, 384, 160, 0.1, "mixed"),      # rank above 96: chunked down-projection
    (40, 1024, 200, 64, 0.5, "mixed"),      # gate_up-like rank, heavy dropout, odd N
    (31, 128, 64, 1, 0.0, "mixed"),         # rank 1, one partial row block
    (50, 272, 100, 24, 0.05, "mixed"),      # in_features not a multiple of 128 (direct-load kernel)
    (70, 320, 512, 16, 0.0, "mixed"),       # ragged rows, in_features 320
    (256, 512, 192, 40, 0.0, None),         # rank 40 (not a multiple of 32), N = 192
    (300, 256, 64, 8, 0.05, "mixed"),       # rank 8 with dropout (the y bound's h-rounding term), N = 64
])
def test_shapes(dev, S, K, N, r, p, gate):
    run_case(dev, S, K, N, r, p, gate=gate, seed=S)


def test_full_qkv_forward_against_fp32(dev):
    """S = 5120 (config 2's chunk): forward against torch fp32 on the GPU."""
    lm = lora_mod()
    S, K, N, r, p, s = 5120, 4096, 6144, 96, 0.05, 2.0
    x, W, A, B, gt = make(S, K, N, r, dev, seed=3)
    y, t, h = lm.gated_lora_forward(x, W, A, B, gt, s, p, 99, keep_h=True)
    hf, xf, Wf, Af, Bf = h.float(), x.float(), W.float(), A.float(), B.float()
    base = xf @ Wf.T
    lora = s * gt[:, None] * ((hf @ Af.T) @ Bf.T)
    ref = base + lora
    lora_abs = s * gt[:, None] * ((hf @ Af.T).abs() @ Bf.abs().T)
    bound = U * (ref.abs() + base.abs() + lora_abs) + 1e-5 * ref.abs().max()
    worst = ((y.float() - ref).abs() / bound).max().item()
    kept = (h != 0).float().mean().item()
    print(f"  S=5120: worst err/bound {worst:.3f}, kept fraction {kept:.4f}", flush=True)
    assert worst <= 1.0
    assert abs(kept - (1 - gl.drop_threshold(p) / 65536)) < 1e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_module_forward_backward(dev, dtype):
    """GatedLoRALinear (the mirror) in train mode through autograd: x, lora_A
    and lora_B get gradients, the base weight none, and the result equals the
    functional entry points with the same seed."""
    lm = lora_mod()
    torch.manual_seed(0)
    base = torch.nn.Linear(256, 384, bias=False).to(dev, dtype)
    layer = lm.GatedLoRALinear(base, rank=16, alpha=32, dropout=0.05, lora_bias=False, use_rslora=False)
    base.weight.requires_grad_(False)
    with torch.no_grad():
        layer.lora_B.weight.normal_(0, 0.05)
    x = torch.randn(1, 100, 256, device=dev).to(dtype).requires_grad_()
    gate = (torch.rand(1, 100, 1, device=dev) < 0.5).long()
    torch.manual_seed(5)
    y = layer(x, gate)
    y.float().square().sum().backward()
    assert y.shape == (1, 100, 384) and y.dtype == dtype
    assert x.grad is not None and layer.lora_A.weight.grad is not None and layer.lora_B.weight.grad is not None
    assert base.weight.grad is None
    torch.manual_seed(5)
    seed = int(torch.randint(0, 2 ** 62, (), dtype=torch.int64).item())
    y2, _, _ = lm.gated_lora_forward(x.detach()[0], base.weight, layer.lora_A.weight, layer.lora_B.weight,
                                     gate.reshape(-1).float(), 2.0, 0.05, seed)
    assert torch.equal(y.detach()[0], y2)
    layer.eval()
    y3 = layer(x.detach(), gate)
    y4, _, _ = lm.gated_lora_forward(x.detach()[0], base.weight, layer.lora_A.weight, layer.lora_B.weight,
                                     gate.reshape(-1).float(), 2.0, 0.0, 0)
    assert torch.equal(y3[0], y4)


def test_argument_errors(dev):
    lm = lora_mod()
    x, W, A, B, gt = make(8, 64, 32, 4, dev)
    with pytest.raises(TypeError):
        lm.gated_lora_linear(x.float(), W, A, B, gt, 2.0)
    with pytest.raises(NotImplementedError):
        lm.gated_lora_linear(x, W.clone().requires_grad_(), A, B, gt, 2.0)
    with pytest.raises(ValueError):
        lm.gated_lora_linear(x, W, A, B, gt[:5], 2.0)
    x2, W2, A2, B2, g2 = make(8, 40, 32, 4, dev)
    with pytest.raises(Exception, match="multiple of 16"):
        lm.gated_lora_linear(x2, W2, A2, B2, g2, 2.0)
    with pytest.raises(RuntimeError):
        lm.gated_lora_linear(x.cpu(), W.cpu(), A.cpu(), B.cpu(), None, 2.0)


def test_dx_row_stride_multiple_of_4(dev):
    """grad_x rows 8-byte aligned only (row stride K + 4): the in-place dropout
    update takes its 8-byte path and still matches the oracle."""
    lm = lora_mod()
    lib = importlib.import_module("mtp-glora_amd._lib")
    S, K, N, r, p, s = 96, 512, 384, 32, 0.1, 2.0
    x, W, A, B, gt = make(S, K, N, r, dev, seed=11)
    sd = 4242
    y, t, h = lm.gated_lora_forward(x, W, A, B, gt, s, p, sd)
    dy = torch.randn(S, N, generator=torch.Generator(device=dev).manual_seed(12), device=dev).bfloat16()
    buf = torch.zeros(S, K + 4, device=dev, dtype=torch.bfloat16)
    gx = buf[:, :K]
    ws = lm._workspace(S, K, N, r, dev)
    lib.call("mga_gated_lora_bwd", dy.data_ptr(), dy.stride(0), x.data_ptr(), x.stride(0), None,
             0, W.data_ptr(), W.stride(0), A.data_ptr(), A.stride(0), B.data_ptr(), B.stride(0),
             t.data_ptr(), t.stride(0), gt.data_ptr(), s, p, sd, S, K, N, r, gx.data_ptr(), gx.stride(0),
             None, 0, None, 0, ws.data_ptr(), ws.numel(), lib.DTYPE_BF16,
             torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    assert torch.count_nonzero(buf[:, K:]).item() == 0   # the 4 pad columns are untouched
    X, Wn, An, Bn, G, DY = f64(x), f64(W), f64(A), f64(B), f64(gt), f64(dy)
    keep = gl.keep_mask(sd, S, K, p)
    dx_ref, _, _ = gl.backward(DY, X, Wn, An, Bn, G, s, keep, p)
    d_a = s * G[:, None] * (DY @ Bn)
    bx = U * (np.abs(dx_ref) + np.abs(DY @ Wn) + 2 / (1 - p) * (np.abs(d_a) @ np.abs(An))) + 1e-5 * np.abs(dx_ref).max()
    check("dX (stride K + 4)", f64(gx), dx_ref, bx)
