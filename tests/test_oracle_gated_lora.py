"""Pins for oracle/gated_lora.py (GatedLoRALinear of
mtp_glora/models/layers/gated_lora.py) that do not restate its formula, and
the CPU-side behaviour of the module mirror:

* forward and gradients against torch autograd in float64 through torch's own
  nn.Linear modules wired as the reference wires them (base, lora_A, lora_B;
  dropout as multiplication by the explicit keep mask and 1 / (1 - p));
* central finite differences for dX, dA, dB;
* closed forms: lora_B = 0 (the reference's initialisation) gives the base
  output and zero dA; gate 0 gives the base output and zero LoRA gradients;
* the keep mask: deterministic per seed, all kept at p = 0, keep rate 1 - p
  within binomial noise, seeds and element pairs independent;
* the module mirror: constructor attributes, parameter names, initialisation
  and apply_lora_to_model's wrapping (x3 rank for qkv_proj, x2 for
  gate_up_proj) and freezing, as the reference's code defines them.
"""
import importlib
import math

import numpy as np
import pytest
import torch

from oracle import gated_lora as gl


def _case(S=7, K=32, N=24, r=6, seed=0, p=0.0):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(S, K))
    W = rng.normal(size=(N, K)) / math.sqrt(K)
    A = rng.normal(size=(r, K)) / math.sqrt(K)
    B = rng.normal(size=(N, r)) / math.sqrt(r)
    gate = (rng.random(S) < 0.6).astype(np.float64)
    keep = gl.keep_mask(seed + 99, S, K, p) if p > 0 else None
    return x, W, A, B, gate, keep


def _torch_reference(x, W, A, B, gate, scaling, keep, p, dy):
    K, N, r = W.shape[1], W.shape[0], A.shape[0]
    base = torch.nn.Linear(K, N, bias=False).double()
    la = torch.nn.Linear(K, r, bias=False).double()
    lb = torch.nn.Linear(r, N, bias=False).double()
    with torch.no_grad():
        base.weight.copy_(torch.as_tensor(W))
        la.weight.copy_(torch.as_tensor(A))
        lb.weight.copy_(torch.as_tensor(B))
    base.weight.requires_grad_(False)
    xt = torch.as_tensor(x).requires_grad_()
    h = xt if keep is None else xt * torch.as_tensor(keep, dtype=torch.float64) / (1 - p)
    g = torch.as_tensor(gate)[:, None]
    y = base(xt) + scaling * lb(la(h)) * g
    y.backward(torch.as_tensor(dy))
    return y.detach().numpy(), xt.grad.numpy(), la.weight.grad.numpy(), lb.weight.grad.numpy()


@pytest.mark.parametrize("p", [0.0, 0.25])
def test_matches_torch_autograd(p):
    x, W, A, B, gate, keep = _case(p=p)
    dy = np.random.default_rng(5).normal(size=(x.shape[0], W.shape[0]))
    y_t, dx_t, dA_t, dB_t = _torch_reference(x, W, A, B, gate, 2.0, keep, p, dy)
    np.testing.assert_allclose(gl.forward(x, W, A, B, gate, 2.0, keep, p), y_t, rtol=1e-12, atol=1e-12)
    dx, dA, dB = gl.backward(dy, x, W, A, B, gate, 2.0, keep, p)
    np.testing.assert_allclose(dx, dx_t, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dA, dA_t, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dB, dB_t, rtol=1e-12, atol=1e-12)


def test_finite_differences():
    x, W, A, B, gate, keep = _case(S=4, K=16, N=10, r=3, p=0.3, seed=2)
    dy = np.random.default_rng(3).normal(size=(4, 10))
    f = lambda xx, AA, BB: (gl.forward(xx, W, AA, BB, gate, 1.5, keep, 0.3) * dy).sum()   # noqa: E731
    dx, dA, dB = gl.backward(dy, x, W, A, B, gate, 1.5, keep, 0.3)
    h = 1e-6
    for arr, grad, which in ((x, dx, 0), (A, dA, 1), (B, dB, 2)):
        for idx in [(0, 0), (1, 2), (arr.shape[0] - 1, arr.shape[1] - 1)]:
            ap, am = arr.copy(), arr.copy()
            ap[idx] += h
            am[idx] -= h
            args_p = [x, A, B]
            args_m = [x, A, B]
            args_p[which], args_m[which] = ap, am
            num = (f(*args_p) - f(*args_m)) / (2 * h)
            assert abs(num - grad[idx]) <= 1e-6 * (1 + abs(num)), (which, idx)


def test_closed_forms():
    x, W, A, B, gate, _ = _case()
    base = x @ W.T
    np.testing.assert_allclose(gl.forward(x, W, A, np.zeros_like(B), gate, 2.0), base, rtol=1e-13, atol=1e-13)
    dy = np.ones((x.shape[0], W.shape[0]))
    _, dA, _ = gl.backward(dy, x, W, A, np.zeros_like(B), gate, 2.0)
    assert np.abs(dA).max() == 0.0
    zero = np.zeros(x.shape[0])
    np.testing.assert_allclose(gl.forward(x, W, A, B, zero, 2.0), base, rtol=1e-13, atol=1e-13)
    dx, dA, dB = gl.backward(dy, x, W, A, B, zero, 2.0)
    assert np.abs(dA).max() == 0.0 and np.abs(dB).max() == 0.0
    np.testing.assert_allclose(dx, dy @ W, rtol=1e-13, atol=1e-13)


def test_keep_mask_properties():
    assert gl.keep_mask(7, 16, 64, 0.0).all()
    a = gl.keep_mask(7, 64, 1024, 0.05)
    np.testing.assert_array_equal(a, gl.keep_mask(7, 64, 1024, 0.05))
    n = a.size
    rate = a.mean()
    assert abs(rate - (1 - gl.drop_threshold(0.05) / 65536)) < 5 * math.sqrt(0.05 * 0.95 / n)
    b = gl.keep_mask(8, 64, 1024, 0.05)
    # two seeds: agreement as for independent draws, P(equal) = q^2 + (1-q)^2
    q = 1 - gl.drop_threshold(0.05) / 65536
    assert abs((a == b).mean() - (q * q + (1 - q) ** 2)) < 5 * math.sqrt(0.1 / n)
    # the even and odd element of a pair come from different bits
    ev, od = a[:, 0::2].ravel(), a[:, 1::2].ravel()
    assert abs((ev & od).mean() - q * q) < 5 * math.sqrt(0.1 / ev.size)
    half = gl.keep_mask(7, 64, 1024, 0.5)
    assert abs(half.mean() - 0.5) < 5 * math.sqrt(0.25 / n)


def test_module_mirror_construction():
    mod = importlib.import_module("mtp-glora_amd")
    base = torch.nn.Linear(64, 48, bias=False, dtype=torch.bfloat16)
    layer = mod.GatedLoRALinear(base, rank=8, alpha=16, dropout=0.05, lora_bias=False, use_rslora=False)
    assert layer.lora_scaling == 2.0 and layer.rank == 8 and layer.alpha == 16
    assert isinstance(layer.dropout, torch.nn.Dropout) and layer.dropout.p == 0.05
    assert sorted(dict(layer.named_parameters())) == ["base_layer.weight", "lora_A.weight", "lora_B.weight"]
    assert tuple(layer.lora_A.weight.shape) == (8, 64) and tuple(layer.lora_B.weight.shape) == (48, 8)
    assert layer.lora_B.weight.abs().max().item() == 0.0 and layer.lora_A.weight.abs().max().item() > 0
    rs = mod.GatedLoRALinear(base, rank=16, alpha=32, dropout=0.0, lora_bias=False, use_rslora=True)
    assert rs.lora_scaling == pytest.approx(32 / 4) and isinstance(rs.dropout, torch.nn.Identity)
    assert layer.lora_A.weight.dtype == torch.bfloat16


def _lora_net(dtype):

    class Attn(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.qkv_proj = torch.nn.Linear(32, 96, bias=False)
            self.o_proj = torch.nn.Linear(32, 32, bias=False)

    class Mlp(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_up_proj = torch.nn.Linear(32, 128, bias=False)
            self.down_proj = torch.nn.Linear(64, 32, bias=False)

    class Net(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.attn, self.mlp = Attn(), Mlp()
            self.lm_head = torch.nn.Linear(32, 100, bias=False)

    return Net().to(dtype)


def test_apply_lora_to_model_wraps_and_freezes():
    mod = importlib.import_module("mtp-glora_amd")
    net = _lora_net(torch.bfloat16)
    mod.apply_lora_to_model(net, rank=4, alpha=8, dropout=0.0)
    assert isinstance(net.attn.qkv_proj, mod.GatedLoRALinear) and net.attn.qkv_proj.rank == 12
    assert net.attn.qkv_proj.alpha == 24 and net.attn.qkv_proj.lora_scaling == 2.0
    assert net.mlp.gate_up_proj.rank == 8 and net.mlp.down_proj.rank == 4 and net.attn.o_proj.rank == 4
    assert isinstance(net.lm_head, torch.nn.Linear)
    trainable = sorted(n for n, p in net.named_parameters() if p.requires_grad)
    assert trainable and all("lora_" in n for n in trainable)
    assert not net.attn.qkv_proj.base_layer.weight.requires_grad


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_apply_lora_to_model_wraps_every_model_dtype(dtype):
    """bf16, fp16 and fp32 models (the reference's dtypes, args.py:15) are all
    wrapped, the LoRA weights in the base layer's dtype."""
    mod = importlib.import_module("mtp-glora_amd")
    net = _lora_net(dtype)
    mod.apply_lora_to_model(net, rank=4, alpha=8, dropout=0.0)
    assert isinstance(net.attn.qkv_proj, mod.GatedLoRALinear)
    assert net.attn.qkv_proj.lora_A.weight.dtype == dtype and net.mlp.down_proj.lora_B.weight.dtype == dtype


def test_apply_lora_to_model_refuses_other_dtypes_up_front():
    """A dtype the layer has no path for (float64) gets a TypeError naming the
    first target layer, before any layer is wrapped or frozen."""
    mod = importlib.import_module("mtp-glora_amd")
    net = _lora_net(torch.float64)
    net.mlp.down_proj.to(torch.bfloat16)   # one matching layer of a supported dtype changes nothing
    with pytest.raises(TypeError, match="attn.qkv_proj.*float64"):
        mod.apply_lora_to_model(net, rank=4, alpha=8, dropout=0.0)
    assert not any(isinstance(m, mod.GatedLoRALinear) for m in net.modules())
    assert all(p.requires_grad for p in net.parameters())
    with pytest.raises(TypeError, match="float64"):
        mod.GatedLoRALinear(torch.nn.Linear(8, 8, bias=False, dtype=torch.float64), 4, 8, 0.0, False, False)
