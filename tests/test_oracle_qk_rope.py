"""Pins for oracle/qk_rope.py (Qwen3 q/k RMSNorm + rotary embedding of
mtp_glora/models/modeling_qwen3.py:61-67, :118-149, :274-279) that do not
restate its formula:

* transformers' own Qwen3RMSNorm and apply_rotary_pos_emb (the library code the
  reference's modeling file carries unchanged) run as torch CPU ops on the same
  bf16 / fp32 tensors, in the reference's call order (norm on [B, S, H, D],
  transpose, rope with unsqueeze_dim=1);
* the same comparison shows that dropping either intermediate bf16 rounding
  (after x * r, after n * cos) is caught;
* closed forms: sin = 0, cos = 1 reduces to the RMSNorm alone; the rotation
  keeps each (d, d + D/2) pair's length; unit weights give unit RMS;
* the gradient against torch autograd through the same library modules (which
  compute in fp32) and against central finite differences.
"""
import numpy as np
import pytest
import torch

from oracle import qk_rope as qr

tm = pytest.importorskip("transformers.models.qwen3.modeling_qwen3")


def _inputs(S, H, D, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(1, S, H, D, generator=g) * 2 + 0.3).to(dtype)
    w = (1 + 0.5 * torch.randn(D, generator=g)).to(dtype)
    c64, s64 = qr.rope_tables(np.arange(S) * 7 + 3, D)
    cos = torch.tensor(c64, dtype=torch.float32).to(dtype)[None]
    sin = torch.tensor(s64, dtype=torch.float32).to(dtype)[None]
    return x, w, cos, sin


def _library(x, w, cos, sin, eps):
    norm = tm.Qwen3RMSNorm(x.shape[-1], eps=eps).to(x.dtype)
    with torch.no_grad():
        norm.weight.copy_(w)
        n = norm(x).transpose(1, 2)                        # modeling_qwen3.py:274-275
        out, _ = tm.apply_rotary_pos_emb(n, n, cos, sin)   # :278
    return out.transpose(1, 2)[0].float().numpy()


def _oracle(x, w, cos, sin, eps, bf16):
    out, r = qr.norm_rope(x[0].float().numpy(), w.float().numpy(), cos[0].float().numpy(),
                          sin[0].float().numpy(), eps, bf16)
    return out, r


@pytest.mark.parametrize("D", [128, 64])
def test_bf16_matches_library_ops(D):
    x, w, cos, sin = _inputs(96, 12, D, D, torch.bfloat16)
    ref = _library(x, w, cos, sin, 1e-6)
    got, _ = _oracle(x, w, cos, sin, 1e-6, True)
    # the library's fp32 mean and rsqrt may differ from the oracle's in the
    # last fp32 bit; that flips a bf16 rounding in a rare element only
    diff = got != ref
    assert diff.mean() < 1e-3, diff.mean()
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 2.0 ** -6 * scale


@pytest.mark.parametrize("D", [128, 64])
def test_f16_matches_library_ops(D):
    x, w, cos, sin = _inputs(96, 12, D, D + 1, torch.float16)
    ref = _library(x, w, cos, sin, 1e-6)
    got, _ = _oracle(x, w, cos, sin, 1e-6, "f16")
    diff = got != ref
    assert diff.mean() < 1e-3, diff.mean()
    assert np.abs(got - ref).max() <= 2.0 ** -9 * np.abs(ref).max()
    # the bf16 rounding in its place is caught
    wrong, _ = _oracle(x, w, cos, sin, 1e-6, "bf16")
    assert (wrong != ref).mean() > 0.1


def test_f16_round_known_values():
    vals = np.array([1.0, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 65504.0, 65520.0, 2.0 ** -25, 2.0 ** -24 * 1.5,
                     -3.0e-5], dtype=np.float32)
    want = np.array([1.0, 1.0, 1.0 + 2.0 ** -9, 65504.0, np.inf, 0.0, 2.0 ** -23, -3.0e-5], dtype=np.float32)
    got = qr.f16_round(vals)
    np.testing.assert_array_equal(got[:7], want[:7])
    assert abs(got[7] - want[7]) <= 2.0 ** -25   # a subnormal: spacing 2^-24
    a = np.random.default_rng(1).standard_normal(4096).astype(np.float32) * 100
    np.testing.assert_array_equal(qr.f16_round(a), torch.tensor(a).half().float().numpy())


def test_dropped_roundings_are_caught():
    x, w, cos, sin = _inputs(64, 8, 128, 5, torch.bfloat16)
    ref = _library(x, w, cos, sin, 1e-6)
    xf, wf = x[0].float().numpy(), w.float().numpy()
    c, s = cos[0].float().numpy()[:, None, :], sin[0].float().numpy()[:, None, :]
    T = qr.bf16_round
    r = 1.0 / np.sqrt((xf * xf).mean(axis=-1, keepdims=True).astype(np.float64) + 1e-6)
    y_exact = (xf * r.astype(np.float32))
    for y in (y_exact, T(y_exact)):
        n = T(wf * y)
        rot = np.concatenate([-n[..., 64:], n[..., :64]], axis=-1)
        no_mid = T(n * c + rot * s)             # one rounding for the whole rope
        assert (no_mid != ref).mean() > 0.01
    n = T(wf * y_exact)                          # norm without the rounding of x * r
    rot = np.concatenate([-n[..., 64:], n[..., :64]], axis=-1)
    assert (T(T(n * c) + T(rot * s)) != ref).mean() > 0.01


def test_fp32_matches_library_ops():
    x, w, cos, sin = _inputs(64, 10, 128, 2, torch.float32)
    ref = _library(x, w, cos, sin, 1e-6)
    got, _ = _oracle(x, w, cos, sin, 1e-6, False)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-6)


def test_closed_forms():
    S, H, D = 16, 4, 128
    rng = np.random.default_rng(3)
    x = rng.normal(size=(S, H, D)).astype(np.float32) * 3
    w = np.ones(D, dtype=np.float32)
    one, zero = np.ones((S, D), np.float32), np.zeros((S, D), np.float32)
    out, r = qr.norm_rope(x, w, one, zero, 1e-6, False)
    # RMSNorm alone with unit weights: unit RMS per row, r = 1 / rms(x)
    np.testing.assert_allclose((out.astype(np.float64) ** 2).mean(axis=-1), 1.0, rtol=1e-5)
    np.testing.assert_allclose(r, 1 / np.sqrt((x.astype(np.float64) ** 2).mean(axis=-1) + 1e-6), rtol=1e-6)
    # a rotation keeps each (d, d + D/2) pair's length
    c64, s64 = qr.rope_tables(np.arange(S) * 11, D)
    rot, _ = qr.norm_rope(x, w, c64.astype(np.float32), s64.astype(np.float32), 1e-6, False)
    pair = lambda a: a[..., :D // 2] ** 2 + a[..., D // 2:] ** 2  # noqa: E731
    np.testing.assert_allclose(pair(rot.astype(np.float64)), pair(out.astype(np.float64)), rtol=1e-5, atol=1e-6)


def test_gradient_matches_autograd_and_finite_differences():
    S, H, D = 6, 3, 64
    x, w, cos, sin = _inputs(S, H, D, 9, torch.float64)
    g = torch.randn(1, S, H, D, generator=torch.Generator().manual_seed(10), dtype=torch.float64)
    norm = tm.Qwen3RMSNorm(D, eps=1e-6).double()
    norm.weight.requires_grad_(False)
    norm.weight.copy_(w)
    xg = x.clone().requires_grad_()
    n = norm(xg).transpose(1, 2)
    out, _ = tm.apply_rotary_pos_emb(n, n, cos, sin)
    (out.transpose(1, 2) * g).sum().backward()
    got = qr.norm_rope_grad(x[0].numpy(), w.numpy(), cos[0].numpy(), sin[0].numpy(), g[0].numpy(), 1e-6)
    # Qwen3RMSNorm computes in fp32 whatever its input dtype, so the library's
    # gradient carries fp32 rounding; a dropped term or sign is O(1)
    np.testing.assert_allclose(got, xg.grad[0].numpy(), rtol=1e-4, atol=1e-5)

    # central differences of the library forward (fp32 inside: h = 1e-3)
    def f(xx):
        with torch.no_grad():
            nn_ = norm(torch.as_tensor(xx)[None]).transpose(1, 2)
            o, _ = tm.apply_rotary_pos_emb(nn_, nn_, cos, sin)
            return (o.transpose(1, 2)[0] * g[0]).sum().item()

    x0 = x[0].numpy()
    h = 1e-3
    for (s_, h_, d_) in [(0, 0, 0), (2, 1, 17), (5, 2, 63), (3, 0, 32)]:
        xp, xm = x0.copy(), x0.copy()
        xp[s_, h_, d_] += h
        xm[s_, h_, d_] -= h
        num = (f(xp) - f(xm)) / (2 * h)
        assert abs(num - got[s_, h_, d_]) <= 2e-3 * (1 + abs(num))


def test_bf16_round_known_values():
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20, -2.5, 3.0e-39],
                    dtype=np.float32)
    want = torch.tensor(vals).bfloat16().float().numpy()
    np.testing.assert_array_equal(qr.bf16_round(vals), want)
    rng = np.random.default_rng(0)
    a = (rng.normal(size=100000) * 10 ** rng.uniform(-30, 30, size=100000)).astype(np.float32)
    np.testing.assert_array_equal(qr.bf16_round(a), torch.tensor(a).bfloat16().float().numpy())
