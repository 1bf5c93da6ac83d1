"""HIP stable soft cross-entropy (mga_soft_ce_*) against the float64 oracle
(oracle/soft_ce.py, pinned by tests/test_oracle_soft_ce.py).

* The reference's own test (mtp_glora/core/loss.py:335-385): fp32 logits
  [4, 4, 4096] and [8, 2, 151936], loss sum and student gradient within its
  tolerances (rtol = atol = 2e-4, and 3e-4 at V = 151936).
* bf16 logits (the model dtype) at the sampler's shape, V = 151936: the oracle
  runs on the same bf16 values; loss within rtol 1e-4, gradient (bf16) within
  one bf16 rounding of the oracle's value (rtol 2^-7) plus atol 1e-7.
* fp16 logits at the same shape: loss within rtol 1e-4, gradient (fp16)
  within 2^-10 of the oracle's value plus 3e-8 (half the spacing of fp16's
  subnormals, where most of the gradient's elements lie).
* A strided teacher (the reference's call site passes a strided view,
  core/mtp.py:124), widths that are not multiples of the vector width, a
  misaligned row stride (element-load path), a single column, and rows whose
  maxima differ by hundreds of units (stable rescaling).
"""
import numpy as np
import pytest
import torch

from oracle import soft_ce as sc

pytestmark = pytest.mark.gpu


def _run(mga, x, t, go=1.0):
    xg = x.detach().clone().requires_grad_()
    loss = mga.StableSoftCrossEntropy.apply(xg, t)
    loss.backward(torch.tensor(go, device=x.device))
    torch.cuda.synchronize()
    return loss.item(), xg.grad


def _f64(t):
    return t.detach().double().cpu().numpy()


@pytest.mark.parametrize("shape,tol", [((4, 4, 4096), 2e-4), ((8, 2, 151936), 3e-4)])
def test_reference_test_shapes_fp32(mga, dev, shape, tol):
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(*shape, generator=g, device=dev)
    t = torch.randn(*shape, generator=g, device=dev)
    loss, grad = _run(mga, x, t)
    ref = sc.soft_ce_loss(_f64(x), _f64(t))
    ref_g = sc.soft_ce_grad(_f64(x), _f64(t))
    print(f"  loss {loss:.6f} ref {ref:.6f}", flush=True)
    assert abs(loss - ref) <= tol + tol * abs(ref)
    assert grad.dtype == torch.float32
    np.testing.assert_allclose(_f64(grad), ref_g, rtol=tol, atol=tol)


@pytest.mark.parametrize("rows", [1, 255, 512])
def test_bf16_sampler_shape(mga, dev, rows):
    g = torch.Generator(device=dev).manual_seed(rows)
    V = 151936
    x = (torch.randn(1, rows, V, generator=g, device=dev) * 3).bfloat16()
    t = (torch.randn(1, rows, V, generator=g, device=dev) * 3).bfloat16()
    loss, grad = _run(mga, x, t, go=0.5)
    ref = sc.soft_ce_loss(_f64(x), _f64(t))
    ref_g = 0.5 * sc.soft_ce_grad(_f64(x), _f64(t))
    assert abs(loss - ref) <= 1e-4 * abs(ref)
    assert grad.dtype == torch.bfloat16
    err = np.abs(_f64(grad) - ref_g)
    print(f"  rows {rows}: loss {loss:.4f} ref {ref:.4f} grad max-abs {err.max():.3e}", flush=True)
    assert (err <= 2.0 ** -7 * np.abs(ref_g) + 1e-7).all()


@pytest.mark.parametrize("rows", [1, 300])
def test_fp16_sampler_shape(mga, dev, rows):
    g = torch.Generator(device=dev).manual_seed(rows + 7)
    V = 151936
    x = (torch.randn(1, rows, V, generator=g, device=dev) * 3).half()
    t = (torch.randn(1, rows, V, generator=g, device=dev) * 3).half()
    loss, grad = _run(mga, x, t, go=0.5)
    ref = sc.soft_ce_loss(_f64(x), _f64(t))
    ref_g = 0.5 * sc.soft_ce_grad(_f64(x), _f64(t))
    assert abs(loss - ref) <= 1e-4 * abs(ref)
    assert grad.dtype == torch.float16
    err = np.abs(_f64(grad) - ref_g)
    print(f"  rows {rows}: loss {loss:.4f} ref {ref:.4f} grad max-abs {err.max():.3e}", flush=True)
    assert (err <= 2.0 ** -10 * np.abs(ref_g) + 3e-8).all()


def test_strided_teacher_and_odd_widths(mga, dev):
    g = torch.Generator(device=dev).manual_seed(3)
    # teacher as a strided row view of a larger logits tensor (every 5th row)
    base = torch.randn(1, 60, 1000, generator=g, device=dev).bfloat16()
    t = base[:, 3::5, :]
    x = torch.randn(1, t.shape[1], 1000, generator=g, device=dev).bfloat16()
    loss, grad = _run(mga, x, t)
    assert abs(loss - sc.soft_ce_loss(_f64(x), _f64(t))) <= 1e-4 * abs(loss)
    np.testing.assert_allclose(_f64(grad), sc.soft_ce_grad(_f64(x), _f64(t)), rtol=2.0 ** -7, atol=1e-6)
    for V in (1, 7, 4099, 20011):   # tails and the element-load path (odd row strides)
        x = torch.randn(2, 3, V, generator=g, device=dev)
        t = torch.randn(2, 3, V, generator=g, device=dev)
        loss, grad = _run(mga, x, t)
        ref = sc.soft_ce_loss(_f64(x), _f64(t))
        assert abs(loss - ref) <= 1e-4 * (1 + abs(ref)), V
        np.testing.assert_allclose(_f64(grad), sc.soft_ce_grad(_f64(x), _f64(t)), rtol=1e-4, atol=1e-6)


def test_large_offsets_and_identical_rows(mga, dev):
    g = torch.Generator(device=dev).manual_seed(4)
    x = torch.randn(1, 6, 70000, generator=g, device=dev)
    x += torch.tensor([0.0, 300.0, -300.0, 80.0, -80.0, 0.0], device=dev)[None, :, None]
    t = x.clone()
    t[0, 5] = torch.randn(70000, generator=g, device=dev) * 20
    loss, grad = _run(mga, x, t)
    ref = sc.soft_ce_loss(_f64(x), _f64(t))
    assert abs(loss - ref) <= 1e-4 * abs(ref)
    ref_g = sc.soft_ce_grad(_f64(x), _f64(t))
    np.testing.assert_allclose(_f64(grad), ref_g, rtol=1e-4, atol=1e-7)
    assert np.abs(_f64(grad)[0, :5]).max() < 1e-6   # identical rows: zero gradient


def test_argument_errors(mga, dev):
    x = torch.randn(1, 2, 64, device=dev)
    with pytest.raises(ValueError):
        mga.StableSoftCrossEntropy.apply(x, torch.randn(1, 2, 65, device=dev))
    with pytest.raises(TypeError):
        mga.StableSoftCrossEntropy.apply(x, x.bfloat16())
    with pytest.raises(RuntimeError):
        mga.StableSoftCrossEntropy.apply(x.cpu(), x.cpu())
