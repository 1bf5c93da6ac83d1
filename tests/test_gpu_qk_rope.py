"""HIP fused q/k RMSNorm + rotary embedding (mga_qk_norm_rope_*) against the
oracle (oracle/qk_rope.py, pinned by tests/test_oracle_qk_rope.py) and against
transformers' Qwen3RMSNorm / apply_rotary_pos_emb run as torch ops on the GPU
(the reference's own call, mtp_glora/models/modeling_qwen3.py:274-279).

Forward tolerance (bf16): the kernel rounds after every op exactly where the
reference does, so outputs are bit-equal except where the fp32 row mean or the
hardware rsqrt differs from the checker's in the last fp32 bit and flips one
bf16 rounding: at most 1e-3 of the elements differ, each by at most 2^-6 of
its row's largest magnitude (fp16: the same fraction, 2^-9). fp32: rtol 1e-5,
atol 1e-6. rstd: rtol 2e-6. Backward: the oracle's float64 gradient on the
same inputs; each bf16 element within 2^-8 of its value plus 1e-5 of the
tensor's largest (one bf16 rounding of an fp32 result), fp16 within 2^-11
plus the same; fp32 within 1e-5 relative.
"""
import numpy as np
import pytest
import torch

from oracle import qk_rope as qr

pytestmark = pytest.mark.gpu


def make(S, Hq, Hkv, D, dtype, dev, seed=0, pos0=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    q = (torch.randn(1, S, Hq, D, generator=g, device=dev) * 2 + 0.2).to(dtype)
    k = (torch.randn(1, S, Hkv, D, generator=g, device=dev) * 3 - 0.1).to(dtype)
    qw = (1 + 0.3 * torch.randn(D, generator=g, device=dev)).to(dtype)
    kw = (1 + 0.3 * torch.randn(D, generator=g, device=dev)).to(dtype)
    c64, s64 = qr.rope_tables(np.arange(pos0, pos0 + S), D)
    cos = torch.tensor(c64, dtype=torch.float32, device=dev).to(dtype)[None]
    sin = torch.tensor(s64, dtype=torch.float32, device=dev).to(dtype)[None]
    return q, k, qw, kw, cos, sin


def npf(t):
    return t.detach().float().cpu().numpy()


def oracle_fwd(q, k, qw, kw, cos, sin, eps, bf16):
    c, s = npf(cos)[0], npf(sin)[0]
    qo, qr_ = qr.norm_rope(npf(q)[0], npf(qw), c, s, eps, bf16)
    ko, kr_ = qr.norm_rope(npf(k)[0], npf(kw), c, s, eps, bf16)
    return qo, ko, np.concatenate([qr_, kr_], axis=1)


def check_bf16(name, got, ref, bound=2.0 ** -6):
    diff = got != ref
    frac = diff.mean()
    rowmax = np.abs(ref).max(axis=-1, keepdims=True)
    err = np.abs(got - ref) / rowmax
    print(f"  {name}: {diff.sum()} of {diff.size} differ ({frac:.2e}), max {err.max():.2e} of row max",
          flush=True)
    assert frac <= 1e-3, name
    assert err.max() <= bound, name


def run_fwd(mga, q, k, qw, kw, cos, sin, eps=1e-6):
    from importlib import import_module
    rope = import_module("mtp-glora_amd.rope")
    qo, ko, rstd = rope.norm_rope_forward(q, k, qw, kw, cos, sin, eps)
    torch.cuda.synchronize()
    return qo, ko, rstd


@pytest.mark.parametrize("S,Hq,Hkv,D", [(1024, 32, 8, 128), (777, 4, 2, 64), (65, 6, 3, 96), (33, 2, 1, 80),
                                        (9, 3, 1, 6), (5, 1, 1, 2)])
def test_forward_bf16_against_oracle(mga, dev, S, Hq, Hkv, D):
    q, k, qw, kw, cos, sin = make(S, Hq, Hkv, D, torch.bfloat16, dev, seed=S, pos0=8192)
    qo, ko, rstd = run_fwd(mga, q, k, qw, kw, cos, sin)
    rq, rk, rr = oracle_fwd(q, k, qw, kw, cos, sin, 1e-6, True)
    check_bf16("q", npf(qo)[0], rq)
    check_bf16("k", npf(ko)[0], rk)
    np.testing.assert_allclose(npf(rstd), rr, rtol=2e-6)


@pytest.mark.parametrize("S,Hq,Hkv,D", [(1024, 32, 8, 128), (65, 6, 3, 96), (33, 2, 1, 80), (5, 1, 1, 2)])
def test_forward_fp16_against_oracle(mga, dev, S, Hq, Hkv, D):
    q, k, qw, kw, cos, sin = make(S, Hq, Hkv, D, torch.float16, dev, seed=S + 2, pos0=4096)
    qo, ko, rstd = run_fwd(mga, q, k, qw, kw, cos, sin)
    assert qo.dtype == torch.float16 and ko.dtype == torch.float16
    rq, rk, rr = oracle_fwd(q, k, qw, kw, cos, sin, 1e-6, "f16")
    check_bf16("q", npf(qo)[0], rq, bound=2.0 ** -9)
    check_bf16("k", npf(ko)[0], rk, bound=2.0 ** -9)
    np.testing.assert_allclose(npf(rstd), rr, rtol=2e-6)


def test_forward_matches_library_ops_on_gpu(mga, dev):
    tm = pytest.importorskip("transformers.models.qwen3.modeling_qwen3")
    q, k, qw, kw, cos, sin = make(1024, 32, 8, 128, torch.bfloat16, dev, seed=7, pos0=100)
    qn = tm.Qwen3RMSNorm(128, eps=1e-6).to(dev, torch.bfloat16)
    kn = tm.Qwen3RMSNorm(128, eps=1e-6).to(dev, torch.bfloat16)
    with torch.no_grad():
        qn.weight.copy_(qw)
        kn.weight.copy_(kw)
        rq, rk = tm.apply_rotary_pos_emb(qn(q).transpose(1, 2), kn(k).transpose(1, 2), cos, sin)
    emb_q, emb_k = mga.qk_norm_rope(q, k, qw, kw, cos, sin, 1e-6)
    torch.cuda.synchronize()
    assert emb_q.shape == rq.shape and emb_k.shape == rk.shape
    check_bf16("q vs torch", npf(emb_q.transpose(1, 2))[0], npf(rq.transpose(1, 2))[0])
    check_bf16("k vs torch", npf(emb_k.transpose(1, 2))[0], npf(rk.transpose(1, 2))[0])


def test_forward_fp32(mga, dev):
    q, k, qw, kw, cos, sin = make(300, 4, 2, 64, torch.float32, dev, seed=3)
    qo, ko, rstd = run_fwd(mga, q, k, qw, kw, cos, sin)
    rq, rk, rr = oracle_fwd(q, k, qw, kw, cos, sin, 1e-6, False)
    np.testing.assert_allclose(npf(qo)[0], rq, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(npf(ko)[0], rk, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(npf(rstd), rr, rtol=2e-6)


def test_strided_fused_projection_and_misaligned(mga, dev):
    """q / k as views of a fused qkv projection output (the reference's
    forward_qkv_proj split, modeling_qwen3.py:249-252), and a base address one
    element off (element-access path)."""
    S, Hq, Hkv, D = 200, 8, 2, 128
    g = torch.Generator(device=dev).manual_seed(11)
    qkv = torch.randn(1, S, (Hq + 2 * Hkv) * D, generator=g, device=dev).bfloat16()
    qf, kf, _ = qkv.split([Hq * D, Hkv * D, Hkv * D], dim=-1)
    q, k = qf.view(1, S, Hq, D), kf.view(1, S, Hkv, D)
    _, _, qw, kw, cos, sin = make(S, Hq, Hkv, D, torch.bfloat16, dev, seed=12)
    qo, ko, _ = run_fwd(mga, q, k, qw, kw, cos, sin)
    rq, rk, _ = oracle_fwd(q, k, qw, kw, cos, sin, 1e-6, True)
    check_bf16("fused q", npf(qo)[0], rq)
    check_bf16("fused k", npf(ko)[0], rk)
    flat = torch.randn(S * Hq * D + 1, generator=g, device=dev).bfloat16()
    q1 = flat[1:].view(1, S, Hq, D)
    qo, ko, _ = run_fwd(mga, q1, k, qw, kw, cos, sin)
    rq, _, _ = oracle_fwd(q1, k, qw, kw, cos, sin, 1e-6, True)
    check_bf16("misaligned q", npf(qo)[0], rq)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("S,Hq,Hkv,D", [(512, 32, 8, 128), (65, 6, 3, 96), (17, 4, 2, 64)])
def test_backward_against_oracle(mga, dev, dtype, S, Hq, Hkv, D):
    q, k, qw, kw, cos, sin = make(S, Hq, Hkv, D, dtype, dev, seed=S + 1)
    qg, kg = q.clone().requires_grad_(), k.clone().requires_grad_()
    eq, ek = mga.qk_norm_rope(qg, kg, qw, kw, cos, sin, 1e-6)
    g = torch.Generator(device=dev).manual_seed(5)
    gq = torch.randn(eq.shape, generator=g, device=dev).to(dtype)
    gk = torch.randn(ek.shape, generator=g, device=dev).to(dtype)
    torch.autograd.backward([eq, ek], [gq, gk])
    torch.cuda.synchronize()
    c, s = npf(cos)[0], npf(sin)[0]
    for name, x, w, gr, got in (("dq", q, qw, gq, qg.grad), ("dk", k, kw, gk, kg.grad)):
        ref = qr.norm_rope_grad(npf(x)[0], npf(w), c, s, npf(gr.transpose(1, 2))[0], 1e-6)
        assert got.dtype == dtype and got.shape == x.shape
        err = np.abs(npf(got)[0] - ref)
        scale = np.abs(ref).max()
        print(f"  {dtype} {name}: max-abs {err.max():.3e} (scale {scale:.3e})", flush=True)
        if dtype == torch.bfloat16:
            assert (err <= 2.0 ** -8 * np.abs(ref) + 1e-5 * scale).all(), name
        elif dtype == torch.float16:
            assert (err <= 2.0 ** -11 * np.abs(ref) + 1e-5 * scale).all(), name
        else:
            assert (err <= 1e-5 * np.abs(ref) + 1e-6 * scale).all(), name


def test_argument_errors(mga, dev):
    q, k, qw, kw, cos, sin = make(8, 2, 1, 64, torch.bfloat16, dev)
    with pytest.raises(NotImplementedError):
        mga.qk_norm_rope(q, k, qw.clone().requires_grad_(), kw, cos, sin)
    with torch.no_grad():   # frozen use needs no weight gradient
        mga.qk_norm_rope(q, k, qw.clone().requires_grad_(), kw, cos, sin)
    with pytest.raises(TypeError):
        mga.qk_norm_rope(q, k, qw.float(), kw, cos, sin)
    with pytest.raises(ValueError):
        mga.qk_norm_rope(q, k, qw, kw, cos[:, :4], sin[:, :4])
    with pytest.raises(RuntimeError):
        mga.qk_norm_rope(q.cpu(), k.cpu(), qw.cpu(), kw.cpu(), cos.cpu(), sin.cpu())
    big = torch.zeros(1, 8, 2, 256, device=dev, dtype=torch.bfloat16)
    with pytest.raises(Exception, match="head_dim"):
        mga.qk_norm_rope(big, big[:, :, :1], torch.ones(256, device=dev, dtype=torch.bfloat16),
                         torch.ones(256, device=dev, dtype=torch.bfloat16),
                         torch.ones(1, 8, 256, device=dev, dtype=torch.bfloat16),
                         torch.zeros(1, 8, 256, device=dev, dtype=torch.bfloat16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("P", [0, 77])
def test_stage_into_cache_matches_update_path(mga, dev, dtype, P):
    """qk_norm_rope_stage writes the chunk's post-RoPE keys and its values into
    the cache rows [P, P + S) in the norm / RoPE launch, and update() then
    copies nothing. Against the copy path (qk_norm_rope, then update's append)
    on the same inputs: the cache buffers bit-equal after the update, the
    query embedding and the q / k / v gradients bit-equal, and after
    commit_regular (the fused path re-stages the regular rows from the
    projections) the prefix bit-equal again, i.e. equal to the reference's
    gather + cat of the post-RoPE keys (collator.py:270-287)."""
    from importlib import import_module
    rope = import_module("mtp-glora_amd.rope")
    S, Hq, Hkv, D = 300, 8, 2, 128
    q, k, qw, kw, cos, sin = make(S, Hq, Hkv, D, dtype, dev, seed=21 + P, pos0=P)
    g = torch.Generator(device=dev).manual_seed(22 + P)
    v = torch.randn(1, S, Hkv, D, generator=g, device=dev).to(dtype)
    kp = torch.randn(1, Hkv, P, D, generator=g, device=dev).to(dtype)
    vp = torch.randn(1, Hkv, P, D, generator=g, device=dev).to(dtype)
    regular = torch.rand(S, generator=g, device=dev) < 0.8
    idx = torch.nonzero(regular).flatten().to(torch.int32)
    R = idx.numel()
    up = [torch.randn(shape, generator=g, device=dev).to(dtype) for shape in
          ((1, Hq, S, D), (1, Hkv, P + S, D), (1, Hkv, P + S, D))]
    res = []
    for fused in (False, True):
        cache = mga.StreamingKVCache(capacity=P + S + 16, num_layers=1)
        if P:
            cache.append_prefix([kp], [vp])
        qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
        if fused:
            qe, ke, ve = rope.qk_norm_rope_stage(qg, kg, vg, qw, kw, cos, sin, 1e-6, cache, 0)
            assert ke.data_ptr() == cache.key_buffer(0)[:, P].data_ptr()
        else:
            qe, ke = mga.qk_norm_rope(qg, kg, qw, kw, cos, sin, 1e-6)
            ve = vg.transpose(1, 2)
        kf, vf = cache.update(ke, ve, 0)
        after_update = (cache.key_buffer(0)[:, :P + S].clone(), cache.value_buffer(0)[:, :P + S].clone())
        torch.autograd.backward([qe, kf, vf], up)
        cache.commit_regular(idx, R)
        torch.cuda.synchronize()
        after_commit = (cache.key_buffer(0)[:, :P + R].clone(), cache.value_buffer(0)[:, :P + R].clone())
        res.append((qe.detach(), after_update, after_commit, qg.grad, kg.grad, vg.grad, ke.detach()))
    (q0, u0, c0, *g0, k0), (q1, u1, c1, *g1, _) = res
    assert torch.equal(q0, q1)
    for a, b in zip(u0, u1):
        assert torch.equal(a, b)
    for a, b in zip(c0, c1):
        assert torch.equal(a, b)
    for a, b in zip(g0, g1):
        assert a is not None and torch.equal(a, b)
    # the committed prefix is the reference chain: cat(prefix, post-RoPE keys[idx])
    assert torch.equal(c1[0][:, P:], k0[0][:, idx.long()])
    assert torch.equal(c1[1][:, P:], v.transpose(1, 2)[0][:, idx.long()])
