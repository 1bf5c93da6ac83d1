"""HIP MTP attention forward/backward against the float64 CPU oracle (small
and medium shapes) and an fp32 torch dense reference on the GPU (full config
sizes). Tolerance (bf16 operands): max-abs <= 2e-2, mean-abs <= 2e-3 on
outputs and on every gradient; LSE within the same bounds; cache contents
bit-exact. fp16 operands (three more mantissa bits than bf16, so every
rounding the kernels share with the reference's flex path -- the
probabilities and dS before their products, the outputs -- is 8x smaller):
max-abs <= 4e-3, mean-abs <= 4e-4, gradients with the max bound relative
above magnitude 1. fp32 operands (fp32 MFMAs, no 16-bit rounding anywhere):
max-abs <= 1e-5, mean-abs <= 1e-6, relative above magnitude 1."""
import numpy as np
import pytest
import torch

from gpu_helpers import (MAX_ABS, MEAN_ABS, check, chunk_layout, f64, qkv, round_to,
                         rounding_model_grad_errors, torch_dense_reference)
from oracle import mtp_oracle as mo

pytestmark = pytest.mark.gpu


def run_case(mga, dev, n_reg, n_anchor, draft, P, Hq, Hkv, D, dtype=torch.bfloat16, seed=0,
             pad=0, tail=False, every=None, use_cache=True, std=0.5):
    print(f"case n_reg={n_reg} anchors={n_anchor} draft={draft} P={P} Hq={Hq} Hkv={Hkv} D={D} "
          f"{dtype} pad={pad} tail={tail} cache={use_cache} std={std}", flush=True)
    seq = chunk_layout(n_reg, n_anchor, draft, P, seed=seed, pad=pad, tail=tail, every=every)
    S = len(seq.gate)
    q, k, v, kp, vp, do = qkv(S, P, Hq, Hkv, D, dtype, dev, seed=seed, std=std)
    q.requires_grad_()
    k.requires_grad_()
    v.requires_grad_()
    bm = mga.build_mtp_block_mask(torch.tensor(seq.gate, device=dev)[None], P)
    if use_cache:
        cache = mga.StreamingKVCache(capacity=P + S + 64, num_layers=1)
        if P:
            cache.append_prefix([kp], [vp])
        kf, vf = cache.update(k, v, 0)
    else:
        kf = torch.cat([kp, k], dim=2)
        vf = torch.cat([vp, v], dim=2)
    o, lse = mga.mtp_attention(q, kf, vf, bm, D ** -0.5)
    o.backward(do)
    torch.cuda.synchronize()
    return seq, q, k, v, kp, vp, do, o, lse


F16_MAX_ABS = 4e-3
F16_MEAN_ABS = 4e-4
F32_MAX_ABS = 1e-5
F32_MEAN_ABS = 1e-6


def compare_oracle(seq, P, q, k, v, kp, vp, do, o, lse, D, grad_start, max_abs=MAX_ABS, mean_abs=MEAN_ABS,
                   scaled=False, tensor_scale=False):
    """scaled: max bounds relative above magnitude 1; tensor_scale: bounds
    times max(1, max |ref|) of each tensor (gpu_helpers.check)."""
    allowed = mo.mtp_mask_dense(seq.gate, P)
    qn = f64(q)[0]
    kn = np.concatenate([f64(kp)[0], f64(k)[0]], axis=1)
    vn = np.concatenate([f64(vp)[0], f64(v)[0]], axis=1)
    on, lsen = mo.attention_fwd(qn, kn, vn, allowed, D ** -0.5)
    tol = dict(max_abs=max_abs, mean_abs=mean_abs, tensor_scale=tensor_scale)
    check("o", f64(o)[0].transpose(1, 0, 2), on, **tol, scale_above_one=scaled)
    got_lse = f64(lse)[0]
    assert np.array_equal(np.isneginf(got_lse), np.isneginf(lsen))
    fin = np.isfinite(lsen)
    check("lse", got_lse[fin], lsen[fin], **tol, scale_above_one=scaled)
    dqn, dkn, dvn = mo.attention_bwd(qn, kn, vn, on, lsen, f64(do)[0].transpose(1, 0, 2),
                                     allowed, D ** -0.5, grad_start=grad_start)
    check("dq", f64(q.grad)[0], dqn, **tol, scale_above_one=scaled)
    check("dk", f64(k.grad)[0], dkn[:, -k.shape[2]:], **tol, scale_above_one=scaled)
    check("dv", f64(v.grad)[0], dvn[:, -v.shape[2]:], **tol, scale_above_one=scaled)


SMALL = [
    dict(n_reg=256, n_anchor=16, draft=4, P=0, Hq=4, Hkv=2, D=128),
    dict(n_reg=256, n_anchor=16, draft=4, P=256, Hq=4, Hkv=2, D=128),
    dict(n_reg=300, n_anchor=25, draft=4, P=200, Hq=8, Hkv=2, D=128, pad=37),   # ragged S and P
    dict(n_reg=200, n_anchor=50, draft=8, P=384, Hq=4, Hkv=1, D=128),           # mask heavy, G=4
    dict(n_reg=256, n_anchor=16, draft=4, P=128, Hq=4, Hkv=2, D=64),            # config-1 head_dim
    dict(n_reg=180, n_anchor=20, draft=4, P=96, Hq=2, Hkv=2, D=64, tail=True, pad=20),  # MHA
    dict(n_reg=60, n_anchor=5, draft=2, P=0, Hq=4, Hkv=2, D=128, pad=3),        # S < 128
    dict(n_reg=200, n_anchor=20, draft=4, P=130, Hq=8, Hkv=1, D=128),           # G = 8: two head slices
    dict(n_reg=220, n_anchor=30, draft=3, P=70, Hq=8, Hkv=2, D=64, pad=9),      # G = 4 at head_dim 64
    dict(n_reg=200, n_anchor=20, draft=4, P=150, Hq=7, Hkv=1, D=128),           # G = 7 (28 / 4 heads): one head per workgroup
    dict(n_reg=180, n_anchor=15, draft=4, P=64, Hq=6, Hkv=2, D=128, pad=5),     # G = 3
    dict(n_reg=160, n_anchor=12, draft=4, P=90, Hq=12, Hkv=2, D=64),            # G = 6: two heads per workgroup
]


@pytest.mark.parametrize("c", SMALL)
def test_attention_small_bf16(mga, dev, c):
    out = run_case(mga, dev, **c)
    seq, q, k, v, kp, vp, do, o, lse = out
    compare_oracle(seq, c["P"], q, k, v, kp, vp, do, o, lse, c["D"], grad_start=c["P"])


@pytest.mark.parametrize("c", SMALL)
def test_attention_small_fp16(mga, dev, c):
    """fp16 operands run the fp16 MFMAs (probabilities and dS rounded to
    fp16, as the reference's flex kernels round them to the operand dtype)."""
    seq, q, k, v, kp, vp, do, o, lse = run_case(mga, dev, dtype=torch.float16, seed=3, **c)
    assert o.dtype == torch.float16 and q.grad.dtype == torch.float16 and k.grad.dtype == torch.float16
    compare_oracle(seq, c["P"], q, k, v, kp, vp, do, o, lse, c["D"], grad_start=c["P"],
                   max_abs=F16_MAX_ABS, mean_abs=F16_MEAN_ABS, scaled=True)


# Keys of at least 16 tiles and at most one round of items per XCD: the
# forward and the dQ pass run every item as two-group workgroups (even and
# odd tiles of the item's list, merged through LDS). Configs 2 and 4 run the
# mixed launches (the last round two-group) in test_attention_full_config.
SPLIT = [
    dict(n_reg=800, n_anchor=50, draft=4, P=1536, Hq=8, Hkv=2, D=128, pad=11),
    dict(n_reg=700, n_anchor=60, draft=4, P=1800, Hq=4, Hkv=1, D=64, tail=True),
    dict(n_reg=600, n_anchor=40, draft=4, P=1700, Hq=8, Hkv=4, D=128),   # G = 2: 64 rows per workgroup
    dict(n_reg=500, n_anchor=30, draft=4, P=1600, Hq=8, Hkv=1, D=128),   # G = 8: two head slices
]


@pytest.mark.parametrize("c", SPLIT)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_attention_two_group_items(mga, dev, c, dtype):
    seq, q, k, v, kp, vp, do, o, lse = run_case(mga, dev, dtype=dtype, seed=9, **c)
    tol = dict(max_abs=F16_MAX_ABS, mean_abs=F16_MEAN_ABS, scaled=True) if dtype == torch.float16 else {}
    compare_oracle(seq, c["P"], q, k, v, kp, vp, do, o, lse, c["D"], grad_start=c["P"], **tol)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_attention_large_logits(mga, dev, dtype):
    """q, k ~ N(0, 2^2): scaled scores spread over tens of log2 units, so the
    forward's lazy softmax offset keeps leaving its bound (2^15 per
    probability for fp16, whose largest finite is 65504; 2^20 for bf16) and
    the exact-max recomputation runs on many steps. Outputs and LSE: the
    dtype's standard bounds, relative above magnitude 1 (v ~ N(0, 2^2) puts
    outputs near 6, where one bf16 rounding is 1.6e-2). Gradients grow to |dq| ~ 13 here and dS to tens
    of units, so the 16-bit roundings of P and dS alone (the reference's
    rounding points) cost more than the O(1)-scale bounds: each gradient must
    stay within 2x the max- and mean-abs error of that rounding model
    (rounding_model_grad_errors: the reference's cast points, delta from the
    stored output and the 16-bit gradient stores included) on the same
    inputs; the factor covers fp32 sums in another order and probabilities
    that round the other way. dS is formed from the fp32 P in both passes and
    the forward's row sums from the fp32 probabilities, as the reference
    does."""
    c = dict(n_reg=320, n_anchor=24, draft=4, P=192, Hq=4, Hkv=2, D=128)
    seq, q, k, v, kp, vp, do, o, lse = run_case(mga, dev, dtype=dtype, seed=11, std=2.0, **c)
    P, D = c["P"], c["D"]
    lse_np = f64(lse)[0]
    print(f"  lse range {lse_np[np.isfinite(lse_np)].min():.1f} .. {lse_np.max():.1f}", flush=True)
    tol = dict(max_abs=F16_MAX_ABS, mean_abs=F16_MEAN_ABS) if dtype == torch.float16 else \
        dict(max_abs=MAX_ABS, mean_abs=MEAN_ABS)
    allowed = mo.mtp_mask_dense(seq.gate, P)
    qn = f64(q)[0]
    kn = np.concatenate([f64(kp)[0], f64(k)[0]], axis=1)
    vn = np.concatenate([f64(vp)[0], f64(v)[0]], axis=1)
    don = f64(do)[0].transpose(1, 0, 2)
    on, lsen = mo.attention_fwd(qn, kn, vn, allowed, D ** -0.5)
    check("o", f64(o)[0].transpose(1, 0, 2), on, **tol, scale_above_one=True)
    fin = np.isfinite(lsen)
    assert np.array_equal(np.isneginf(lse_np), np.isneginf(lsen))
    check("lse", lse_np[fin], lsen[fin], **tol, scale_above_one=True)
    dqn, dkn, dvn = mo.attention_bwd(qn, kn, vn, on, lsen, don, allowed, D ** -0.5, grad_start=P)
    model = rounding_model_grad_errors(qn, kn, vn, don, allowed, D ** -0.5, P, round_to(dtype))
    for name, got, ref in (("dq", q.grad, dqn), ("dk", k.grad, dkn), ("dv", v.grad, dvn)):
        mx, mn = model[name]
        err = np.abs(f64(got)[0] - ref)
        print(f"  {name} rounding model: max-abs {mx:.3e} mean-abs {mn:.3e}; kernel / model: "
              f"max {err.max() / mx:.2f} mean {err.mean() / mn:.2f}", flush=True)
        check(name, f64(got)[0], ref, max_abs=2 * mx, mean_abs=2 * mn)


@pytest.mark.parametrize("c", SMALL)
def test_attention_small_fp32(mga, dev, c):
    """fp32 operands run the fp32 MFMAs: fp32 products, softmax and
    gradients, as the reference computes an fp32 model's attention."""
    seq, q, k, v, kp, vp, do, o, lse = run_case(mga, dev, dtype=torch.float32, seed=5, **c)
    assert o.dtype == torch.float32 and q.grad.dtype == torch.float32 and k.grad.dtype == torch.float32
    compare_oracle(seq, c["P"], q, k, v, kp, vp, do, o, lse, c["D"], grad_start=c["P"],
                   max_abs=F32_MAX_ABS, mean_abs=F32_MEAN_ABS, scaled=True)


def test_attention_large_logits_fp32(mga, dev):
    """The large-logit case of the 16-bit test in fp32: no 16-bit rounding,
    so the fp32 bounds hold, scaled by each tensor's largest magnitude (the
    raw scores reach about 45 here, where fp32 spacing is 4e-6, so every
    probability carries a relative error near 1e-6; an output summed from
    terms of magnitude 8 -- v ~ N(0, 2^2) -- then has an absolute error near
    1e-5 whatever its own size)."""
    c = dict(n_reg=320, n_anchor=24, draft=4, P=192, Hq=4, Hkv=2, D=128)
    seq, q, k, v, kp, vp, do, o, lse = run_case(mga, dev, dtype=torch.float32, seed=11, std=2.0, **c)
    compare_oracle(seq, c["P"], q, k, v, kp, vp, do, o, lse, c["D"], grad_start=c["P"],
                   max_abs=F32_MAX_ABS, mean_abs=F32_MEAN_ABS, tensor_scale=True)


def test_plain_key_tensor_gets_full_gradient(mga, dev):
    """Keys passed as one plain tensor (e.g. from a DynamicCache): every key
    row, prefix included, receives its gradient."""
    c = dict(n_reg=200, n_anchor=20, draft=4, P=128, Hq=4, Hkv=2, D=128)
    seq = chunk_layout(200, 20, 4, 128, seed=4)
    S = len(seq.gate)
    q, k, v, kp, vp, do = qkv(S, 128, 4, 2, 128, torch.bfloat16, dev, seed=4)
    kf = torch.cat([kp, k], dim=2).requires_grad_()
    vf = torch.cat([vp, v], dim=2).requires_grad_()
    q.requires_grad_()
    bm = mga.build_mtp_block_mask(torch.tensor(seq.gate, device=dev)[None], 128)
    o, lse = mga.mtp_attention(q, kf, vf, bm, 128 ** -0.5)
    o.backward(do)
    allowed = mo.mtp_mask_dense(seq.gate, 128)
    on, lsen = mo.attention_fwd(f64(q)[0], f64(kf)[0], f64(vf)[0], allowed, 128 ** -0.5)
    dqn, dkn, dvn = mo.attention_bwd(f64(q)[0], f64(kf)[0], f64(vf)[0], on, lsen,
                                     f64(do)[0].transpose(1, 0, 2), allowed, 128 ** -0.5)
    check("o", f64(o)[0].transpose(1, 0, 2), on)
    check("dq", f64(q.grad)[0], dqn)
    check("dk", f64(kf.grad)[0], dkn)
    check("dv", f64(vf.grad)[0], dvn)


@pytest.mark.parametrize("heads,D,dtype", [((8, 2), 128, torch.bfloat16), ((6, 2), 128, torch.bfloat16),
                                            ((8, 2), 64, torch.bfloat16), ((4, 2), 128, torch.float16)],
                         ids=["G4", "G3", "G4-d64", "G2-fp16"])
def test_key_value_row_strides_differ(mga, dev, heads, D, dtype):
    """K and V as views of wider buffers with different row and head strides
    (the kernels stage each tile with its own tensor's stride); G = 4 and
    G = 2 take the forward's 8-wave pair form, G = 3 the 4-wave one. L = P + S
    is not a multiple of 64, so the last step of the key list is partly past
    L."""
    Hq, Hkv = heads
    P = 300
    print(f"row strides differ Hq={Hq} Hkv={Hkv} D={D} {dtype}", flush=True)
    seq = chunk_layout(260, 24, 4, P, seed=11)
    S = len(seq.gate)
    L = P + S
    q, k, v, kp, vp, do = qkv(S, P, Hq, Hkv, D, dtype, dev, seed=11)
    kbig = torch.zeros(1, Hkv, L, D + 64, dtype=dtype, device=dev)
    vbig = torch.zeros(1, Hkv, L, D + 192, dtype=dtype, device=dev)
    kf = kbig[..., :D]
    vf = vbig[..., 64:64 + D]
    kf.copy_(torch.cat([kp, k], dim=2))
    vf.copy_(torch.cat([vp, v], dim=2))
    assert kf.stride(2) != vf.stride(2) and kf.stride(1) != vf.stride(1)
    kf.requires_grad_()
    vf.requires_grad_()
    q.requires_grad_()
    bm = mga.build_mtp_block_mask(torch.tensor(seq.gate, device=dev)[None], P)
    o, lse = mga.mtp_attention(q, kf, vf, bm, D ** -0.5)
    o.backward(do)
    torch.cuda.synchronize()
    allowed = mo.mtp_mask_dense(seq.gate, P)
    kn, vn = f64(kf.detach())[0], f64(vf.detach())[0]
    on, lsen = mo.attention_fwd(f64(q)[0], kn, vn, allowed, D ** -0.5)
    dqn, dkn, dvn = mo.attention_bwd(f64(q)[0], kn, vn, on, lsen, f64(do)[0].transpose(1, 0, 2), allowed,
                                     D ** -0.5)
    tol = (dict(max_abs=F16_MAX_ABS, mean_abs=F16_MEAN_ABS) if dtype == torch.float16
           else dict(max_abs=MAX_ABS, mean_abs=MEAN_ABS))
    check("o", f64(o)[0].transpose(1, 0, 2), on, **tol)
    got_lse = f64(lse)[0]
    assert np.array_equal(np.isneginf(got_lse), np.isneginf(lsen))
    fin = np.isfinite(lsen)
    check("lse", got_lse[fin], lsen[fin], **tol)
    scaled = dtype == torch.float16   # fp16 gradients: max bound relative above magnitude 1
    check("dq", f64(q.grad)[0], dqn, **tol, scale_above_one=scaled)
    check("dk", f64(kf.grad)[0], dkn, **tol, scale_above_one=scaled)
    check("dv", f64(vf.grad)[0], dvn, **tol, scale_above_one=scaled)


def test_transformers_wrapper_contract(mga, dev):
    """Output [B, S, Hq, D] contiguous and LSE cast to the value dtype, as
    flex_attention_forward returns ([tf]integrations/flex_attention.py:346, 367)."""
    seq = chunk_layout(128, 8, 4, 0, seed=5)
    S = len(seq.gate)
    q, k, v, *_ = qkv(S, 0, 4, 2, 128, torch.bfloat16, dev)
    bm = mga.build_mtp_block_mask(torch.tensor(seq.gate, device=dev)[None], 0)
    o, lse = mga.mtp_attention_forward(torch.nn.Module(), q, k, v, bm, scaling=0.1, dropout=0.0,
                                       sliding_window=None)
    assert o.shape == (1, S, 4, 128) and o.is_contiguous() and lse.dtype == torch.bfloat16


@pytest.mark.parametrize("cfg", [
    dict(name="config2", n_reg=4096, n_anchor=256, draft=4, P=8192),
    dict(name="config5", n_reg=2048, n_anchor=512, draft=8, P=16384, every=4),
    # the last chunk of config 3's stream and of config 4's 32 full chunks
    dict(name="config3_last", n_reg=4096, n_anchor=512, draft=4, P=28672),
    dict(name="config4_last", n_reg=4096, n_anchor=256, draft=4, P=126976),
], ids=lambda c: c["name"])
def test_attention_full_config(mga, dev, cfg):
    """Full attention geometry of Qwen3-8B / Llama-3.1-8B (32 q / 8 kv heads,
    D = 128) against an fp32 dense reference on the GPU fed the same bf16
    values, up to config 4's 131 072-token cache."""
    full_config_case(mga, dev, cfg, torch.bfloat16)


# Config 2's chunk and prefix with other head geometries, each launching the
# dQ pass as 8-wave pair items plus a two-group last round: G = 2 (two heads
# per slice, 128 rows per item: 320 items), G = 8 (two slices of four heads:
# 640 items) and D = 64.
@pytest.mark.parametrize("heads", [dict(Hq=16, Hkv=8, D=128), dict(Hq=32, Hkv=4, D=128),
                                   dict(Hq=32, Hkv=8, D=64)],
                         ids=lambda h: f"hq{h['Hq']}_hkv{h['Hkv']}_d{h['D']}")
def test_attention_config2_head_geometries(mga, dev, heads):
    full_config_case(mga, dev, dict(n_reg=4096, n_anchor=256, draft=4, P=8192, **heads), torch.bfloat16)


def test_attention_full_config_fp16(mga, dev):
    """Config 2's geometry with fp16 operands, fp16 bounds."""
    full_config_case(mga, dev, dict(n_reg=4096, n_anchor=256, draft=4, P=8192), torch.float16,
                     max_abs=F16_MAX_ABS, mean_abs=F16_MEAN_ABS, grad_scaled=True)


def test_attention_full_config_fp32(mga, dev):
    """Config 2's geometry with fp32 operands against the fp32 dense
    reference (its own fp32 rounding included in the bound)."""
    full_config_case(mga, dev, dict(n_reg=4096, n_anchor=256, draft=4, P=8192), torch.float32,
                     max_abs=F32_MAX_ABS, mean_abs=F32_MEAN_ABS, grad_scaled=True)


def full_config_case(mga, dev, cfg, dtype, max_abs=MAX_ABS, mean_abs=MEAN_ABS, grad_scaled=False):
    Hq, Hkv, D = cfg.get("Hq", 32), cfg.get("Hkv", 8), cfg.get("D", 128)
    seq, q, k, v, kp, vp, do, o, lse = run_case(
        mga, dev, cfg["n_reg"], cfg["n_anchor"], cfg["draft"], cfg["P"], Hq, Hkv, D, seed=2,
        every=cfg.get("every"), dtype=dtype)
    P = cfg["P"]
    allowed = mo.mtp_mask_dense(seq.gate, P)
    kfull = torch.cat([kp, k.detach()], dim=2)
    vfull = torch.cat([vp, v.detach()], dim=2)
    ro, rlse, rdq, rdk, rdv = torch_dense_reference(q.detach(), kfull, vfull, allowed, D ** -0.5,
                                                    do=do, grad_start=P)
    tol = dict(max_abs=max_abs, mean_abs=mean_abs)
    check("o", f64(o)[0].transpose(1, 0, 2), ro.cpu().numpy(), **tol)
    check("lse", f64(lse)[0], rlse.cpu().numpy(), **tol, scale_above_one=grad_scaled)
    check("dq", f64(q.grad)[0], rdq.cpu().numpy(), **tol, scale_above_one=grad_scaled)
    check("dk", f64(k.grad)[0], rdk.cpu().numpy(), **tol, scale_above_one=grad_scaled)
    check("dv", f64(v.grad)[0], rdv.cpu().numpy(), **tol, scale_above_one=grad_scaled)
