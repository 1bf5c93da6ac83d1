"""The reference's own token layout on the GPU.

The reference's dataset makes every response token an anchor and labels a
mask token only when the token it predicts exists (dataset.py:25-56), so a
sequence ends in partly labelled blocks whose gate-0 mask tokens act as x keys
for every later query without being cached. Its collator cuts the sequence at
whole blocks and pads the last chunk to a bucket (collator.py:104-175). Here a
whole such sequence streams through StreamingKVCacheManager and
StreamingKVCache chunk by chunk (trainer.py:95-136). Every chunk's BlockMask is
compared bit for bit with torch's create_block_mask on the reference mask_mod
(on the GPU) and with the oracle. o, lse, dQ, dK and dV are compared with the
float64 oracle (max-abs 2e-2, mean-abs 2e-3; each gradient within that bound or
within 2x the error of the reference's rounding model on the same inputs, see
gpu_helpers.check_grad). The cache after every carry-over
equals the reference's split + gather + cat chain bit for bit.

A second test feeds arbitrary gate vectors (pads, x and m tokens in any
order, pads in the middle of a chunk) through the same path.
"""
import numpy as np
import pytest
import torch

from gpu_helpers import check, check_grad, f64, round_to, rounding_model_grad_errors
from oracle import flex_ref as fr
from oracle import mtp_oracle as mo

pytestmark = pytest.mark.gpu

NAMES = ["kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
         "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices"]


def _rand(shape, gen, dev, std=0.5, dtype=torch.bfloat16):
    return (torch.randn(*shape, generator=gen, device=dev) * std).to(dtype)


def _check_block_mask(bm, gate, P, dev):
    want = mo.block_mask_mtp(gate, P)
    ref = fr.block_mask_tensors(fr.reference_block_mask(torch.tensor(gate, device=dev)[None], P, device=dev))
    for n in NAMES:
        got = getattr(bm, n).cpu().numpy()
        assert np.array_equal(got, want[n]), n
        assert np.array_equal(got, ref[n]), n
    assert np.array_equal(bm.mtp_code.cpu().numpy(), mo.mtp_codes(gate, P))


def _check_attention(gate, P, q, kp, vp, k, v, do, o, lse, D):
    """With every response token an anchor, a few regular keys collect the
    probability of hundreds of rows of G heads, so |dV| reaches 7, where one
    bf16 rounding is 1.6e-2: each gradient is held to 2x the error of the
    reference's rounding model on the same inputs, or to the absolute bound,
    whichever is larger (check_grad)."""
    allowed = mo.mtp_mask_dense(gate, P)
    qn = f64(q)[0]
    kn = np.concatenate([f64(kp)[0], f64(k)[0]], axis=1)
    vn = np.concatenate([f64(vp)[0], f64(v)[0]], axis=1)
    on, lsen = mo.attention_fwd(qn, kn, vn, allowed, D ** -0.5)
    check("o", f64(o)[0].transpose(1, 0, 2), on)
    got_lse = f64(lse)[0]
    assert np.array_equal(np.isneginf(got_lse), np.isneginf(lsen))
    fin = np.isfinite(lsen)
    check("lse", got_lse[fin], lsen[fin])
    dqn, dkn, dvn = mo.attention_bwd(qn, kn, vn, on, lsen, f64(do)[0].transpose(1, 0, 2), allowed,
                                     D ** -0.5, grad_start=P)
    don = f64(do)[0].transpose(1, 0, 2)
    model = rounding_model_grad_errors(qn, kn, vn, don, allowed, D ** -0.5, P, round_to(q.dtype))
    check_grad("dq", f64(q.grad)[0], dqn, model["dq"])
    check_grad("dk", f64(k.grad)[0], dkn[:, -k.shape[2]:], model["dk"])
    check_grad("dv", f64(v.grad)[0], dvn[:, -v.shape[2]:], model["dv"])


@pytest.mark.parametrize("case", [
    # prompt, response tokens, draft length, chunk size, min chunk size, heads
    dict(n_in=300, n_out=700, D=4, C=1024, mn=512, Hq=4, Hkv=2, hd=128),
    dict(n_in=45, n_out=260, D=8, C=768, mn=256, Hq=8, Hkv=2, hd=128),
    dict(n_in=17, n_out=400, D=3, C=640, mn=512, Hq=4, Hkv=1, hd=64),
], ids=lambda c: f"in{c['n_in']}_out{c['n_out']}_D{c['D']}")
def test_reference_layout_stream(mga, dev, case):
    """Prompt + every response token an anchor, chunked and padded as the
    collator does; the last chunk holds the partly labelled tail blocks and
    its bucket padding."""
    seq = mo.insert_mask_tokens(case["n_in"], case["n_out"], case["D"])
    chunks = mo.chunk_sequence(seq, case["C"], case["D"], case["mn"])
    assert len(chunks) >= 2
    tail = chunks[-1]
    assert ((tail.gate == 0) & (tail.regular == 0)).any(), "the last chunk must hold gate-0 mask tokens"
    Hq, Hkv, hd = case["Hq"], case["Hkv"], case["hd"]
    gen = torch.Generator(device=dev).manual_seed(7)
    mgr = mga.StreamingKVCacheManager(capacity=len(seq.gate) + 256)
    cache = mgr.new_cache(num_layers=1)
    ref_k = torch.zeros(1, Hkv, 0, hd, device=dev, dtype=torch.bfloat16)
    ref_v = ref_k.clone()
    P = 0
    for c, ch in enumerate(chunks):
        S = len(ch.gate)
        print(f"chunk {c}: S={S} P={P} gate-0 masks={int(((ch.gate == 0) & (ch.regular == 0)).sum())} "
              f"pads={int((ch.gate == -1).sum())}", flush=True)
        data = {"input_ids": torch.zeros(1, S, dtype=torch.long, device=dev),
                "gate_mask": torch.tensor(ch.gate, device=dev)[None],
                "regular_token_mask": torch.tensor(ch.regular, device=dev)[None],
                "position_ids": torch.tensor(ch.position, device=dev)[None]}
        data = mgr.prepare_data_with_kv_cache(data)
        bm = data["attention_mask"]
        _check_block_mask(bm, ch.gate, P, dev)
        assert torch.equal(data["gate_mask"][0, :, 0].cpu(), torch.tensor(ch.gate).clamp(min=0))
        q = _rand((1, S, Hq, hd), gen, dev).transpose(1, 2).requires_grad_()
        k = _rand((1, S, Hkv, hd), gen, dev).transpose(1, 2).requires_grad_()
        v = _rand((1, S, Hkv, hd), gen, dev).transpose(1, 2).requires_grad_()
        do = _rand((1, S, Hq, hd), gen, dev, std=1.0)
        kf, vf = cache.update(k, v, 0)
        assert torch.equal(kf, torch.cat([ref_k, k.detach()], dim=2))
        o, lse = mga.mtp_attention(q, kf, vf, bm, hd ** -0.5)
        o.backward(do)
        torch.cuda.synchronize()
        _check_attention(ch.gate, P, q, ref_k, ref_v, k, v, do, o, lse, hd)
        if c + 1 < len(chunks):
            cache = mgr.extract_regular_kv_cache_for_next_chunk(data, cache)
            reg = torch.tensor(ch.regular, device=dev)[None]
            _, ref_k = fr.reference_cache_ops(ref_k, k.detach(), reg)
            _, ref_v = fr.reference_cache_ops(ref_v, v.detach(), reg)
            got_k, got_v = cache[0]
            assert torch.equal(got_k, ref_k) and torch.equal(got_v, ref_v)
            P += int(ch.regular.sum())
            assert mgr.past_seen_tokens == P == cache.prefix_len


@pytest.mark.parametrize("seed,S,P,probs", [
    (0, 700, 300, (0.1, 0.5, 0.4)),
    (1, 333, 0, (0.3, 0.3, 0.4)),
    (2, 1000, 1111, (0.05, 0.2, 0.75)),   # mask-token heavy
    (3, 260, 520, (0.6, 0.2, 0.2)),       # pad heavy
    (4, 900, 256, None),                  # structured runs
], ids=lambda x: str(x))
def test_arbitrary_gates(mga, dev, seed, S, P, probs):
    """Gate vectors drawn freely from {-1, 0, 1}: pads in the middle of a
    chunk, mask tokens with no anchor, long runs of each. The predicate of
    collator.py:311-355 is defined for any such vector; the kernels' single
    ordered compare relies only on num_prefix_x never decreasing."""
    rng = np.random.default_rng(seed)
    if probs is None:
        # mostly x (full tiles occur), a run of pads mid-chunk, a run of m
        # tokens with no anchor and a trailing pad run
        gate = np.zeros(S, np.int64)
        gate[400:410] = -1
        gate[600:640] = 1
        gate[-30:] = -1
    else:
        gate = rng.choice(np.array([-1, 0, 1], np.int64), size=S, p=probs)
    Hq, Hkv, hd = 4, 2, 128
    gen = torch.Generator(device=dev).manual_seed(seed)
    bm = mga.build_mtp_block_mask(torch.tensor(gate, device=dev)[None], P)
    _check_block_mask(bm, gate, P, dev)
    q = _rand((1, S, Hq, hd), gen, dev).transpose(1, 2).requires_grad_()
    k = _rand((1, S, Hkv, hd), gen, dev).transpose(1, 2).requires_grad_()
    v = _rand((1, S, Hkv, hd), gen, dev).transpose(1, 2).requires_grad_()
    kp = _rand((1, Hkv, P, hd), gen, dev)
    vp = _rand((1, Hkv, P, hd), gen, dev)
    do = _rand((1, S, Hq, hd), gen, dev, std=1.0)
    cache = mga.StreamingKVCache(capacity=P + S + 64, num_layers=1)
    if P:
        cache.append_prefix([kp], [vp])
    kf, vf = cache.update(k, v, 0)
    o, lse = mga.mtp_attention(q, kf, vf, bm, hd ** -0.5)
    o.backward(do)
    torch.cuda.synchronize()
    _check_attention(gate, P, q, kp, vp, k, v, do, o, lse, hd)
