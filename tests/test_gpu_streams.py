"""Configs 3 and 4 as chunk streams on the GPU, at full attention geometry
(32 query / 8 KV heads, head_dim 128, bf16), through StreamingKVCacheManager
and StreamingKVCache in the reference's loop order (trainer.py:95-136):
prepare -> per layer update + attention forward + backward -> carry-over
(not after the last chunk).

Config 3: 8 chunks of 4096 regular + 512 anchors x 4 mask rows, the prefix
growing 0 -> 28672, all 36 layers of Qwen3-8B with their own K/V. Every chunk's BlockMask
equals the oracle's bit for bit; after every carry-over each layer's cache
equals the reference's split + gather + cat chain (collator.py:270-287) bit
for bit; attention and gradients at chunks 0, 3 and 7 (layer 0, and the
last layer at chunk 7) are within the bf16
tolerance (max-abs 2e-2, mean-abs 2e-3) of an fp32 dense reference; each
gradient within that bound or within 2x the error of the reference's
rounding model on the same inputs (gpu_helpers.check_grad).

Config 4: one layer filled chunk by chunk (32 chunks of 4096 regular + 256 x
4) to a 131072-token cache, compared with the reference chain after every
carry-over; then the remainder chunk of the reference's layout (every
response token an anchor, the partly labelled tail blocks) padded to its
1024-row bucket (collator.py:158-166) at P = 131072, against the fp32 dense
reference, as is the last full chunk.
"""
import numpy as np
import pytest
import torch

from gpu_helpers import check, check_grad, f64, torch_dense_reference, torch_rounding_model_grads
from oracle import flex_ref as fr
from oracle import mtp_oracle as mo

pytestmark = pytest.mark.gpu

NAMES = ["kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
         "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices"]
HQ, HKV, HD = 32, 8, 128


def _chunk_dict(seq, dev):
    S = len(seq.gate)
    return {"input_ids": torch.zeros(1, S, dtype=torch.long, device=dev),
            "gate_mask": torch.tensor(seq.gate, device=dev)[None],
            "regular_token_mask": torch.tensor(seq.regular, device=dev)[None],
            "position_ids": torch.tensor(seq.position, device=dev)[None]}


def _projections(S, gen, dev):
    r = lambda shape, sd: (torch.randn(*shape, generator=gen, device=dev) * sd).bfloat16()
    q = r((1, S, HQ, HD), 0.5).transpose(1, 2).requires_grad_()
    k = r((1, S, HKV, HD), 0.5).transpose(1, 2).requires_grad_()
    v = r((1, S, HKV, HD), 0.5).transpose(1, 2).requires_grad_()
    do = r((1, S, HQ, HD), 1.0)
    return q, k, v, do


def _dense_check(tag, seq, P, q, k, v, do, o, lse, ref_k, ref_v):
    allowed = mo.mtp_mask_dense(seq.gate, P)
    kfull = torch.cat([ref_k, k.detach()], dim=2)
    vfull = torch.cat([ref_v, v.detach()], dim=2)
    ro, rlse, rdq, rdk, rdv = torch_dense_reference(q.detach(), kfull, vfull, allowed, HD ** -0.5,
                                                    do=do, grad_start=P)
    print(f"{tag}: dense reference at S={len(seq.gate)} P={P}", flush=True)
    check("o", f64(o)[0].transpose(1, 0, 2), ro.cpu().numpy())
    got_lse, want_lse = f64(lse)[0], rlse.double().cpu().numpy()
    # pad rows see no key: LSE -inf in both, the output 0 (checked above)
    assert np.array_equal(np.isneginf(got_lse), np.isneginf(want_lse))
    fin = np.isfinite(want_lse)
    check("lse", got_lse[fin], want_lse[fin])
    # at P = 0 the first keys of the chunk collect the probability of every
    # later row: |dV| reaches ~7, where one bf16 rounding is 1.6e-2; each
    # gradient is held to 2x the error of the reference's rounding points on
    # these inputs (or the absolute bound, whichever is larger)
    mq, mk, mv = torch_rounding_model_grads(q.detach(), kfull, vfull, allowed, HD ** -0.5, do, P, torch.bfloat16)
    check_grad("dq", f64(q.grad)[0], rdq.cpu().numpy(), mq.cpu().numpy())
    check_grad("dk", f64(k.grad)[0], rdk.cpu().numpy(), mk.cpu().numpy())
    check_grad("dv", f64(v.grad)[0], rdv.cpu().numpy(), mv.cpu().numpy())


def test_config3_stream(mga, dev):
    n_chunks, layers = 8, 36
    gen = torch.Generator(device=dev).manual_seed(33)
    seqs, P = [], 0
    for c in range(n_chunks):
        seqs.append(mo.synth_sequence(4096, mo.sample_anchors(4096, 512, 300 + c), 4, pos0=P))
        P += 4096
    mgr = mga.StreamingKVCacheManager(capacity=P + 6144 + 128)
    cache = mgr.new_cache(num_layers=layers)
    ref = [[torch.zeros(1, HKV, 0, HD, device=dev, dtype=torch.bfloat16)] * 2 for _ in range(layers)]
    P = 0
    for c, seq in enumerate(seqs):
        data = mgr.prepare_data_with_kv_cache(_chunk_dict(seq, dev))
        bm = data["attention_mask"]
        want = mo.block_mask_mtp(seq.gate, P)
        for n in NAMES:
            assert np.array_equal(getattr(bm, n).cpu().numpy(), want[n]), (c, n)
        S = len(seq.gate)
        kept = []
        for layer in range(layers):
            q, k, v, do = _projections(S, gen, dev)
            kf, vf = cache.update(k, v, layer)
            assert torch.equal(kf, torch.cat([ref[layer][0], k.detach()], dim=2))
            assert torch.equal(vf, torch.cat([ref[layer][1], v.detach()], dim=2))
            o, lse = mga.mtp_attention(q, kf, vf, bm, HD ** -0.5)
            o.backward(do)
            kept.append((q, k, v, do, o, lse))
        torch.cuda.synchronize()
        print(f"config 3 chunk {c}: S={S} P={P} done", flush=True)
        if c in (0, 3, 7):
            _dense_check(f"chunk {c} layer 0", seq, P, *kept[0], ref[0][0], ref[0][1])
        if c == 7:
            _dense_check(f"chunk {c} layer {layers - 1}", seq, P, *kept[-1], ref[-1][0], ref[-1][1])
        if c + 1 < n_chunks:
            cache = mgr.extract_regular_kv_cache_for_next_chunk(data, cache)
            reg = torch.tensor(seq.regular, device=dev)[None]
            for layer in range(layers):
                _, k, v, *_ = kept[layer]
                _, ref[layer][0] = fr.reference_cache_ops(ref[layer][0], k.detach(), reg)
                _, ref[layer][1] = fr.reference_cache_ops(ref[layer][1], v.detach(), reg)
                got_k, got_v = cache[layer]
                assert torch.equal(got_k, ref[layer][0]) and torch.equal(got_v, ref[layer][1]), (c, layer)
            P += 4096
            assert mgr.past_seen_tokens == P == cache.prefix_len
        del kept
    assert P == 28672


def test_config4_stream_and_remainder(mga, dev):
    n_full = 32
    gen = torch.Generator(device=dev).manual_seed(44)
    # remainder chunk: the tail of a sequence in the reference's own layout,
    # cut and padded by the collator's rule
    tail_seq = mo.insert_mask_tokens(0, 180, 4)
    rem = mo.chunk_sequence(tail_seq, 4096, 4, 1024)
    assert len(rem) == 1 and len(rem[0].gate) == 1024 and (rem[0].gate == -1).sum() == 124
    rem_seq = rem[0]
    mgr = mga.StreamingKVCacheManager(capacity=n_full * 4096 + 5120 + 128)
    cache = mgr.new_cache(num_layers=1)
    ref_k = torch.zeros(1, HKV, 0, HD, device=dev, dtype=torch.bfloat16)
    ref_v = ref_k.clone()
    P = 0
    for c in range(n_full + 1):
        if c < n_full:
            seq = mo.synth_sequence(4096, mo.sample_anchors(4096, 256, 400 + c), 4, pos0=P)
        else:
            seq = mo.Sequence(rem_seq.gate, rem_seq.regular,
                              np.where(rem_seq.gate == -1, 0, rem_seq.position + P),
                              rem_seq.block, rem_seq.is_anchor)
        data = mgr.prepare_data_with_kv_cache(_chunk_dict(seq, dev))
        bm = data["attention_mask"]
        if c in (0, n_full - 1, n_full):
            want = mo.block_mask_mtp(seq.gate, P)
            for n in NAMES:
                assert np.array_equal(getattr(bm, n).cpu().numpy(), want[n]), (c, n)
        S = len(seq.gate)
        q, k, v, do = _projections(S, gen, dev)
        kf, vf = cache.update(k, v, 0)
        o, lse = mga.mtp_attention(q, kf, vf, bm, HD ** -0.5)
        o.backward(do)
        torch.cuda.synchronize()
        if c % 8 == 0 or c >= n_full - 1:
            print(f"config 4 chunk {c}: S={S} P={P} done", flush=True)
        if c >= n_full - 1:
            _dense_check(f"chunk {c}", seq, P, q, k, v, do, o, lse, ref_k, ref_v)
        if c < n_full:
            cache = mgr.extract_regular_kv_cache_for_next_chunk(data, cache)
            reg = torch.tensor(seq.regular, device=dev)[None]
            _, ref_k = fr.reference_cache_ops(ref_k, k.detach(), reg)
            _, ref_v = fr.reference_cache_ops(ref_v, v.detach(), reg)
            got_k, got_v = cache[0]
            assert torch.equal(got_k, ref_k) and torch.equal(got_v, ref_v), c
            P += 4096
            assert mgr.past_seen_tokens == P == cache.prefix_len
        del q, k, v, do, o, lse
    assert P == 131072
