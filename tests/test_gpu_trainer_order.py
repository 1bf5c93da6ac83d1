"""The trainer's ordering contract on the GPU (mtp_glora/trainer/trainer.py:95-136)
and the raise paths of the cache and the manager.

* A chunk without a labelled mask token (gate == 1) is skipped after
  ``prepare_data_with_kv_cache`` and before the forward and the carry-over
  (trainer.py:111, 116-117): its regular tokens never enter the cache, the next
  chunk is prepared against the unchanged prefix, and the next carry-over's
  position check prints the reference's mismatch message (the positions have
  moved on by the skipped chunk).
* A second sequence after ``reset_cache()`` (trainer.py:99-100) through the
  same manager and cache gives bit for bit what a fresh manager gives.
* Raise paths: commit with a layer that was never updated, a cache whose
  prefix disagrees with the manager, a full cache (prefix at capacity, and
  prefix + chunk past it), and a reset between update and carry-over.

Caches are compared bit for bit with the reference's split + gather + cat
chain (collator.py:270-287); attention and gradients with the float64 oracle
under the attention bounds (gradients within 2x the reference's rounding
model, see gpu_helpers.check_grad).
"""
import numpy as np
import pytest
import torch

from gpu_helpers import check, check_grad, f64, round_to, rounding_model_grad_errors
from oracle import flex_ref as fr
from oracle import mtp_oracle as mo

pytestmark = pytest.mark.gpu

HQ, HKV, HD = 4, 2, 128
NAMES = ["kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
         "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices"]


def _chunk(seq, dev):
    S = len(seq.gate)
    return {"input_ids": torch.zeros(1, S, dtype=torch.long, device=dev),
            "gate_mask": torch.tensor(seq.gate, device=dev)[None],
            "regular_token_mask": torch.tensor(seq.regular, device=dev)[None],
            "position_ids": torch.tensor(seq.position, device=dev)[None]}


def _proj(S, gen, dev):
    r = lambda shape, sd: (torch.randn(*shape, generator=gen, device=dev) * sd).bfloat16()
    q = r((1, S, HQ, HD), 0.5).transpose(1, 2).requires_grad_()
    k = r((1, S, HKV, HD), 0.5).transpose(1, 2).requires_grad_()
    v = r((1, S, HKV, HD), 0.5).transpose(1, 2).requires_grad_()
    do = r((1, S, HQ, HD), 1.0)
    return q, k, v, do


def _sequence(specs):
    """Chunks of (regular tokens, anchors) with positions running on across
    chunks, as the collator cuts one sequence; 0 anchors: no labelled mask
    token, a chunk the trainer skips."""
    seqs, pos = [], 0
    for c, (n_reg, n_anchor) in enumerate(specs):
        anchors = mo.sample_anchors(n_reg, n_anchor, 50 + c) if n_anchor else np.zeros(0, dtype=np.int64)
        seqs.append(mo.synth_sequence(n_reg, anchors, 4, pos0=pos))
        pos += n_reg
    return seqs


def _run_loop(mga, mgr, cache, seqs, layers, gen, dev, reset=True):
    """trainer.py:95-136 with the adapter's update + attention per layer: reset,
    then per chunk prepare -> skip without gate == 1 -> forward + backward ->
    carry-over unless last. Returns, per chunk, None (skipped) or (P, block
    mask, per-layer (q, k, v, do, o, lse) with gradients, per-layer caches
    after the carry-over)."""
    if reset:
        mgr.reset_cache()
    out = []
    for c, seq in enumerate(seqs):
        data = mgr.prepare_data_with_kv_cache(_chunk(seq, dev))
        if not bool((torch.tensor(seq.gate) == 1).any()):
            out.append(None)
            continue
        P = mgr.past_seen_tokens
        S = len(seq.gate)
        kept = []
        for layer in range(layers):
            q, k, v, do = _proj(S, gen, dev)
            kf, vf = cache.update(k, v, layer)
            o, lse = mga.mtp_attention(q, kf, vf, data["attention_mask"], HD ** -0.5)
            o.backward(do)
            kept.append((q, k, v, do, o, lse))
        caches = None
        if c < len(seqs) - 1:
            cache = mgr.extract_regular_kv_cache_for_next_chunk(data, cache)
            caches = [tuple(t.clone() for t in cache[layer]) for layer in range(layers)]
        torch.cuda.synchronize()
        out.append((P, data["attention_mask"], kept, caches))
    return out


def test_skipped_chunk_leaves_the_cache_unchanged(mga, dev, capsys):
    # chunk 1 has no anchor, so no labelled mask token: skipped
    seqs = _sequence([(256, 16), (200, 0), (256, 16), (128, 8)])
    layers = 2
    mgr = mga.StreamingKVCacheManager(capacity=2048)
    cache = mgr.new_cache(layers)
    gen = torch.Generator(device=dev).manual_seed(7)
    capsys.readouterr()
    res = _run_loop(mga, mgr, cache, seqs, layers, gen, dev)
    printed = capsys.readouterr().out
    assert res[1] is None
    # the prefix after chunk 0 is its 256 regular rows; chunk 1 adds nothing
    P0, _, kept0, caches0 = res[0]
    P2, bm2, kept2, caches2 = res[2]
    assert P0 == 0 and P2 == 256
    want = mo.block_mask_mtp(seqs[2].gate, 256)
    for n in NAMES:
        assert np.array_equal(getattr(bm2, n).cpu().numpy(), want[n]), n
    reg0 = torch.tensor(seqs[0].regular, device=dev)[None]
    reg2 = torch.tensor(seqs[2].regular, device=dev)[None]
    for layer in range(layers):
        empty = torch.zeros(1, HKV, 0, HD, device=dev, dtype=torch.bfloat16)
        _, k0 = fr.reference_cache_ops(empty, kept0[layer][1].detach(), reg0)
        _, v0 = fr.reference_cache_ops(empty, kept0[layer][2].detach(), reg0)
        assert torch.equal(caches0[layer][0], k0) and torch.equal(caches0[layer][1], v0)
        _, k2 = fr.reference_cache_ops(k0, kept2[layer][1].detach(), reg2)
        _, v2 = fr.reference_cache_ops(v0, kept2[layer][2].detach(), reg2)
        assert torch.equal(caches2[layer][0], k2) and torch.equal(caches2[layer][1], v2), layer
        if layer == 0:
            # chunk 2's attention ran against chunk 0's regular rows only
            q, k, v, do, o, lse = kept2[0]
            allowed = mo.mtp_mask_dense(seqs[2].gate, 256)
            qn = f64(q)[0]
            kn = np.concatenate([f64(k0)[0], f64(k)[0]], axis=1)
            vn = np.concatenate([f64(v0)[0], f64(v)[0]], axis=1)
            don = f64(do)[0].transpose(1, 0, 2)
            on, lsen = mo.attention_fwd(qn, kn, vn, allowed, HD ** -0.5)
            check("o", f64(o)[0].transpose(1, 0, 2), on)
            fin = np.isfinite(lsen)
            check("lse", f64(lse)[0][fin], lsen[fin])
            dqn, dkn, dvn = mo.attention_bwd(qn, kn, vn, on, lsen, don, allowed, HD ** -0.5, grad_start=256)
            model = rounding_model_grad_errors(qn, kn, vn, don, allowed, HD ** -0.5, 256, round_to(torch.bfloat16))
            check_grad("dq", f64(q.grad)[0], dqn, model["dq"])
            check_grad("dk", f64(k.grad)[0], dkn, model["dk"])
            check_grad("dv", f64(v.grad)[0], dvn, model["dv"])
    assert mgr.past_seen_tokens == 256 + 256
    # chunk 2's regular positions start after the skipped chunk's: the
    # reference's sanity check reports the mismatch, once (chunk 2's carry-over)
    assert printed.count("Sanity check failed. Position IDs mismatch.") == 1
    assert "self.past_seen_tokens: 256, num_new_regular_tokens: 256" in printed


def test_second_sequence_after_reset_matches_a_fresh_manager(mga, dev):
    first = _sequence([(300, 20), (260, 12), (200, 10)])
    second = _sequence([(240, 16), (280, 20), (150, 8)])
    layers = 2
    shared = mga.StreamingKVCacheManager(capacity=2048)
    cache = shared.new_cache(layers)
    _run_loop(mga, shared, cache, first, layers, torch.Generator(device=dev).manual_seed(1), dev)
    assert shared.past_seen_tokens == 300 + 260
    got = _run_loop(mga, shared, cache, second, layers, torch.Generator(device=dev).manual_seed(2), dev)
    fresh = mga.StreamingKVCacheManager(capacity=2048)
    want = _run_loop(mga, fresh, fresh.new_cache(layers), second, layers,
                     torch.Generator(device=dev).manual_seed(2), dev)
    for c, (a, b) in enumerate(zip(got, want)):
        Pa, bma, kepta, ca = a
        Pb, bmb, keptb, cb = b
        assert Pa == Pb, c
        for n in NAMES:
            assert torch.equal(getattr(bma, n), getattr(bmb, n)), (c, n)
        for la, lb in zip(kepta, keptb):
            for x, y in zip(la, lb):
                assert torch.equal(x.detach(), y.detach()), c
            for x, y in zip(la[:3], lb[:3]):
                assert torch.equal(x.grad, y.grad), c
        if ca is not None:
            for (ka, va), (kb, vb) in zip(ca, cb):
                assert torch.equal(ka, kb) and torch.equal(va, vb), c
    assert shared.past_seen_tokens == fresh.past_seen_tokens == 240 + 280


def test_raise_paths(mga, dev):
    seq = _sequence([(200, 12)])[0]
    S = len(seq.gate)
    gen = torch.Generator(device=dev).manual_seed(3)

    # a layer with no staged chunk: only layer 0 of 2 was updated
    mgr = mga.StreamingKVCacheManager(capacity=1024)
    cache = mgr.new_cache(2)
    data = mgr.prepare_data_with_kv_cache(_chunk(seq, dev))
    _, k, v, _ = _proj(S, gen, dev)
    cache.update(k.detach(), v.detach(), 0)
    with pytest.raises(RuntimeError, match="layer 1 has no staged chunk"):
        mgr.extract_regular_kv_cache_for_next_chunk(data, cache)

    # the cache's prefix disagrees with the manager's count
    mgr = mga.StreamingKVCacheManager(capacity=1024)
    cache = mgr.new_cache(1)
    data = mgr.prepare_data_with_kv_cache(_chunk(seq, dev))
    cache.update(k.detach(), v.detach(), 0)
    mgr.past_seen_tokens = 5
    with pytest.raises(RuntimeError, match="cache holds 0 prefix tokens but the manager has seen 5"):
        mgr.extract_regular_kv_cache_for_next_chunk(data, cache)

    # a reset between update and carry-over drops the staged chunk
    mgr = mga.StreamingKVCacheManager(capacity=1024)
    cache = mgr.new_cache(1)
    data = mgr.prepare_data_with_kv_cache(_chunk(seq, dev))
    cache.update(k.detach(), v.detach(), 0)
    mgr.reset_cache()
    with pytest.raises(RuntimeError, match="no staged chunk"):
        mgr.extract_regular_kv_cache_for_next_chunk(data, cache)
    # and the next sequence starts from an empty prefix
    data = mgr.prepare_data_with_kv_cache(_chunk(seq, dev))
    cache.update(k.detach(), v.detach(), 0)
    cache = mgr.extract_regular_kv_cache_for_next_chunk(data, cache)
    R = int(seq.regular.sum())
    assert cache.prefix_len == mgr.past_seen_tokens == R
    keep = torch.tensor(mo.regular_index(seq.regular), device=dev).long()
    assert torch.equal(cache[0][0], k.detach()[:, :, keep])

    # a full cache: prefix at capacity (no row P exists), then prefix + chunk past it
    for cap, P in ((64, 64), (S + 10, 20)):
        c2 = mga.StreamingKVCache(capacity=cap, num_layers=1)
        pk = torch.zeros(1, HKV, P, HD, device=dev, dtype=torch.bfloat16)
        c2.append_prefix([pk], [pk])
        assert c2.prefix_len == P
        with pytest.raises(RuntimeError, match="capacity"):
            c2.update(k.detach(), v.detach(), 0)
    # appending a prefix past capacity raises too
    c3 = mga.StreamingKVCache(capacity=32, num_layers=1)
    with pytest.raises(RuntimeError, match="capacity"):
        c3.append_prefix([torch.zeros(1, HKV, 40, HD, device=dev, dtype=torch.bfloat16)],
                         [torch.zeros(1, HKV, 40, HD, device=dev, dtype=torch.bfloat16)])
