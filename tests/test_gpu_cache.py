"""KV append / regular index / streaming cache on the GPU: bit-exact against
the reference's torch.cat + regular-token gather + cat (collator.py:273-282,
[tf]cache_utils.py:144-146)."""
import numpy as np
import pytest
import torch

from gpu_helpers import chunk_layout
from oracle import flex_ref as fr
from oracle import mtp_oracle as mo

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
def test_kv_append_identity_and_gather(mga, dev, dtype, D):
    torch.manual_seed(0)
    H, S, cap, off = 8, 777, 2048, 301
    src_k = torch.randn(1, S, H, D, device=dev).to(dtype).transpose(1, 2)   # strided projection view
    src_v = torch.randn(1, S, H, D, device=dev).to(dtype).transpose(1, 2)
    dk = torch.full((H, cap, D), 7.0, device=dev, dtype=dtype)
    dv = torch.full((H, cap, D), 7.0, device=dev, dtype=dtype)
    mga.ops.kv_append(src_k, src_v, dk, dv, dst_offset=off)
    torch.cuda.synchronize()
    assert torch.equal(dk[:, off:off + S], src_k[0]) and torch.equal(dv[:, off:off + S], src_v[0])
    assert (dk[:, :off] == 7).all() and (dk[:, off + S:] == 7).all()
    reg = (torch.rand(S, device=dev) > 0.3).long()
    idx, cnt = mga.ops.regular_index(reg[None])
    R = int(cnt.item())
    ref_idx = reg.nonzero(as_tuple=True)[0]
    assert R == ref_idx.numel() and torch.equal(idx[:R].long(), ref_idx)
    mga.ops.kv_append(src_k, src_v, dk, dv, dst_offset=5, idx=idx, n_rows=R)
    torch.cuda.synchronize()
    assert torch.equal(dk[:, 5:5 + R], src_k[0][:, ref_idx]) and torch.equal(dv[:, 5:5 + R], src_v[0][:, ref_idx])


def test_kv_append_capacity_error(mga, dev):
    k = torch.zeros(1, 2, 10, 64, device=dev, dtype=torch.bfloat16)
    buf = torch.zeros(2, 16, 64, device=dev, dtype=torch.bfloat16)
    with pytest.raises(mga._lib.CapacityError):
        mga.ops.kv_append(k, k, buf, buf, dst_offset=7)
    with pytest.raises(RuntimeError, match="capacity"):
        mga.StreamingKVCache(capacity=8, num_layers=1).update(k, k, 0)


@pytest.mark.parametrize("P,n_reg,n_anchor", [(8192, 4096, 256), (28672, 4096, 512)])
def test_append_at_config_sizes(mga, dev, P, n_reg, n_anchor):
    """Configs 2 and 3 (last chunk): regular-token carry-over bit-exact."""
    seq = chunk_layout(n_reg, n_anchor, 4, P, seed=1)
    S = len(seq.gate)
    H, D = 8, 128
    prefix_k = torch.randn(1, H, P, D, device=dev).bfloat16()
    prefix_v = torch.randn(1, H, P, D, device=dev).bfloat16()
    cur_k = torch.randn(1, S, H, D, device=dev).bfloat16().transpose(1, 2)
    cur_v = torch.randn(1, S, H, D, device=dev).bfloat16().transpose(1, 2)
    reg = torch.tensor(seq.regular, device=dev)[None]
    cache = mga.StreamingKVCache(capacity=P + S + 128, num_layers=1)
    cache.append_prefix([prefix_k], [prefix_v])
    kf, vf = cache.update(cur_k, cur_v, 0)
    full_k, want_k = fr.reference_cache_ops(prefix_k, cur_k, reg)
    full_v, want_v = fr.reference_cache_ops(prefix_v, cur_v, reg)
    assert torch.equal(kf, full_k) and torch.equal(vf, full_v)      # update == torch.cat
    idx, cnt = mga.ops.regular_index(reg)
    cache.commit_regular(idx, int(cnt.item()))
    k2, v2 = cache[0]
    assert cache.prefix_len == P + n_reg
    assert torch.equal(k2, want_k) and torch.equal(v2, want_v)


def test_stream_of_chunks_matches_reference(mga, dev):
    """Manager + cache over 5 chunks, 3 layers: after every extract the cache
    equals the reference's filtered DynamicCache tensors; the manager counts
    P = sum of regular tokens and the position check passes silently."""
    L, H, D = 3, 2, 64
    mgr = mga.StreamingKVCacheManager(capacity=4096)
    cache = mgr.new_cache(L)
    ref = [(torch.zeros(1, H, 0, D, device=dev, dtype=torch.bfloat16),) * 2 for _ in range(L)]
    P = 0
    for c in range(5):
        seq = chunk_layout(200 + 13 * c, 20, 4, P, seed=c, pad=(17 if c == 4 else 0))
        S = len(seq.gate)
        chunk = {"input_ids": torch.zeros(1, S, dtype=torch.long, device=dev),
                 "gate_mask": torch.tensor(seq.gate, device=dev)[None],
                 "regular_token_mask": torch.tensor(seq.regular, device=dev)[None],
                 "position_ids": torch.tensor(seq.position, device=dev)[None]}
        chunk = mgr.prepare_data_with_kv_cache(chunk)
        assert chunk["gate_mask"].shape == (1, S, 1) and int(chunk["gate_mask"].min()) >= 0
        new_ref = []
        for layer in range(L):
            k = torch.randn(1, S, H, D, device=dev).bfloat16().transpose(1, 2)
            v = torch.randn(1, S, H, D, device=dev).bfloat16().transpose(1, 2)
            kf, vf = cache.update(k, v, layer)
            fk, nk = fr.reference_cache_ops(ref[layer][0], k, chunk["regular_token_mask"])
            fv, nv = fr.reference_cache_ops(ref[layer][1], v, chunk["regular_token_mask"])
            assert torch.equal(kf, fk) and torch.equal(vf, fv)
            new_ref.append((nk, nv))
        assert cache.get_seq_length(0) == P + S
        cache = mgr.extract_regular_kv_cache_for_next_chunk(chunk, cache)
        P += int(seq.regular.sum())
        assert mgr.past_seen_tokens == P == cache.prefix_len
        for layer, (k, v) in enumerate(cache):
            assert torch.equal(k, new_ref[layer][0]) and torch.equal(v, new_ref[layer][1])
        ref = new_ref
    legacy = cache.to_legacy_cache()
    again = mga.StreamingKVCache.from_legacy_cache(legacy, capacity=4096)
    for (a, b), (c_, d) in zip(again, legacy):
        assert torch.equal(a, c_) and torch.equal(b, d)


def test_position_check_queued_with_the_index(mga, dev, capsys):
    """The position sanity check of collator.py:251-258 is formed on the device
    when the chunk is prepared and read with the regular-row count: correct
    positions print nothing, a wrong position prints the reference's message,
    and positions changed in place after prepare are compared again."""
    H, D = 2, 64
    seq = chunk_layout(180, 16, 4, 0, seed=9)
    S = len(seq.gate)
    first_regular = int(np.flatnonzero(seq.regular)[3])
    for case in ("right", "wrong", "changed"):
        mgr = mga.StreamingKVCacheManager(capacity=1024)
        cache = mgr.new_cache(1)
        pos = torch.tensor(seq.position, device=dev)[None]
        if case == "wrong":
            pos[0, first_regular] += 1
        chunk = {"input_ids": torch.zeros(1, S, dtype=torch.long, device=dev),
                 "gate_mask": torch.tensor(seq.gate, device=dev)[None],
                 "regular_token_mask": torch.tensor(seq.regular, device=dev)[None], "position_ids": pos}
        chunk = mgr.prepare_data_with_kv_cache(chunk)
        k = torch.randn(1, S, H, D, device=dev).bfloat16().transpose(1, 2)
        cache.update(k, k + 1, 0)
        if case == "changed":
            pos[0, first_regular] += 1
        capsys.readouterr()
        mgr.extract_regular_kv_cache_for_next_chunk(chunk, cache)
        out = capsys.readouterr().out
        if case == "right":
            assert out == "" and int(mgr._host[1]) == 0
        else:
            assert "Sanity check failed. Position IDs mismatch." in out, case
            assert int(mgr._host[1]) == (1 if case == "wrong" else 0)
        assert mgr.past_seen_tokens == int(seq.regular.sum())


def test_extract_after_mask_changed_in_place(mga, dev):
    """prepare builds the regular-token index early; a regular_token_mask
    changed in place between prepare and extract (or replaced by another
    tensor) must be read again, not served from the early index."""
    H, D = 2, 64
    seq = chunk_layout(180, 16, 4, 0, seed=9)
    S = len(seq.gate)
    for replace in (False, True):
        mgr = mga.StreamingKVCacheManager(capacity=1024)
        cache = mgr.new_cache(1)
        reg = torch.tensor(seq.regular, device=dev)[None]
        chunk = {"input_ids": torch.zeros(1, S, dtype=torch.long, device=dev),
                 "gate_mask": torch.tensor(seq.gate, device=dev)[None], "regular_token_mask": reg}
        chunk = mgr.prepare_data_with_kv_cache(chunk)
        k = torch.randn(1, S, H, D, device=dev).bfloat16().transpose(1, 2)
        cache.update(k, k + 1, 0)
        changed = reg.clone()
        changed[0, : S // 3] = 0
        if replace:
            chunk["regular_token_mask"] = changed
        else:
            reg.copy_(changed)
        cache = mgr.extract_regular_kv_cache_for_next_chunk(chunk, cache)
        keep = changed[0].nonzero().flatten()
        assert mgr.past_seen_tokens == len(keep) == cache.prefix_len
        kc, vc = cache[0]
        assert torch.equal(kc, k[:, :, keep]) and torch.equal(vc, (k + 1)[:, :, keep])


def test_take_over_dynamic_cache(mga, dev):
    """First chunk through the model's own DynamicCache (past_key_values=None in
    the trainer), then extract moves it into the streaming cache."""
    from transformers.cache_utils import DynamicCache
    seq = chunk_layout(150, 20, 4, 0, seed=3)
    S = len(seq.gate)
    dc = DynamicCache()
    ks = [torch.randn(1, 2, S, 64, device=dev).bfloat16() for _ in range(2)]
    for i, k in enumerate(ks):
        dc.update(k, k + 1, i)
    mgr = mga.StreamingKVCacheManager(capacity=1024)
    chunk = {"input_ids": torch.zeros(1, S, dtype=torch.long, device=dev),
             "regular_token_mask": torch.tensor(seq.regular, device=dev)[None],
             "position_ids": torch.tensor(seq.position, device=dev)[None]}
    out = mgr.extract_regular_kv_cache_for_next_chunk(chunk, dc)
    idx = torch.tensor(mo.regular_index(seq.regular), device=dev).long()
    assert isinstance(out, mga.StreamingKVCache) and out.prefix_len == len(idx)
    for i, (k, v) in enumerate(out):
        assert torch.equal(k, ks[i][:, :, idx]) and torch.equal(v, (ks[i] + 1)[:, :, idx])
