"""Host-side behaviour that needs no GPU: the product refuses CPU tensors
(there is no CPU path), the MTP BlockMask is a torch BlockMask that the
transformers mask plumbing passes through, its mask_mod equals the reference
predicate, and the attention function is registered with transformers."""
import numpy as np
import pytest
import torch

from oracle import flex_ref as fr
from oracle import mtp_oracle as mo


def test_ops_refuse_cpu_tensors(mga):
    with pytest.raises(RuntimeError, match="no CPU path"):
        mga.ops.regular_index(torch.ones(1, 8, dtype=torch.long))
    with pytest.raises(RuntimeError, match="no CPU path"):
        mga.ops.mtp_block_mask_tensors(torch.zeros(1, 8, dtype=torch.long), 0)
    with pytest.raises(RuntimeError, match="no CPU path"):
        mga.build_mtp_block_mask(torch.zeros(1, 8, dtype=torch.long), 0)
    k = torch.zeros(1, 2, 4, 64)
    with pytest.raises(RuntimeError):
        mga.StreamingKVCache(capacity=16, num_layers=1).update(k, k, 0)


def test_cache_refuses_cpu_device(mga):
    with pytest.raises(RuntimeError, match="GPU memory"):
        mga.StreamingKVCache(capacity=16, num_layers=1, num_kv_heads=2, head_dim=64,
                             dtype=torch.bfloat16, device="cpu")
    with pytest.raises(ValueError):
        mga.StreamingKVCache(capacity=0)


def _cpu_mtp_mask(mga, gate, P):
    """An MTPBlockMask assembled on the CPU from the oracle's tensors (the GPU
    builds the same tensors; see the GPU tests)."""
    t = {k: torch.tensor(v) for k, v in mo.block_mask_mtp(gate, P).items()}
    t["code"] = torch.tensor(mo.mtp_codes(gate, P))
    return mga.MTPBlockMask.from_tensors(t, len(gate), P)


def test_mask_mod_equals_reference_predicate(mga):
    from torch.nn.attention.flex_attention import create_mask
    seq = mo.pad_to(mo.synth_sequence(150, [3, 40, 41, 99, 149], 4, tail_unlabelled=True), 200)
    P = 77
    bm = _cpu_mtp_mask(mga, seq.gate, P)
    S = len(seq.gate)
    mine = create_mask(bm.mask_mod, None, None, S, P + S, device="cpu")[0, 0].numpy()
    ref = create_mask(fr.mtp_mask_mod(torch.tensor(seq.gate)[None], P), None, None, S, P + S,
                      device="cpu")[0, 0].numpy()
    assert np.array_equal(mine, ref)
    # to_dense() of the product mask equals the reference block structure
    assert np.array_equal(bm.to_dense()[0, 0].numpy(),
                          fr.reference_block_mask(torch.tensor(seq.gate)[None], P).to_dense()[0, 0].numpy())


def test_mtp_block_mask_passes_transformers_plumbing(mga):
    from torch.nn.attention.flex_attention import BlockMask
    from transformers.masking_utils import _preprocess_mask_arguments
    seq = mo.synth_sequence(100, [5, 50], 4)
    bm = _cpu_mtp_mask(mga, seq.gate, 64)
    assert isinstance(bm, BlockMask) and len(bm.shape) == 4
    early, mask, *_ = _preprocess_mask_arguments(None, None, bm, None, None, 0)
    assert early and mask is bm
    moved = bm.to("cpu")
    assert isinstance(moved, mga.MTPBlockMask) and moved.prefix_len == 64
    assert torch.equal(moved.mtp_code, bm.mtp_code)


def test_attention_rejects_foreign_masks_and_options(mga):
    q = torch.zeros(1, 4, 8, 64)
    k = torch.zeros(1, 2, 8, 64)
    with pytest.raises(TypeError, match="MTPBlockMask"):
        mga.mtp_attention_forward(torch.nn.Module(), q, k, k, None, scaling=0.1)
    with pytest.raises(ValueError, match="dropout"):
        mga.mtp_attention_forward(torch.nn.Module(), q, k, k, None, dropout=0.1)
    with pytest.raises(NotImplementedError):
        mga.mtp_attention_forward(torch.nn.Module(), q, k, k, None, softcap=30.0)
    bm = _cpu_mtp_mask(mga, np.zeros(8, np.int64), 0)
    with pytest.raises(ValueError, match="prefix"):
        mga.mtp_attention(q, torch.zeros(1, 2, 9, 64), torch.zeros(1, 2, 9, 64), bm)


def test_register_with_transformers(mga):
    from transformers import AttentionInterface
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    mga.register("mtp_hip")
    assert ALL_ATTENTION_FUNCTIONS["mtp_hip"] is mga.mtp_attention_forward
    assert AttentionInterface()["mtp_hip"] is mga.mtp_attention_forward


def test_manager_api_surface(mga):
    m = mga.StreamingKVCacheManager(capacity=64)
    assert m.past_seen_tokens == 0
    m.past_seen_tokens = 5
    m.reset_cache()
    assert m.past_seen_tokens == 0
    assert m.extract_regular_kv_cache_for_next_chunk({"input_ids": torch.zeros(1, 4)}, None) is None


def test_cache_raise_paths_before_allocation(mga):
    """Raise paths that need no device memory: a carry-over before any update,
    an update of a cache that does not know its layer count, a crop below an
    empty prefix."""
    c = mga.StreamingKVCache(capacity=16, num_layers=2)
    with pytest.raises(RuntimeError, match="commit_regular before any update"):
        c.commit_regular(torch.zeros(4, dtype=torch.int32), 0)
    k = torch.zeros(1, 2, 4, 64)
    with pytest.raises(RuntimeError, match="needs num_layers"):
        mga.StreamingKVCache(capacity=16).update(k, k, 0)
    with pytest.raises(ValueError, match="negative"):
        c.crop(-1)
