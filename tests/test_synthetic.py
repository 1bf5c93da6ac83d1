"""The package's synthetic chunk generator (used by bench.py and smoke()) lays
tokens out exactly as the oracle's restatement of dataset.py:25-56 for the
same anchors, and its anchor samplers follow their stated rules."""
import importlib

import numpy as np
import pytest
import torch

from oracle import mtp_oracle as mo

syn = importlib.import_module("mtp-glora_amd.synthetic")


@pytest.mark.parametrize("n_reg,anchors,draft,pos0,pad", [
    (50, [0, 7, 8, 49], 4, 0, 0),
    (300, list(range(0, 300, 4)), 8, 1234, 13),
    (10, [], 3, 5, 2),
    (64, list(range(64)), 1, 0, 0),
])
def test_layout_matches_oracle(n_reg, anchors, draft, pos0, pad):
    c = syn.mtp_chunk(n_reg, torch.tensor(anchors, dtype=torch.long), draft, pos0=pos0, pad=pad,
                      device="cpu")
    seq = mo.pad_to(mo.synth_sequence(n_reg, np.array(anchors, dtype=np.int64), draft, pos0=pos0),
                    n_reg + draft * len(anchors) + pad)
    assert np.array_equal(c["gate_mask"][0].numpy(), seq.gate)
    assert np.array_equal(c["regular_token_mask"][0].numpy(), seq.regular)
    assert np.array_equal(c["position_ids"][0].numpy(), seq.position)
    ids = c["input_ids"][0]
    is_mask = (seq.regular == 0) & (seq.gate != -1)
    assert bool((ids[torch.tensor(is_mask)] == syn.MASK_TOKEN_ID).all())
    assert bool((ids[torch.tensor(seq.regular == 1)] != syn.MASK_TOKEN_ID).all())


def test_anchor_samplers():
    a = syn.sample_anchors(4096, 256, 7)
    assert a.numel() == 256 and torch.equal(a, a.unique()) and int(a.max()) < 4096
    assert torch.equal(a, syn.sample_anchors(4096, 256, 7))
    assert not torch.equal(a, syn.sample_anchors(4096, 256, 8))
    e = syn.every_kth_anchor(2048, 4, 512)
    assert torch.equal(e, torch.arange(0, 2048, 4))
    with pytest.raises(ValueError):
        syn.sample_anchors(10, 11, 0)
