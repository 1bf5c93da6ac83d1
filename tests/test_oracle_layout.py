"""Pins for the oracle's token layout (``insert_mask_tokens``, dataset.py:25-56)
and chunking (``split_points`` / ``pick_last_bucket`` / ``chunk_sequence``,
collator.py:47-175).

The layout is checked against what it means rather than against its formula:
the prompt is regular and unlabelled, regular tokens carry consecutive
positions, each response token is followed by its D mask tokens at the next D
positions, and a mask token is labelled (gate 1) exactly when the token it
predicts -- the regular token one position later -- exists. The chunker is
checked against split points and bucket sizes worked out by hand, and against
invariants a slip in the cursor arithmetic breaks (blocks never straddle a
chunk, unpadded chunks concatenate to the sequence, pad values).
"""
import numpy as np
import pytest

from oracle import mtp_oracle as mo


@pytest.mark.parametrize("n_in,n_out,D", [(0, 9, 4), (5, 12, 4), (37, 40, 1), (3, 20, 8), (11, 2, 3)])
def test_insert_mask_tokens_meaning(n_in, n_out, D):
    s = mo.insert_mask_tokens(n_in, n_out, D)
    T = n_in + n_out * (1 + D)
    assert len(s.gate) == T
    # the prompt: regular, unlabelled, positions 0..n_in-1
    assert (s.regular[:n_in] == 1).all() and (s.gate[:n_in] == 0).all()
    assert s.position[:n_in].tolist() == list(range(n_in))
    # regular tokens in order carry consecutive positions
    reg_pos = s.position[s.regular == 1]
    assert reg_pos.tolist() == list(range(n_in + n_out))
    last_regular_pos = n_in + n_out - 1
    for j in range(n_out):
        a = n_in + j * (1 + D)               # response token j
        assert s.regular[a] == 1 and s.gate[a] == 0 and s.is_anchor[a]
        p = s.position[a]
        for k in range(1, D + 1):
            t = a + k
            assert s.regular[t] == 0 and s.position[t] == p + k and s.block[t] == s.block[a]
            # the label of a mask token is the token at its position + 1
            want = 1 if s.position[t] + 1 <= last_regular_pos else 0
            assert s.gate[t] == want, (j, k)


def test_insert_mask_tokens_tail_pattern():
    """D = 4: the last six response blocks are labelled [1,1,1,1], [1,1,1,0],
    [1,1,0,0], [1,0,0,0], [0,0,0,0], [0,0,0,0]: a mask token k of response
    token j predicts response token j + k + 1."""
    D, n_out = 4, 10
    s = mo.insert_mask_tokens(7, n_out, D)
    blocks = s.gate[7:].reshape(n_out, 1 + D)[:, 1:]
    assert blocks[-6:].tolist() == [[1, 1, 1, 1], [1, 1, 1, 0], [1, 1, 0, 0], [1, 0, 0, 0],
                                    [0, 0, 0, 0], [0, 0, 0, 0]]
    assert (blocks[:-5] == 1).all()
    # count of labelled mask tokens: sum over j of #{k in 1..D : j + k + 1 <= n_out - 1}
    assert int(s.gate.sum()) == sum(max(0, min(D, n_out - 2 - j)) for j in range(n_out))


def test_insert_mask_tokens_gate_zero_masks_are_x_keys():
    """A tail mask token with gate 0 is an x key in the MTP predicate (it is
    seen by every later query, including the next block's anchor) but not a
    regular token (never cached)."""
    s = mo.insert_mask_tokens(3, 8, 4)
    allowed = mo.mtp_mask_dense(s.gate, 0)
    g0 = np.nonzero((s.gate == 0) & (s.regular == 0))[0]
    assert len(g0) > 0
    t = g0[0]
    later = np.arange(t + 1, len(s.gate))
    assert allowed[later, t].all()


@pytest.mark.parametrize("n_in,n_out,D,C,mn,points,targets", [
    # first chunk: prompt + floor((C - prompt) / (1 + D)) blocks; later: floor(C / (1 + D)) blocks
    (100, 1000, 4, 1024, 512, [0, 1020, 2040, 3060, 4080, 5100], [1024] * 5),
    # last chunk of 5 tokens: bucket list [512] (range(1024, 513, 1024) is empty), need 256
    (37, 300, 4, 512, 256, [0, 512, 1022, 1532, 1537], [512] * 4),
    # no prompt; default buckets 1024..5120: the 4880-token tail goes to 5120
    (0, 2000, 4, 5120, 1024, [0, 5120, 10000], [5120, 5120]),
    # a 380-token tail is padded to max(380, min_chunk_size) -> 1024
    (0, 1100, 4, 5120, 1024, [0, 5120, 5500], [5120, 1024]),
    # a 985-token tail with min_chunk_size 1024 is padded to 1024 (a remainder chunk)
    (60, 1004, 4, 4096, 1024, [0, 4095, 5080], [4096, 1024]),
])
def test_chunking_by_hand(n_in, n_out, D, C, mn, points, targets):
    s = mo.insert_mask_tokens(n_in, n_out, D)
    assert mo.split_points(s.gate, C, D) == points
    chunks = mo.chunk_sequence(s, C, D, mn)
    assert [len(c.gate) for c in chunks] == targets
    for i, c in enumerate(chunks):
        a, b = points[i], points[i + 1]
        n = b - a
        assert np.array_equal(c.gate[:n], s.gate[a:b])
        assert np.array_equal(c.regular[:n], s.regular[a:b])
        assert np.array_equal(c.position[:n], s.position[a:b])
        # pad values of collator.py:150-156
        assert (c.gate[n:] == -1).all() and (c.regular[n:] == 0).all() and (c.position[n:] == 0).all()


@pytest.mark.parametrize("D", [1, 3, 4, 8])
def test_chunks_keep_blocks_whole(D):
    s = mo.insert_mask_tokens(29, 700, D)
    chunks = mo.chunk_sequence(s, 1024, D, 256)
    pts = mo.split_points(s.gate, 1024, D)
    # unpadded chunks concatenate back to the sequence
    parts = [c.gate[:pts[i + 1] - pts[i]] for i, c in enumerate(chunks)]
    assert np.array_equal(np.concatenate(parts), s.gate)
    for p in pts[1:-1]:
        assert s.regular[p] == 1 and s.is_anchor[p]          # every later chunk opens with an anchor
        assert (s.regular[p + 1:p + 1 + D] == 0).all()
    # every non-last chunk is padded to chunk_size and holds at most chunk_size tokens
    for c in chunks[:-1]:
        assert len(c.gate) == 1024


def test_bucket_rule_by_hand():
    assert mo.pick_last_bucket(1, 4096, 1024) == 1024
    assert mo.pick_last_bucket(1024, 4096, 1024) == 1024
    assert mo.pick_last_bucket(3073, 4096, 1024) == 4096
    assert mo.pick_last_bucket(700, 4096, 512) == 1024
    assert mo.pick_last_bucket(700, 4096, 512, buckets=[512, 768, 4096]) == 768
    assert mo.pick_last_bucket(5000, 4096, 1024) == 5000          # past every bucket: falls back to need
