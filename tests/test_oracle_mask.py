"""Pins for the oracle's mask, BlockMask metadata, layout and credited work.

The predicate is checked against (a) the mask built from the plain-language
rule of the layout (a mask token sees the regular tokens up to its anchor and
the earlier mask tokens of its own block; a regular token sees the regular
tokens before it), computed from the generator's block ids, never from
num_prefix_x; (b) torch's own ``create_mask``/``create_block_mask`` on the
reference's mask_mod composition. The BlockMask tensors are checked against
``create_block_mask`` (exact int32 equality, index order included).
"""
import numpy as np
import pytest
import torch

from oracle import flex_ref as fr
from oracle import mtp_oracle as mo


def semantic_mask(full: mo.Sequence, start: int, end: int, P: int) -> np.ndarray:
    """Mask of chunk tokens [start, end) over [cached regular prefix ++ chunk],
    from block membership. ``full`` is the unpadded sequence; the chunk may be
    padded beyond ``end`` (pad rows/cols see nothing)."""
    g = full.gate
    T = len(g)
    tok = np.arange(T)
    # global causal rule over the whole sequence
    allowed_full = np.zeros((T, T), bool)
    for i in range(T):
        for j in range(i + 1):
            if g[i] == -1 or g[j] == -1:
                continue
            if g[j] == 0:                       # regular key (or gate-0 tail mask): visible
                allowed_full[i, j] = True
            elif g[i] == 1 and full.block[i] == full.block[j] and not full.is_anchor[j]:
                allowed_full[i, j] = True       # earlier mask token of the same block
    # streaming view: keys = regular tokens before the chunk, then the chunk
    prefix_keys = tok[:start][full.regular[:start] == 1]
    assert len(prefix_keys) == P
    keys = np.concatenate([prefix_keys, tok[start:end]])
    return allowed_full[start:end][:, keys]


def random_seq(rng, n_reg, n_anchor, D, tail=False):
    anchors = rng.choice(n_reg, size=n_anchor, replace=False)
    return mo.synth_sequence(n_reg, anchors, D, tail_unlabelled=tail)


@pytest.mark.parametrize("seed", range(6))
def test_predicate_matches_layout_meaning(seed):
    rng = np.random.default_rng(seed)
    D = int(rng.integers(1, 6))
    seq = random_seq(rng, 120, 25, D, tail=bool(seed % 2))
    # anchor of the last regular token so the gate-0 tail case occurs
    pts = mo.split_points(seq.gate, 96, D)
    for c in range(len(pts) - 1):
        s, e = pts[c], pts[c + 1]
        P = int(seq.regular[:s].sum())
        want = semantic_mask(seq, s, e, P)
        got = mo.mtp_mask_dense(seq.gate[s:e], P)
        assert np.array_equal(got, want), (seed, c)
        # the code form used by the kernels is the same predicate
        assert np.array_equal(mo.mask_from_codes(mo.mtp_codes(seq.gate[s:e], P), P), want)


def test_padding_rows_and_cols_are_empty():
    seq = mo.pad_to(mo.synth_sequence(40, [3, 10, 20], 4), 80)
    m = mo.mtp_mask_dense(seq.gate, 16)
    pad = seq.gate == -1
    assert not m[pad].any()
    assert not m[:, 16:][:, pad].any()
    assert m[~pad][:, :16].all()          # every real query sees the whole regular prefix


def _cmp_block_mask(gate, P, device="cpu"):
    bm = fr.reference_block_mask(torch.tensor(gate)[None], P, device=device)
    ref = fr.block_mask_tensors(bm)
    dense = mo.block_mask_from_dense(mo.mtp_mask_dense(gate, P))
    tiles = mo.block_mask_mtp(gate, P)
    for k, v in ref.items():
        assert v.dtype == np.int32
        assert dense[k].shape == v.shape and np.array_equal(dense[k], v), k
        assert tiles[k].shape == v.shape and np.array_equal(tiles[k], v), k
    # the dense mask itself equals torch's create_mask of the reference mask_mod
    from torch.nn.attention.flex_attention import create_mask
    S = len(gate)
    tm = create_mask(fr.mtp_mask_mod(torch.tensor(gate)[None], P), None, None, S, P + S, device="cpu")
    assert np.array_equal(tm[0, 0].numpy(), mo.mtp_mask_dense(gate, P))


@pytest.mark.parametrize("case", [
    dict(n_reg=300, n_anchor=20, D=4, P=0, pad=0),
    dict(n_reg=300, n_anchor=20, D=4, P=128, pad=0),
    dict(n_reg=250, n_anchor=40, D=3, P=200, pad=70),      # ragged S, P not a tile multiple
    dict(n_reg=100, n_anchor=60, D=8, P=384, pad=0),       # mask-token heavy
    dict(n_reg=60, n_anchor=5, D=2, P=0, pad=3),           # S < 128
    dict(n_reg=512, n_anchor=128, D=4, P=1024, pad=0),     # tile-aligned S
])
def test_block_mask_matches_create_block_mask(case):
    rng = np.random.default_rng(case["n_reg"] + case["P"])
    seq = random_seq(rng, case["n_reg"], case["n_anchor"], case["D"])
    seq = mo.pad_to(seq, len(seq.gate) + case["pad"])
    _cmp_block_mask(seq.gate, case["P"])


def test_block_mask_all_pad_and_tail_unlabelled():
    _cmp_block_mask(np.full(200, -1, np.int64), 64)
    seq = mo.synth_sequence(90, [10, 50, 89], 4, tail_unlabelled=True)
    _cmp_block_mask(mo.pad_to(seq, 130).gate, 256)


def test_full_tile_requires_complete_tile():
    # a 128-row chunk of regular tokens against a 128-token prefix: the prefix
    # tile is full, the diagonal tile is partial (causal)
    bm = mo.block_mask_mtp(np.zeros(128, np.int64), 128)
    assert bm["full_kv_num_blocks"][0, 0].tolist() == [1]
    assert bm["kv_num_blocks"][0, 0].tolist() == [1]
    assert bm["full_kv_indices"][0, 0, 0, 0] == 0 and bm["kv_indices"][0, 0, 0, 0] == 1


def test_chunked_masks_equal_single_pass():
    """Streaming invariant: each chunk's mask is the single-pass mask of the
    whole sequence restricted to [earlier regular tokens ++ chunk]."""
    rng = np.random.default_rng(7)
    seq = random_seq(rng, 400, 60, 4)
    full = mo.mtp_mask_dense(seq.gate, 0)
    pts = mo.split_points(seq.gate, 160, 4)
    tok = np.arange(len(seq.gate))
    for c in range(len(pts) - 1):
        s, e = pts[c], pts[c + 1]
        keys = np.concatenate([tok[:s][seq.regular[:s] == 1], tok[s:e]])
        P = int(seq.regular[:s].sum())
        assert np.array_equal(mo.mtp_mask_dense(seq.gate[s:e], P), full[s:e][:, keys])


def test_split_points_keep_blocks_whole():
    rng = np.random.default_rng(3)
    for D in (1, 4, 8):
        n = 500
        seq = mo.synth_sequence(n, np.arange(n), D)      # every token is an anchor (dataset.py layout)
        # prompt of 37 regular tokens: first mask token at index 38
        prompt = mo.synth_sequence(37, [], D)
        gate = np.concatenate([prompt.gate, seq.gate])
        pts = mo.split_points(gate, 256, D)
        assert pts[0] == 0 and pts[-1] == len(gate)
        for p in pts[1:-1]:
            # a split never separates a mask token from its block
            assert gate[p] == 0, (D, p)
            assert (p - 37) % (1 + D) == 0


def test_last_bucket():
    assert mo.pick_last_bucket(100, 5120, 1024) == 1024
    assert mo.pick_last_bucket(1025, 5120, 1024) == 2048
    assert mo.pick_last_bucket(5120, 5120, 1024) == 5120
    assert mo.pick_last_bucket(4100, 4500, 1024) == 4500


def test_credited_flops_match_published_figures():
    """Config 2 (S=5120, P=8192) and config 5 (S=6144, P=16384) credited work:
    907.3 / 1581.1 GFLOP and 1964.9 / 3263.1 GFLOP (fwd / bwd) per layer."""
    seq = mo.synth_sequence(4096, mo.sample_anchors(4096, 256, 0), 4, pos0=8192)
    S = len(seq.gate)
    f, b = mo.credited_flops(mo.block_mask_mtp(seq.gate, 8192), S, 8192 + S, 8192, 32, 128)
    assert round(f / 1e9, 1) == 907.3 and round(b / 1e9, 1) == 1581.1
    seq = mo.synth_sequence(2048, np.arange(0, 2048, 4), 8, pos0=16384)
    S = len(seq.gate)
    f, b = mo.credited_flops(mo.block_mask_mtp(seq.gate, 16384), S, 16384 + S, 16384, 32, 128)
    assert round(f / 1e9, 1) == 1964.9 and round(b / 1e9, 1) == 3263.1


def test_layout_positions():
    seq = mo.synth_sequence(10, [2, 5], 3, pos0=100)
    # regular tokens have consecutive positions; mask k of anchor p has p + k
    reg = seq.position[seq.regular == 1]
    assert reg.tolist() == list(range(100, 110))
    i = int(np.nonzero(seq.is_anchor)[0][0])
    assert seq.position[i + 1:i + 4].tolist() == [seq.position[i] + 1, seq.position[i] + 2, seq.position[i] + 3]
    assert (seq.gate[seq.regular == 0] == 1).all()


def test_cache_append_equals_reference_cat():
    rng = np.random.default_rng(0)
    prefix = rng.standard_normal((2, 7, 4)).astype(np.float32)
    cur = rng.standard_normal((2, 9, 4)).astype(np.float32)
    reg = (rng.random(9) > 0.4).astype(np.int64)
    full, out = fr.reference_cache_ops(torch.tensor(prefix)[None], torch.tensor(cur)[None],
                                       torch.tensor(reg)[None])
    assert np.array_equal(mo.cache_append(prefix, cur, reg), out[0].numpy())
    assert full.shape[2] == 16


@pytest.mark.parametrize("seed", range(4))
def test_ordered_compare_form_equals_predicate(seed):
    """The single ordered compare the GPU kernels evaluate equals the
    reference predicate, on real layouts and on arbitrary gate vectors (pads
    and gate-0 tokens anywhere, which the predicate still defines)."""
    rng = np.random.default_rng(100 + seed)
    for _ in range(400):
        n_reg = int(rng.integers(1, 50))
        D = int(rng.integers(1, 9))
        seq = random_seq(rng, n_reg, int(rng.integers(0, n_reg + 1)), D, tail=bool(rng.integers(0, 2)))
        g = seq.gate if rng.integers(0, 2) else rng.choice([-1, 0, 1], size=len(seq.gate))
        P = int(rng.integers(0, 40))
        want = mo.mtp_mask_dense(g, P)
        assert np.array_equal(mo.mask_from_order(mo.mtp_codes(g, P), P), want)
