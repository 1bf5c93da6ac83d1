"""CPU oracle for MTP-GLoRA's chunked-training hot path (numpy).

TEST INFRASTRUCTURE. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` import this module, and only as the
checker. The product package never imports it and has no CPU fallback.

What it restates (each function cites the reference lines it follows; paths
are relative to the reference checkout, ``[torch]`` / ``[tf]`` are the
installed torch / transformers trees):

* ``synth_sequence`` / ``synth_chunk``   - token layout of
  ``mtp_glora/data_utils/dataset.py:25-56`` (anchor followed by its D mask
  tokens; positions; gate / regular masks) for seeded synthetic inputs.
* ``insert_mask_tokens``                 - the dataset's own layout of one
  example (dataset.py:25-56): every response token an anchor, labels by the
  position + 1 gather, so the last blocks are partly labelled.
* ``split_points`` / ``pick_last_bucket`` / ``chunk_sequence`` - chunking and
  padding of ``mtp_glora/data_utils/collator.py:73-175``.
* ``mtp_mask_dense``                     - the MTP ``mask_mod`` predicate of
  ``collator.py:311-355`` over ``[S, P+S]``.
* ``mtp_codes``                          - one int32 code per chunk token
  (pad -1, x -2, m -> num_prefix_x) that encodes the same predicate;
  ``mask_from_codes`` / ``mask_from_order`` rebuild it in the two forms the
  GPU kernels evaluate.
* ``block_mask_from_dense``              - ``create_block_mask``'s tile
  classification and ordering, ``[torch]nn/attention/flex_attention.py``
  ``:399-442`` (``_ordered_to_dense``/``_dense_to_ordered``/
  ``_transpose_ordered``) and ``:979-1022`` (``_convert_mask_to_block_mask``).
* ``block_mask_mtp``                     - the same eight tensors computed tile
  by tile from the codes (no dense ``S x (P+S)`` mask), for large shapes.
* ``cache_append``                       - ``collator.py:249, 270-285``
  (regular-token gather + cat with the detached prefix).
* ``attention_fwd`` / ``attention_bwd``  - dense masked GQA attention with the
  fully-masked-row rules of ``[torch]_higher_order_ops/flex_attention.py``
  ``:202-267`` (fwd) and ``:826-990`` (bwd).
* ``credited_flops``                     - the credited-work count used for the
  roofline numerator (only non-empty 128x128 tiles; no prefix dK/dV).

Parity pins for every function live in ``tests/test_oracle_*.py``.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

BLOCK = 128  # [torch]nn/attention/flex_attention.py:395 _DEFAULT_SPARSE_BLOCK_SIZE

CODE_PAD = -1
CODE_X = -2


# ----------------------------------------------------------------------------
# Token layout and chunking
# ----------------------------------------------------------------------------

@dataclass
class Sequence:
    """One MTP training sequence in the layout of dataset.py:25-56.

    ``gate``: 0 regular (x), 1 mask token with a label (m), -1 pad.
    ``regular``: 1 for non-mask tokens (dataset.py:54).
    ``position``: regular tokens consecutive; mask k of an anchor at
    position p has position p + k (dataset.py:30-36).
    ``block``: anchor ordinal for mask tokens and their anchor, -1 otherwise
    (used only by tests to build the mask from its plain-language meaning).
    """
    gate: np.ndarray
    regular: np.ndarray
    position: np.ndarray
    block: np.ndarray
    is_anchor: np.ndarray


def synth_sequence(n_regular: int, anchors: np.ndarray, draft_length: int,
                   pos0: int = 0, tail_unlabelled: bool = False) -> Sequence:
    """Lay out ``n_regular`` regular tokens with ``draft_length`` mask tokens
    inserted after every regular token whose index is in ``anchors``.

    Follows dataset.py:30-54: the D masks follow their anchor immediately,
    mask k of an anchor at position p gets position p + k, ``gate`` is 1 on a
    mask token whose label is valid and ``regular`` is 1 on non-mask tokens.
    With ``tail_unlabelled`` the masks of the last regular token get gate 0
    (their labels run past the sequence end, dataset.py:39-41, 53).
    """
    anchors = np.unique(np.asarray(anchors, dtype=np.int64))
    is_anchor_reg = np.zeros(n_regular, dtype=bool)
    is_anchor_reg[anchors] = True
    total = n_regular + draft_length * int(is_anchor_reg.sum())
    gate = np.zeros(total, dtype=np.int64)
    regular = np.zeros(total, dtype=np.int64)
    position = np.zeros(total, dtype=np.int64)
    block = np.full(total, -1, dtype=np.int64)
    is_anchor = np.zeros(total, dtype=bool)
    t = 0
    b = 0
    for r in range(n_regular):
        gate[t] = 0
        regular[t] = 1
        position[t] = pos0 + r
        if is_anchor_reg[r]:
            is_anchor[t] = True
            block[t] = b
        t += 1
        if is_anchor_reg[r]:
            lab_ok = not (tail_unlabelled and r == n_regular - 1)
            for k in range(1, draft_length + 1):
                gate[t] = 1 if lab_ok else 0
                regular[t] = 0
                position[t] = pos0 + r + k
                block[t] = b
                t += 1
            b += 1
    return Sequence(gate, regular, position, block, is_anchor)


def insert_mask_tokens(input_len: int, output_len: int, draft_length: int) -> Sequence:
    """The token layout the reference's dataset builds for one example
    (``insert_mask_tokens``, dataset.py:25-56): ``input_len`` prompt tokens,
    then every one of the ``output_len`` response tokens followed by its
    ``draft_length`` mask tokens (every response token is an anchor).

    Positions (dataset.py:30-36): the prompt gets 0 .. input_len - 1; response
    token j and its masks get input_len + j + (0 .. D). Labels (dataset.py:38-41)
    are the label row ``[-100] * input_len ++ response ++ [-100] * (D + 1)``
    gathered at position + 1. gate = 1 on a mask token whose label is not
    -100, else 0 (dataset.py:53); regular = 1 on non-mask tokens (:54).
    """
    D = int(draft_length)
    n_in, n_out = int(input_len), int(output_len)
    blk = (np.arange(n_out)[:, None] + np.arange(D + 1)[None, :]).reshape(-1)
    position = np.concatenate([np.arange(n_in), blk + n_in]).astype(np.int64)
    response = np.arange(1, n_out + 1, dtype=np.int64)          # any ids other than -100
    label_row = np.concatenate([np.full(n_in, -100, np.int64), response,
                                np.full(D + 1, -100, np.int64)])
    labels = label_row[position + 1]
    is_mask = np.concatenate([np.zeros(n_in, bool),
                              np.tile(np.arange(D + 1) > 0, n_out)])
    gate = np.where(is_mask & (labels != -100), 1, 0).astype(np.int64)
    regular = (~is_mask).astype(np.int64)
    block = np.concatenate([np.full(n_in, -1, np.int64),
                            np.repeat(np.arange(n_out, dtype=np.int64), D + 1)])
    is_anchor = np.concatenate([np.zeros(n_in, bool), np.tile(np.arange(D + 1) == 0, n_out)])
    return Sequence(gate, regular, position, block, is_anchor)


def sample_anchors(n_regular: int, n_anchors: int, seed: int) -> np.ndarray:
    """``n_anchors`` distinct regular-token indices drawn uniformly from a seed."""
    rng = np.random.default_rng(seed)
    return np.sort(rng.choice(n_regular, size=n_anchors, replace=False))


def pad_to(seq: Sequence, length: int) -> Sequence:
    """Pad per collator.py:150-156 (gate -1, regular 0, position 0)."""
    n = len(seq.gate)
    if length <= n:
        return seq
    extra = length - n
    return Sequence(
        np.concatenate([seq.gate, np.full(extra, -1, np.int64)]),
        np.concatenate([seq.regular, np.zeros(extra, np.int64)]),
        np.concatenate([seq.position, np.zeros(extra, np.int64)]),
        np.concatenate([seq.block, np.full(extra, -1, np.int64)]),
        np.concatenate([seq.is_anchor, np.zeros(extra, bool)]),
    )


def pick_last_bucket(content_len: int, chunk_size: int, min_chunk_size: int,
                     buckets=None) -> int:
    """collator.py:47-53 (default buckets) and :73-84 (smallest bucket >= need)."""
    if buckets is None:
        buckets = list(range(1024, chunk_size + 1, 1024))
        if chunk_size not in buckets:
            buckets.append(chunk_size)
    buckets = sorted(set(buckets))
    need = max(content_len, min_chunk_size)
    for b in buckets:
        if b >= need:
            return b
    return need


def split_points(gate: np.ndarray, chunk_size: int, draft_length: int) -> list:
    """collator.py:131-148: chunk boundaries on whole (1 + D)-token blocks
    after the prompt."""
    total_len = len(gate)
    block_len = 1 + draft_length
    ones = np.nonzero(gate == 1)[0]
    prompt_len = int(ones[0]) - 1 if len(ones) > 0 else total_len
    pts = [0]
    cursor = 0
    while cursor < total_len:
        first = cursor == 0
        base = chunk_size - prompt_len if first else chunk_size
        nblk = max(0, base // block_len)
        content = (prompt_len if first else 0) + nblk * block_len
        cursor += content
        pts.append(min(cursor, total_len))
    if len(pts) > 1 and pts[-1] == pts[-2]:
        pts.pop()
    return pts


def chunk_sequence(seq: Sequence, chunk_size: int, draft_length: int,
                   min_chunk_size: int) -> list:
    """collator.py:158-175: slice at ``split_points`` and pad non-last chunks
    to ``chunk_size``, the last to its bucket."""
    pts = split_points(seq.gate, chunk_size, draft_length)
    out = []
    for i in range(len(pts) - 1):
        s, e = pts[i], pts[i + 1]
        last = i == len(pts) - 2
        tgt = pick_last_bucket(e - s, chunk_size, min_chunk_size) if last else chunk_size
        part = Sequence(seq.gate[s:e], seq.regular[s:e], seq.position[s:e],
                        seq.block[s:e], seq.is_anchor[s:e])
        out.append(pad_to(part, tgt))
    return out


# ----------------------------------------------------------------------------
# The MTP predicate
# ----------------------------------------------------------------------------

def _gate_with_past(gate: np.ndarray, P: int) -> np.ndarray:
    """collator.py:311-318: P zeros (the cached prefix is all regular) then the chunk gate."""
    gate = np.asarray(gate, dtype=np.int64)
    return np.concatenate([np.zeros(P, np.int64), gate]) if P > 0 else gate


def mtp_mask_dense(gate: np.ndarray, P: int) -> np.ndarray:
    """Boolean ``[S, P+S]`` mask of collator.py:320-355.

    allowed(i, j) = causal(i+P >= j) & q not pad & k not pad &
                    ((q x & k x) | (q m & (k x | (k m & npx[i+P] == npx[j]))))
    with npx = inclusive cumsum of (g == 0) over [0]*P ++ gate (collator.py:320).
    """
    g = _gate_with_past(gate, P)
    S = len(gate)
    L = P + S
    npx = np.cumsum(g == 0)
    qi = np.arange(S)[:, None] + P
    kj = np.arange(L)[None, :]
    gq = g[P:][:, None]
    gk = g[None, :]
    causal = qi >= kj
    q_np = gq != -1
    k_np = gk != -1
    x_rule = (gq == 0) & (gk == 0)
    same_blk = npx[P:][:, None] == npx[None, :]
    m_rule = (gq == 1) & ((gk == 0) | ((gk == 1) & same_blk))
    return causal & q_np & k_np & (x_rule | m_rule)


def mtp_codes(gate: np.ndarray, P: int) -> np.ndarray:
    """int32 code per chunk token: -1 pad, -2 regular (x), npx for m.

    With these codes (and code -2 for every prefix key j < P)
    allowed(i, j) == (i+P >= j) & code[i] != -1 & (kcode[j] == -2 | kcode[j] == code[i]),
    which is the predicate of ``mtp_mask_dense`` (pinned in the tests).
    """
    g = np.asarray(gate, dtype=np.int64)
    npx = P + np.cumsum(g == 0)
    code = np.where(g == -1, CODE_PAD, np.where(g == 0, CODE_X, npx))
    return code.astype(np.int32)


def mask_from_codes(code: np.ndarray, P: int) -> np.ndarray:
    """Dense mask rebuilt from the codes (the form the GPU kernels evaluate)."""
    S = len(code)
    kcode = np.concatenate([np.full(P, CODE_X, np.int32), code])
    qi = np.arange(S)[:, None] + P
    kj = np.arange(P + S)[None, :]
    qc = code[:, None]
    kc = kcode[None, :]
    return (qi >= kj) & (qc != CODE_PAD) & ((kc == CODE_X) | (kc == qc))


def mask_from_order(code: np.ndarray, P: int) -> np.ndarray:
    """The predicate as one causal bound and one ordered compare, the form the
    GPU kernels evaluate: with w(key) = +inf for a regular key, -inf for a
    pad key, else its num_prefix_x code, and v(query) = +inf for a regular
    query, else its code,

        allowed(i, j) = (j <= qlim(i)) & (w(j) >= v(i)),  qlim = -1 for a pad query.

    Equal to ``mask_from_codes`` because num_prefix_x never decreases along the
    sequence, so a mask key at or before the query carries a code <= the
    query's, with equality exactly for keys of the query's own block."""
    big = np.int64(2 ** 31 - 1)
    S = len(code)
    c = code.astype(np.int64)
    kcode = np.concatenate([np.full(P, CODE_X, np.int64), c])
    w = np.where(kcode == CODE_X, big, np.where(kcode == CODE_PAD, -big, kcode))
    v = np.where(c == CODE_X, big, c)
    qlim = np.where(c == CODE_PAD, -1, np.arange(S) + P)
    return (np.arange(P + S)[None, :] <= qlim[:, None]) & (w[None, :] >= v[:, None])


# ----------------------------------------------------------------------------
# BlockMask metadata
# ----------------------------------------------------------------------------

def _dense_to_ordered(dense: np.ndarray):
    """[torch]flex_attention.py:429-436: row sums and a stable descending argsort."""
    dense = dense.astype(np.int32)
    num = dense.sum(axis=-1).astype(np.int32)
    # stable descending sort of 0/1 flags == selected columns ascending, then the rest ascending
    idx = np.argsort(-dense, axis=-1, kind="stable").astype(np.int32)
    return num, idx


def _ordered_to_dense(num: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """[torch]flex_attention.py:399-426 for one (rows, cols) matrix."""
    rows, cols = idx.shape
    dense = np.zeros((rows, cols), np.int32)
    for r in range(rows):
        dense[r, idx[r, :num[r]]] = 1
    return dense


def _transpose_ordered(num: np.ndarray, idx: np.ndarray):
    """[torch]flex_attention.py:439-441."""
    return _dense_to_ordered(_ordered_to_dense(num, idx).T)


def classify_tiles_dense(mask: np.ndarray, block: int = BLOCK):
    """[torch]flex_attention.py:979-1022 (pad with False, 128x128 sums,
    full == block*block, partial == 0 < sum < full). Returns int8 (partial, full)."""
    Q, KV = mask.shape
    nq = -(-Q // block)
    nk = -(-KV // block)
    padded = np.zeros((nq * block, nk * block), bool)
    padded[:Q, :KV] = mask
    sums = padded.reshape(nq, block, nk, block).sum(axis=(1, 3))
    full = sums == block * block
    partial = (sums > 0) & (sums < block * block)
    return partial.astype(np.int8), full.astype(np.int8)


def ordered_from_classes(partial: np.ndarray, full: np.ndarray) -> dict:
    """[torch]flex_attention.py:1067-1090 + from_kv_blocks :586-658: the eight
    int32 tensors of a BlockMask with B = H = 1."""
    kv_num, kv_idx = _dense_to_ordered(partial)
    fkv_num, fkv_idx = _dense_to_ordered(full)
    q_num, q_idx = _transpose_ordered(kv_num, kv_idx)
    fq_num, fq_idx = _transpose_ordered(fkv_num, fkv_idx)
    out = dict(kv_num_blocks=kv_num, kv_indices=kv_idx,
               full_kv_num_blocks=fkv_num, full_kv_indices=fkv_idx,
               q_num_blocks=q_num, q_indices=q_idx,
               full_q_num_blocks=fq_num, full_q_indices=fq_idx)
    return {k: v[None, None] for k, v in out.items()}


def block_mask_from_dense(mask: np.ndarray, block: int = BLOCK) -> dict:
    """create_block_mask(mask_mod, B=None, H=None, Q_LEN, KV_LEN) on a dense mask."""
    return ordered_from_classes(*classify_tiles_dense(mask, block))


def classify_tiles_mtp(gate: np.ndarray, P: int, block: int = BLOCK):
    """Tile classes for the MTP mask without the dense ``S x (P+S)`` matrix.

    Tiles whose keys all lie in the prefix only depend on which query rows are
    pads; the others are evaluated element-wise from the codes, one tile at a time.
    """
    code = mtp_codes(gate, P)
    S = len(code)
    L = P + S
    nq = -(-S // block)
    nk = -(-L // block)
    partial = np.zeros((nq, nk), np.int8)
    full = np.zeros((nq, nk), np.int8)
    kcode = np.concatenate([np.full(P, CODE_X, np.int32), code])
    for qt in range(nq):
        q0, q1 = qt * block, min(S, qt * block + block)
        qc = code[q0:q1]
        nvalid = int((qc != CODE_PAD).sum())
        for kt in range(nk):
            k0, k1 = kt * block, min(L, kt * block + block)
            if k1 <= P:   # every key is a cached regular token, causal holds
                cnt = nvalid * (k1 - k0)
            else:
                qi = np.arange(q0, q1)[:, None] + P
                kj = np.arange(k0, k1)[None, :]
                kc = kcode[k0:k1][None, :]
                qcc = qc[:, None]
                m = (qi >= kj) & (qcc != CODE_PAD) & ((kc == CODE_X) | (kc == qcc))
                cnt = int(m.sum())
            if cnt == block * block:
                full[qt, kt] = 1
            elif cnt > 0:
                partial[qt, kt] = 1
    return partial, full


def block_mask_mtp(gate: np.ndarray, P: int, block: int = BLOCK) -> dict:
    return ordered_from_classes(*classify_tiles_mtp(gate, P, block))


# ----------------------------------------------------------------------------
# Cache
# ----------------------------------------------------------------------------

def regular_index(regular: np.ndarray) -> np.ndarray:
    """collator.py:249: indices of the regular tokens of the chunk."""
    return np.nonzero(np.asarray(regular))[0].astype(np.int32)


def cache_append(prefix: np.ndarray, current: np.ndarray, regular: np.ndarray) -> np.ndarray:
    """collator.py:273-280: cat([prefix, current[:, idx]], axis=seq) for one
    layer's K or V laid out [H, seq, D]."""
    idx = regular_index(regular)
    return np.concatenate([prefix, current[:, idx, :]], axis=1)


# ----------------------------------------------------------------------------
# Dense masked GQA attention (float64 by default)
# ----------------------------------------------------------------------------

def attention_fwd(q: np.ndarray, k: np.ndarray, v: np.ndarray, allowed: np.ndarray,
                  scale: float, p_round=None):
    """q [Hq, S, D], k/v [Hkv, L, D], allowed [S, L] -> (o [Hq, S, D], lse [Hq, S]).

    Dense semantics of [torch]_higher_order_ops/flex_attention.py:159-267:
    s = scale * q k^T, masked -> -inf, lse = logsumexp (fully masked row -> -inf),
    o = softmax(s) v with fully masked rows -> 0 (``_safe_softmax``), query head
    h reads kv head h // G (``repeat_interleave`` :227-229). ``p_round``
    optionally rounds the probabilities before ``p @ v`` (the math path casts
    them to the query dtype there, :264).
    """
    Hq, S, D = q.shape
    Hkv = k.shape[0]
    G = Hq // Hkv
    wd = np.float64
    o = np.zeros((Hq, S, v.shape[2]), wd)
    lse = np.full((Hq, S), -np.inf, wd)
    for h in range(Hq):
        kh = k[h // G].astype(wd)
        vh = v[h // G].astype(wd)
        s = scale * (q[h].astype(wd) @ kh.T)
        s = np.where(allowed, s, -np.inf)
        m = s.max(axis=1)
        rowok = np.isfinite(m)
        msafe = np.where(rowok, m, 0.0)
        e = np.exp(s - msafe[:, None])
        den = e.sum(axis=1)
        p = np.where(rowok[:, None], e / np.where(rowok, den, 1.0)[:, None], 0.0)
        if p_round is not None:
            p = p_round(p)
        o[h] = p @ vh
        lse[h] = np.where(rowok, msafe + np.log(np.where(rowok, den, 1.0)), -np.inf)
    return o, lse


def attention_bwd(q, k, v, o, lse, do, allowed, scale, grad_start: int = 0):
    """Gradients of ``attention_fwd`` (grad_lse = 0), following
    [torch]_higher_order_ops/flex_attention.py:826-990:
    P = exp(s - lse) (fully masked rows -> 0), dV = P^T dO, dP = dO V^T,
    delta = rowsum(O * dO), dS = P * (dP - delta) * scale (masked -> 0),
    dQ = dS K, dK = dS^T Q, dK/dV summed over the G query heads of a kv head.

    Returns (dq [Hq,S,D], dk [Hkv, L-grad_start, D], dv [...]); rows below
    ``grad_start`` are the detached prefix (collator.py:279-280) and dropped.
    """
    Hq, S, D = q.shape
    Hkv, L, _ = k.shape
    G = Hq // Hkv
    wd = np.float64
    dq = np.zeros((Hq, S, D), wd)
    dk = np.zeros((Hkv, L, D), wd)
    dv = np.zeros((Hkv, L, v.shape[2]), wd)
    for h in range(Hq):
        g = h // G
        kh = k[g].astype(wd)
        vh = v[g].astype(wd)
        qh = q[h].astype(wd)
        doh = do[h].astype(wd)
        s = scale * (qh @ kh.T)
        rowok = np.isfinite(lse[h])
        p = np.where(allowed & rowok[:, None],
                     np.exp(s - np.where(rowok, lse[h], 0.0)[:, None]), 0.0)
        dv[g] += p.T @ doh
        dp = doh @ vh.T
        delta = (o[h].astype(wd) * doh).sum(axis=1)
        ds = p * (dp - delta[:, None]) * scale
        dq[h] = ds @ kh
        dk[g] += ds.T @ qh
    return dq, dk[:, grad_start:], dv[:, grad_start:]


# ----------------------------------------------------------------------------
# Credited work
# ----------------------------------------------------------------------------

def tile_areas(bm: dict, S: int, L: int, P: int, block: int = BLOCK):
    """Clipped areas of the non-empty tiles split by key range: (A_pre, A_cur).
    Keys below P are the cached prefix; the rest belong to the chunk."""
    kv_num = bm["kv_num_blocks"][0, 0]
    kv_idx = bm["kv_indices"][0, 0]
    fkv_num = bm["full_kv_num_blocks"][0, 0]
    fkv_idx = bm["full_kv_indices"][0, 0]
    a_pre = 0
    a_cur = 0
    for qt in range(len(kv_num)):
        rows = int(min(block, S - qt * block))
        tiles = [int(t) for t in kv_idx[qt, :kv_num[qt]]] + [int(t) for t in fkv_idx[qt, :fkv_num[qt]]]
        for kt in tiles:
            k0, k1 = kt * block, min(L, kt * block + block)
            npre = max(0, min(k1, P) - k0)
            ncur = (k1 - k0) - npre
            a_pre += rows * npre
            a_cur += rows * ncur
    return a_pre, a_cur


def credited_flops(bm: dict, S: int, L: int, P: int, Hq: int, D: int):
    """FLOP = Hq*D*[4*(A_pre + A_cur) + 6*A_pre + 10*A_cur] (fwd QK^T + PV;
    bwd 3 GEMMs on prefix tiles, 5 on chunk tiles). Returns (fwd, bwd)."""
    a_pre, a_cur = tile_areas(bm, S, L, P)
    fwd = Hq * D * 4 * (a_pre + a_cur)
    bwd = Hq * D * (6 * a_pre + 10 * a_cur)
    return fwd, bwd
