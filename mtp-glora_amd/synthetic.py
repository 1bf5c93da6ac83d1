"""Seeded synthetic MTP chunks in the reference's token layout.

The layout follows mtp_glora/data_utils/dataset.py:25-56: every anchor (a
regular token) is followed immediately by its ``draft_length`` mask tokens;
regular tokens carry consecutive positions starting at ``pos0`` and mask k of
an anchor at position p carries p + k; ``gate_mask`` is 0 on regular tokens, 1
on mask tokens with a label and -1 on padding (collator.py:150-156);
``regular_token_mask`` is 1 exactly on the regular tokens. The benchmark and
the smoke test build their chunks here; no reference data is needed.
"""
from __future__ import annotations

import torch

MASK_TOKEN_ID = 1023


def sample_anchors(n_regular: int, n_anchors: int, seed: int) -> torch.Tensor:
    """``n_anchors`` distinct regular-token indices, uniform without
    replacement from ``seed``, ascending."""
    if not 0 <= n_anchors <= n_regular:
        raise ValueError(f"cannot draw {n_anchors} anchors from {n_regular} regular tokens")
    g = torch.Generator().manual_seed(int(seed))
    return torch.randperm(n_regular, generator=g)[:n_anchors].sort().values


def every_kth_anchor(n_regular: int, k: int, n_anchors: int | None = None) -> torch.Tensor:
    """Anchors at regular indices 0, k, 2k, ... (the dense-MTP stress layout)."""
    a = torch.arange(0, n_regular, k)
    return a if n_anchors is None else a[:n_anchors]


def mtp_chunk(n_regular: int, anchors: torch.Tensor, draft_length: int, pos0: int = 0,
              pad: int = 0, device="cuda", vocab: int = 1024, seed: int = 0) -> dict:
    """One chunk dict (``input_ids``, ``gate_mask``, ``regular_token_mask``,
    ``position_ids``; each ``[1, S]`` int64 on ``device``) with
    S = n_regular + draft_length * len(anchors) + pad."""
    anchors = torch.as_tensor(anchors, dtype=torch.long).unique()
    if anchors.numel() and (anchors.min() < 0 or anchors.max() >= n_regular):
        raise ValueError("anchor index outside the regular tokens")
    is_anchor = torch.zeros(n_regular, dtype=torch.bool)
    is_anchor[anchors] = True
    run = 1 + draft_length * is_anchor.long()            # tokens each regular token contributes
    start = torch.cumsum(run, 0) - run                   # chunk index of each regular token
    content = int(run.sum())
    S = content + pad
    gate = torch.full((S,), -1, dtype=torch.long)
    regular = torch.zeros(S, dtype=torch.long)
    position = torch.zeros(S, dtype=torch.long)
    gate[:content] = 1
    gate[start] = 0
    regular[start] = 1
    position[start] = pos0 + torch.arange(n_regular)
    a_start = start[anchors]
    a_pos = pos0 + anchors
    for k in range(1, draft_length + 1):
        position[a_start + k] = a_pos + k
    g = torch.Generator().manual_seed(int(seed))
    ids = torch.randint(0, vocab - 1, (S,), generator=g)
    ids[(regular == 0) & (gate != -1)] = MASK_TOKEN_ID
    ids[gate == -1] = 0
    dev = torch.device(device)
    return {"input_ids": ids[None].to(dev), "gate_mask": gate[None].to(dev),
            "regular_token_mask": regular[None].to(dev), "position_ids": position[None].to(dev)}
