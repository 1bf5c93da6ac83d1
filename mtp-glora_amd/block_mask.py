"""The MTP BlockMask: torch's ``BlockMask`` built on the GPU, plus the per-token
codes the HIP attention kernels evaluate inside partial tiles.

``build_mtp_block_mask(gate, P)`` returns the same eight tensors as the
reference's ``create_block_mask(mask_mod, B=None, H=None, Q_LEN=S,
KV_LEN=P+S)`` (mtp_glora/data_utils/collator.py:290-363) without evaluating
the dense S x (P+S) mask: a code kernel, a per-tile classifier and a list
builder (mtp-glora_amd/csrc/mga_mask.hip).
"""
from __future__ import annotations

import torch
from torch.nn.attention.flex_attention import BlockMask

from . import ops

CODE_PAD = -1
CODE_X = -2


def _code_mask_mod(code: torch.Tensor, P: int):
    """A mask_mod equal to the reference predicate (collator.py:323-355),
    written over the codes, so the mask stays usable by torch's flex_attention,
    ``to_dense()`` and printing. A cached prefix key (kv_idx < P) is a regular
    token; nothing is computed until the mask_mod is called."""

    def mask_mod(b, h, q_idx, kv_idx):
        qc = code[q_idx]
        kc = torch.where(kv_idx < P, CODE_X, code[(kv_idx - P).clamp(min=0)])
        return (q_idx + P >= kv_idx) & (qc != CODE_PAD) & ((kc == CODE_X) | (kc == qc))

    return mask_mod


class MTPBlockMask(BlockMask):
    """``BlockMask`` carrying ``mtp_code`` (int32 [S]) and ``prefix_len`` (P)."""

    mtp_code: torch.Tensor
    prefix_len: int

    @classmethod
    def from_tensors(cls, t: dict, S: int, P: int) -> "MTPBlockMask":
        code = t["code"]
        bm = cls(
            seq_lengths=(S, P + S),
            kv_num_blocks=t["kv_num_blocks"], kv_indices=t["kv_indices"],
            full_kv_num_blocks=t["full_kv_num_blocks"], full_kv_indices=t["full_kv_indices"],
            q_num_blocks=t["q_num_blocks"], q_indices=t["q_indices"],
            full_q_num_blocks=t["full_q_num_blocks"], full_q_indices=t["full_q_indices"],
            BLOCK_SIZE=(ops.BLOCK, ops.BLOCK),
            mask_mod=_code_mask_mod(code, P),
        )
        bm.mtp_code = code
        bm.prefix_len = int(P)
        return bm

    def kernel_tensors(self) -> dict:
        return dict(kv_num_blocks=self.kv_num_blocks, kv_indices=self.kv_indices,
                    full_kv_num_blocks=self.full_kv_num_blocks, full_kv_indices=self.full_kv_indices,
                    q_num_blocks=self.q_num_blocks, q_indices=self.q_indices,
                    full_q_num_blocks=self.full_q_num_blocks, full_q_indices=self.full_q_indices)

    def to(self, device) -> "MTPBlockMask":
        """Keeps the MTP metadata (``BlockMask.to`` would return a plain BlockMask);
        a mask already on ``device`` is returned as is."""
        names = ["kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
                 "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices"]
        if torch.device(device) == self.mtp_code.device:
            return self
        t = {n: getattr(self, n).to(device) for n in names}
        t["code"] = self.mtp_code.to(device)
        return MTPBlockMask.from_tensors(t, self.seq_lengths[0], self.prefix_len)


def build_mtp_block_mask(gate: torch.Tensor, P: int) -> MTPBlockMask:
    """MTP BlockMask for a chunk (``gate``: [1, S] int64, -1 pad / 0 / 1) that
    attends to a cached prefix of ``P`` regular tokens."""
    S = gate.shape[-1]
    t = ops.mtp_block_mask_tensors(gate, int(P))
    return MTPBlockMask.from_tensors(t, S, int(P))
