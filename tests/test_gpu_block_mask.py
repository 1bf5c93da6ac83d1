"""GPU block-mask construction: the eight BlockMask tensors and the per-token
codes equal the oracle's (itself pinned to torch's create_block_mask), and
torch's create_block_mask on the reference mask_mod on the GPU, bit-exact."""
import numpy as np
import pytest
import torch

from gpu_helpers import chunk_layout
from oracle import flex_ref as fr
from oracle import mtp_oracle as mo

pytestmark = pytest.mark.gpu

NAMES = ["kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
         "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices"]


def _gpu_mask(mga, dev, gate, P):
    bm = mga.build_mtp_block_mask(torch.tensor(gate, device=dev)[None], P)
    torch.cuda.synchronize()
    return bm


@pytest.mark.parametrize("case", [
    dict(n_reg=300, n_anchor=20, draft=4, P=0),
    dict(n_reg=300, n_anchor=20, draft=4, P=128),
    dict(n_reg=250, n_anchor=40, draft=3, P=200, pad=70),
    dict(n_reg=100, n_anchor=60, draft=8, P=384),
    dict(n_reg=60, n_anchor=5, draft=2, P=0, pad=3),
    dict(n_reg=512, n_anchor=128, draft=4, P=1024),
    dict(n_reg=90, n_anchor=30, draft=4, P=256, pad=30, tail=True),
])
def test_block_mask_small(mga, dev, case):
    seq = chunk_layout(case["n_reg"], case["n_anchor"], case["draft"], case["P"], seed=case["n_reg"],
                       pad=case.get("pad", 0), tail=case.get("tail", False))
    bm = _gpu_mask(mga, dev, seq.gate, case["P"])
    want = mo.block_mask_mtp(seq.gate, case["P"])
    assert np.array_equal(bm.mtp_code.cpu().numpy(), mo.mtp_codes(seq.gate, case["P"]))
    ref = fr.block_mask_tensors(fr.reference_block_mask(torch.tensor(seq.gate, device=dev)[None],
                                                        case["P"], device=dev))
    for n in NAMES:
        got = getattr(bm, n).cpu().numpy()
        assert got.dtype == np.int32 and np.array_equal(got, want[n]), n
        assert np.array_equal(got, ref[n]), n
    assert bm.seq_lengths == (len(seq.gate), case["P"] + len(seq.gate))


def test_all_pad_chunk(mga, dev):
    gate = np.full(300, -1, np.int64)
    bm = _gpu_mask(mga, dev, gate, 128)
    for n, v in mo.block_mask_mtp(gate, 128).items():
        assert np.array_equal(getattr(bm, n).cpu().numpy(), v), n
    assert int(bm.kv_num_blocks.sum()) == 0 and int(bm.full_kv_num_blocks.sum()) == 0


@pytest.mark.parametrize("cfg", [
    dict(n_reg=4096, n_anchor=256, draft=4, P=8192),            # config 2
    dict(n_reg=4096, n_anchor=512, draft=4, P=28672),           # config 3, last chunk
    dict(n_reg=2048, n_anchor=512, draft=8, P=16384, every=4),  # config 5
    dict(n_reg=4096, n_anchor=256, draft=4, P=126976),          # config 4, chunk 32
])
def test_block_mask_config_sizes(mga, dev, cfg):
    seq = chunk_layout(cfg["n_reg"], cfg["n_anchor"], cfg["draft"], cfg["P"], seed=2,
                       every=cfg.get("every"))
    bm = _gpu_mask(mga, dev, seq.gate, cfg["P"])
    want = mo.block_mask_mtp(seq.gate, cfg["P"])
    for n in NAMES:
        assert np.array_equal(getattr(bm, n).cpu().numpy(), want[n]), n
