"""mga_attn_bwd_noalloc (the attention backward whose delta workspace is the
library's fixed per-GPU array) against mga_attn_bwd with a caller-allocated
delta, through the C ABI: dQ, dK and dV equal bit for bit, on two calls in a
row with the second smaller, and with the two passes issued as separate
calls (the dK/dV call reading the delta the dQ call left in the array)."""
import pytest
import torch

from gpu_helpers import chunk_layout, qkv

pytestmark = pytest.mark.gpu


def _inputs(mga, dev, n_reg, n_anchor, P, Hq, Hkv, D, seed):
    seq = chunk_layout(n_reg, n_anchor, 4, P, seed=seed)
    S = len(seq.gate)
    q, k, v, kp, vp, do = qkv(S, P, Hq, Hkv, D, torch.bfloat16, dev, seed=seed)
    bm = mga.build_mtp_block_mask(torch.tensor(seq.gate, device=dev)[None], P)
    kf = torch.cat([kp, k], dim=2)
    vf = torch.cat([vp, v], dim=2)
    bmt = bm.kernel_tensors()
    o, lse = mga.ops.attn_fwd(q, kf, vf, bm.mtp_code, bmt, P, D ** -0.5)
    return q, kf, vf, o, lse, do, bm.mtp_code, bmt, P, D


@pytest.mark.parametrize("split_passes", [False, True])
def test_noalloc_equals_allocating_entry_point(mga, dev, split_passes):
    ops, lib = mga.ops, mga._lib
    cases = [dict(n_reg=1024, n_anchor=64, P=2048, Hq=32, Hkv=8, D=128, seed=1),   # Hq * S = 40 960
             dict(n_reg=256, n_anchor=16, P=256, Hq=4, Hkv=2, D=128, seed=2)]      # then a smaller call
    for c in cases:
        print(f"case {c} split={split_passes}", flush=True)
        q, kf, vf, o, lse, do, code, bmt, P, D = _inputs(mga, dev, **c)
        want = ops.attn_bwd(q, kf, vf, o, lse, do, code, bmt, P, D ** -0.5, P)
        if split_passes:
            bufs = ops.bwd_buffers(q, kf, P)
            ops.attn_bwd(q, kf, vf, o, lse, do, code, bmt, P, D ** -0.5, P, passes=lib.BWD_DQ,
                         buffers=bufs, no_alloc=True)
            got = ops.attn_bwd(q, kf, vf, o, lse, do, code, bmt, P, D ** -0.5, P, passes=lib.BWD_DKDV,
                               buffers=bufs, no_alloc=True)
            got = (bufs["dq"].transpose(1, 2), got[1], got[2])
        else:
            got = ops.attn_bwd(q, kf, vf, o, lse, do, code, bmt, P, D ** -0.5, P, no_alloc=True)
        torch.cuda.synchronize()
        for name, g, w in zip(("dq", "dk", "dv"), got, want):
            assert g is not None and torch.equal(g, w), name


def test_noalloc_rejects_oversized_calls(mga, dev):
    """Hq * S above the fixed workspace is an error before any device work."""
    q, kf, vf, o, lse, do, code, bmt, P, D = _inputs(mga, dev, 256, 16, 0, 4, 2, 128, 3)
    lib = mga._lib
    with pytest.raises(lib.MGAError, match="workspace"):
        lib.call("mga_attn_bwd_noalloc", q.data_ptr(), 128, 128 * 4, kf.data_ptr(), 128, 128,
                 vf.data_ptr(), 128, 128, o.data_ptr(), 128, 512, do.data_ptr(), 128, 512,
                 lse.data_ptr(), q.data_ptr(), 128, 512, None, 128, 256, None, 128, 256, 0,
                 code.data_ptr(), *[bmt[n].data_ptr() for n in (
                     "kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
                     "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices")],
                 1 << 20, 1 << 20, 0, 4, 2, 128, 0, 0.1, lib.BWD_DQ, None)
