"""The hot path inside one captured HIP graph: block-mask build, K/V staging
append, attention forward, both backward passes and the regular-row commit
(the tensor-level calls a training step makes, no host sync inside) are
captured once and replayed. Every kernel is deterministic (fixed-order
reductions, no atomics) and nothing in the path clears memory with
hipMemsetAsync, so each replay must reproduce the eager results bit for bit,
with eager work and synchronisations between the replays."""
import pytest
import torch

from gpu_helpers import chunk_layout, qkv

pytestmark = pytest.mark.gpu


# the last case runs the forward's two launches (4-wave items, then the last
# round as two-group workgroups); the middle one only two-group workgroups
CASES = [(300, 25, 4, 200, 8, 2, 128), (800, 50, 4, 1536, 8, 2, 128), (4000, 250, 4, 2048, 32, 8, 128)]


@pytest.mark.parametrize("case", CASES)
def test_attention_step_graph_replays_bit_exact(mga, dev, case):
    ops = mga.ops
    n_reg, n_anchor, draft, P, Hq, Hkv, D = case
    print(f"case n_reg={n_reg} P={P} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    seq = chunk_layout(n_reg, n_anchor, draft, P, seed=3, pad=11)
    S = len(seq.gate)
    L = P + S
    gate = torch.tensor(seq.gate, device=dev)[None]
    reg = torch.tensor(seq.regular, device=dev)
    q, k, v, kp, vp, do = qkv(S, P, Hq, Hkv, D, torch.bfloat16, dev, seed=5)
    kbuf = torch.zeros(Hkv, L + 64, D, dtype=torch.bfloat16, device=dev)
    vbuf = torch.zeros_like(kbuf)
    kbuf[:, :P] = kp[0]
    vbuf[:, :P] = vp[0]
    committed_k = torch.zeros(Hkv, S + 16, D, dtype=torch.bfloat16, device=dev)
    committed_v = torch.zeros_like(committed_k)
    idx, cnt = ops.regular_index(reg)
    torch.cuda.synchronize()
    R = int(cnt.item())
    scale = D ** -0.5

    def work():
        t = ops.mtp_block_mask_tensors(gate, P)
        bm = {n: t[n] for n in ("kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
                                "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices")}
        ops.kv_append(k, v, kbuf, vbuf, dst_offset=P)
        kf, vf = kbuf[None, :, :L], vbuf[None, :, :L]
        o, lse = ops.attn_fwd(q, kf, vf, t["code"], bm, P, scale)
        dq, dk, dv = ops.attn_bwd(q, kf, vf, o, lse, do, t["code"], bm, P, scale, P)
        ops.kv_append(k, v, committed_k, committed_v, dst_offset=0, idx=idx, n_rows=R)
        return [t["code"], *bm.values(), o, lse, dq, dk, dv, committed_k[:, :R], committed_v[:, :R]]

    eager = [x.clone() for x in work()]
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        work()   # warm-up on a side stream before capture, as torch requires
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = work()

    for rep in range(3):
        # eager work between replays: scribble over the outputs and the cache rows
        for x in out:
            if x.dtype.is_floating_point:
                x.fill_(float("nan"))
            else:
                x.fill_(-7)
        kbuf[:, P:].fill_(3.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, want) in enumerate(zip(out, eager)):
            assert torch.equal(got, want), f"replay {rep}: output {i} differs from the eager run"
        print(f"  replay {rep}: {len(out)} outputs bit-exact", flush=True)


@pytest.mark.parametrize("split_passes", [False, True])
def test_noalloc_backward_graph_replays_bit_exact(mga, dev, split_passes):
    """mga_attn_bwd_noalloc captured in a HIP graph, both passes in one call
    and as two calls, replayed three times against the eager allocating
    mga_attn_bwd, bit for bit. Between replays an eager no-alloc call on other
    inputs overwrites the per-GPU workspace the graph's calls share, and the
    outputs are scribbled over. The first no-alloc call of a test process is
    this test's capture, so the per-device lookup of the workspace runs under
    capture."""
    ops, lib = mga.ops, mga._lib
    print(f"noalloc graph split={split_passes}", flush=True)

    def inputs(n_reg, n_anchor, P, Hq, Hkv, D, seed):
        seq = chunk_layout(n_reg, n_anchor, 4, P, seed=seed, pad=9)
        S = len(seq.gate)
        q, k, v, kp, vp, do = qkv(S, P, Hq, Hkv, D, torch.bfloat16, dev, seed=seed)
        bm = mga.build_mtp_block_mask(torch.tensor(seq.gate, device=dev)[None], P)
        kf, vf = torch.cat([kp, k], dim=2), torch.cat([vp, v], dim=2)
        bmt = bm.kernel_tensors()
        o, lse = ops.attn_fwd(q, kf, vf, bm.mtp_code, bmt, P, D ** -0.5)
        return q, kf, vf, o, lse, do, bm.mtp_code, bmt, P, D

    q, kf, vf, o, lse, do, code, bmt, P, D = inputs(800, 50, 1536, 8, 2, 128, 4)
    other = inputs(300, 20, 256, 4, 2, 128, 5)
    scale = D ** -0.5
    want = ops.attn_bwd(q, kf, vf, o, lse, do, code, bmt, P, scale, P)
    bufs = ops.bwd_buffers(q, kf, P)
    torch.cuda.synchronize()

    def work():
        if split_passes:
            ops.attn_bwd(q, kf, vf, o, lse, do, code, bmt, P, scale, P, passes=lib.BWD_DQ, buffers=bufs,
                         no_alloc=True)
            ops.attn_bwd(q, kf, vf, o, lse, do, code, bmt, P, scale, P, passes=lib.BWD_DKDV, buffers=bufs,
                         no_alloc=True)
        else:
            ops.attn_bwd(q, kf, vf, o, lse, do, code, bmt, P, scale, P, buffers=bufs, no_alloc=True)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        work()
    got = (bufs["dq"].transpose(1, 2), bufs["dk"].transpose(1, 2), bufs["dv"].transpose(1, 2))
    for rep in range(3):
        oq, okf, ovf, oo, olse, odo, ocode, obmt, oP, oD = other
        ops.attn_bwd(oq, okf, ovf, oo, olse, odo, ocode, obmt, oP, oD ** -0.5, oP, no_alloc=True)
        for t in (bufs["dq"], bufs["dk"], bufs["dv"]):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, g, w in zip(("dq", "dk", "dv"), got, want):
            assert torch.equal(g, w), f"replay {rep}: {name} differs from the eager allocating call"
        print(f"  replay {rep}: dq, dk, dv bit-exact", flush=True)
