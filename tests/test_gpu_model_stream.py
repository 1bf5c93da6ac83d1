"""Config 1 end to end: a random-init Qwen3-style decoder (transformers'
Qwen3ForCausalLM: 2 layers, hidden 256, 4 query / 2 KV heads, head_dim 64,
vocab 1024, fp32) with Gated LoRA (rank 8) on q/k/v/o, trained over an MTP
sequence in chunks exactly as the reference's chunk loop drives it
(mtp_glora/trainer/trainer.py:95-136): reset -> per chunk prepare (BlockMask)
-> forward with the cache -> loss.backward -> extract the regular-token K/V.
The same stream also runs through transformers' LlamaForCausalLM, the Llama
call site (modeling_llama.py:292-332): there the first chunk gets
past_key_values=None, so the model makes its own DynamicCache
(modeling_llama.py:451-452) and the manager takes it over, and the attention
is found under the reference's own key "flex_attention"
(trainer/utils.py:68) after register(replace_flex=True).

The HIP path runs through the drop-in boundary only: the attention function
registered with transformers, StreamingKVCache as past_key_values and
StreamingKVCacheManager. It is checked against
  * the reference's chunked procedure on the CPU in float64: the same model
    with dense masked attention (the flex_attention semantics, the oracle's
    MTP mask), transformers' DynamicCache, and the regular-token gather + cat +
    detach of collator.py:270-287 between chunks -- forward logits and the
    LoRA gradients accumulated over all chunks;
  * a single pass over the whole sequence with the full MTP mask (forward
    logits), the chunk-equivalence invariant: blocks never straddle chunks.
Tolerance (fp32 model, fp32 arithmetic throughout: the attention runs the
fp32 MFMAs): logits max-abs 1e-5 and mean-abs 1e-6; LoRA gradients within
1e-5 of the largest reference entry (max) and 1e-6 of it (mean).

A bf16 model with the package's own apply_lora_to_model / GatedLoRALinear is
checked against the same float64 procedure, bounded by 2x the deviation of
the reference's procedure run in bf16 (test at the end of the file).
"""
import importlib

import numpy as np
import pytest
import torch

from oracle import mtp_oracle as mo

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")
from transformers import (AttentionInterface, LlamaConfig, LlamaForCausalLM, Qwen3Config,  # noqa: E402
                          Qwen3ForCausalLM)
from transformers.cache_utils import DynamicCache  # noqa: E402

N_REG, N_CHUNKS, N_ANCHOR, DRAFT, RANK, VOCAB = 1024, 4, 16, 4, 8, 1024
MASK_ID = VOCAB - 1


class GatedLoRA(torch.nn.Module):
    """base(x) + s * B(A(x)) * gate, the gate being the chunk's clamped
    gate_mask [1, S, 1] (1 on mask tokens with a label)."""

    def __init__(self, base: torch.nn.Linear, rank: int, gen: torch.Generator):
        super().__init__()
        self.base = base
        self.A = torch.nn.Parameter(torch.randn(rank, base.in_features, generator=gen) * 0.05)
        self.B = torch.nn.Parameter(torch.randn(base.out_features, rank, generator=gen) * 0.05)
        self.scale = 2.0
        self.gate = None

    def forward(self, x):
        return self.base(x) + self.scale * ((x @ self.A.t()) @ self.B.t()) * self.gate


def dense_masked_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kw):
    """flex_attention's dense semantics with a boolean [.., S, L] mask: GQA,
    masked scores -inf, a fully masked row gives 0."""
    G = query.shape[1] // key.shape[1]
    k = key.repeat_interleave(G, dim=1)
    v = value.repeat_interleave(G, dim=1)
    s = (query @ k.transpose(-1, -2)) * scaling
    m = attention_mask.bool()
    s = s.masked_fill(~m, float("-inf"))
    rowok = m.any(dim=-1, keepdim=True)
    p = torch.softmax(s.masked_fill(~rowok, 0.0), dim=-1) * rowok
    return (p @ v).transpose(1, 2).contiguous(), None


def flex_like_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kw):
    """The reference's compiled flex path on 16-bit operands: scores and
    softmax in fp32, the probabilities rounded to the operand dtype before
    P V (fp32 accumulation), the output rounded to the operand dtype."""
    dt = query.dtype
    G = query.shape[1] // key.shape[1]
    k = key.float().repeat_interleave(G, dim=1)
    v = value.float().repeat_interleave(G, dim=1)
    s = (query.float() @ k.transpose(-1, -2).contiguous()) * scaling
    m = attention_mask.bool()
    s = s.masked_fill(~m, float("-inf"))
    rowok = m.any(dim=-1, keepdim=True)
    p = torch.softmax(s.masked_fill(~rowok, 0.0), dim=-1) * rowok
    o = (p.to(dt).float() @ v).to(dt)
    return o.transpose(1, 2).contiguous(), None


def build_model(attn: str, dtype, device, seed: int = 0, family: str = "qwen3", lora: bool = True):
    dims = dict(vocab_size=VOCAB, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                max_position_embeddings=4096, tie_word_embeddings=False)
    cfg = Qwen3Config(**dims) if family == "qwen3" else LlamaConfig(**dims)
    cfg._attn_implementation = attn
    torch.manual_seed(seed)
    model = Qwen3ForCausalLM(cfg) if family == "qwen3" else LlamaForCausalLM(cfg)
    if not lora:
        return model.to(device=device, dtype=dtype), []
    gen = torch.Generator().manual_seed(seed + 1)
    loras = []
    for layer in model.model.layers:
        att = layer.self_attn
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            lo = GatedLoRA(getattr(att, name), RANK, gen)
            setattr(att, name, lo)
            loras.append(lo)
    for p in model.parameters():
        p.requires_grad_(False)
    for lo in loras:
        lo.A.requires_grad_(True)
        lo.B.requires_grad_(True)
    return model.to(device=device, dtype=dtype), loras


def make_sequence(seed: int = 0):
    """N_CHUNKS chunks of N_REG / N_CHUNKS regular tokens with N_ANCHOR anchors
    each; token ids uniform from the seed, <mask> = MASK_ID; labels for the loss."""
    rng = np.random.default_rng(seed)
    per = N_REG // N_CHUNKS
    chunks = []
    for c in range(N_CHUNKS):
        seq = mo.synth_sequence(per, mo.sample_anchors(per, N_ANCHOR, seed + c), DRAFT, pos0=c * per)
        ids = rng.integers(0, VOCAB - 1, size=len(seq.gate))
        ids[seq.regular == 0] = MASK_ID
        labels = rng.integers(0, VOCAB - 1, size=len(seq.gate))
        chunks.append((seq, ids, labels))
    return chunks


def chunk_loss(logits, labels):
    return torch.nn.functional.cross_entropy(logits[0].float(), labels, reduction="sum") / labels.numel()


def run_hip(mga, chunks, dev, family="qwen3", attn="mtp_hip"):
    model, loras = build_model(attn, torch.float32, dev, family=family)
    mgr = mga.StreamingKVCacheManager(capacity=4096)
    mgr.reset_cache()
    # Qwen3: the manager's cache from the first chunk on; Llama: None, as the
    # reference trainer passes it (trainer.py:100), so the model builds a
    # DynamicCache that the first carry-over takes over
    pkv = mgr.new_cache(num_layers=2) if family == "qwen3" else None
    logits_out = []
    for c, (seq, ids, labels) in enumerate(chunks):
        chunk = {"input_ids": torch.tensor(ids, device=dev)[None],
                 "gate_mask": torch.tensor(seq.gate, device=dev)[None],
                 "regular_token_mask": torch.tensor(seq.regular, device=dev)[None],
                 "position_ids": torch.tensor(seq.position, device=dev)[None]}
        chunk = mgr.prepare_data_with_kv_cache(chunk)
        gate = chunk["gate_mask"].to(torch.float32)
        for lo in loras:
            lo.gate = gate
        out = model(input_ids=chunk["input_ids"], attention_mask=chunk["attention_mask"],
                    position_ids=chunk["position_ids"], past_key_values=pkv, use_cache=True)
        chunk_loss(out.logits, torch.tensor(labels, device=dev)).backward()
        logits_out.append(out.logits.detach().double().cpu())
        if c + 1 < len(chunks):
            pkv = mgr.extract_regular_kv_cache_for_next_chunk(chunk, out.past_key_values)
    torch.cuda.synchronize()
    grads = [torch.cat([lo.A.grad.flatten(), lo.B.grad.flatten()]).double().cpu() for lo in loras]
    return logits_out, grads


def run_reference(chunks, family="qwen3", dtype=torch.float64, device="cpu", attn="mtp_dense_ref", state=None):
    """The reference's chunk procedure (DynamicCache, gather + cat + detach
    between chunks); state: weights to load (the test GatedLoRA's names)."""
    model, loras = build_model(attn, dtype, device, family=family)
    if state is not None:
        model.load_state_dict({k: v.to(dtype) for k, v in state.items()}, strict=True)
    pkv = None
    P = 0
    logits_out = []
    for c, (seq, ids, labels) in enumerate(chunks):
        mask = torch.tensor(mo.mtp_mask_dense(seq.gate, P), device=device)[None, None]
        gate = torch.tensor(seq.gate, device=device).clamp(min=0)[None, :, None].to(dtype)
        for lo in loras:
            lo.gate = gate
        out = model(input_ids=torch.tensor(ids, device=device)[None], attention_mask=mask,
                    position_ids=torch.tensor(seq.position, device=device)[None], past_key_values=pkv,
                    use_cache=True)
        chunk_loss(out.logits, torch.tensor(labels, device=device)).backward()
        logits_out.append(out.logits.detach().double().cpu())
        # collator.py:270-287: keep the regular rows, detached
        idx = torch.tensor(np.nonzero(seq.regular)[0], device=device)
        new = DynamicCache()
        for li, layer in enumerate(out.past_key_values.layers):
            k = torch.cat([layer.keys[:, :, :P], layer.keys[:, :, P:][:, :, idx]], dim=2).detach()
            v = torch.cat([layer.values[:, :, :P], layer.values[:, :, P:][:, :, idx]], dim=2).detach()
            new.update(k, v, li)
        pkv = new
        P += len(idx)
    grads = [torch.cat([lo.A.grad.flatten(), lo.B.grad.flatten()]).double().cpu() for lo in loras]
    return logits_out, grads


def run_single_pass(chunks, family="qwen3"):
    """One forward over the whole sequence with the full MTP mask."""
    model, loras = build_model("mtp_dense_ref", torch.float64, "cpu", family=family)
    gate_all = np.concatenate([s.gate for s, _, _ in chunks])
    ids = np.concatenate([i for _, i, _ in chunks])
    pos = np.concatenate([s.position for s, _, _ in chunks])
    for lo in loras:
        lo.gate = torch.tensor(gate_all).clamp(min=0)[None, :, None].double()
    mask = torch.tensor(mo.mtp_mask_dense(gate_all, 0))[None, None]
    with torch.no_grad():
        out = model(input_ids=torch.tensor(ids)[None], attention_mask=mask,
                    position_ids=torch.tensor(pos)[None], use_cache=False)
    return torch.split(out.logits, [len(s.gate) for s, _, _ in chunks], dim=1)


def _check(name, got, ref, max_abs, mean_abs):
    err = (got - ref).abs()
    print(f"  {name}: max-abs {err.max().item():.3e} mean-abs {err.mean().item():.3e}", flush=True)
    assert err.max().item() <= max_abs and err.mean().item() <= mean_abs, name


def _stream_against_reference(dev, fused_qk_norm_rope: bool, monkeypatch, family="qwen3"):
    mga = importlib.import_module("mtp-glora_amd")
    AttentionInterface.register("mtp_dense_ref", dense_masked_attention)
    chunks = make_sequence(0)
    with monkeypatch.context() as m:
        if family == "llama":
            # the reference's attn_implementation="flex_attention" finds the
            # HIP attention; the original entry comes back after the test
            from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
            m.setitem(ALL_ATTENTION_FUNCTIONS._global_mapping, "flex_attention",
                      ALL_ATTENTION_FUNCTIONS._global_mapping["flex_attention"])
            mga.register("mtp_hip", replace_flex=True)
            attn = "flex_attention"
        else:
            mga.register("mtp_hip")
            attn = "mtp_hip"
        if fused_qk_norm_rope:
            from transformers.models.qwen3 import modeling_qwen3
            m.setattr(modeling_qwen3.Qwen3Attention, "forward", mga.qwen3_attention_forward)
        hip_logits, hip_grads = run_hip(mga, chunks, dev, family=family, attn=attn)
    ref_logits, ref_grads = run_reference(chunks, family=family)
    one_pass = run_single_pass(chunks, family=family)
    for c in range(len(chunks)):
        # chunk equivalence of the reference itself, then the HIP stream against both
        assert torch.allclose(ref_logits[c], one_pass[c], atol=1e-9, rtol=0)
        _check(f"logits chunk {c}", hip_logits[c], ref_logits[c], 1e-5, 1e-6)
    for i, (g, r) in enumerate(zip(hip_grads, ref_grads)):
        scale = r.abs().max().item()
        assert scale > 0
        _check(f"lora grad {i} (scale {scale:.2e})", g / scale, r / scale, 1e-5, 1e-6)


def test_config1_chunk_stream_through_transformers_qwen3(dev, monkeypatch):
    _stream_against_reference(dev, False, monkeypatch)


def test_config1_chunk_stream_with_fused_qk_norm_rope(dev, monkeypatch):
    """The same stream with Qwen3Attention.forward replaced by the adapter that
    runs q_norm / k_norm / rope as one HIP kernel (forward and backward): the
    LoRA gradients of q_proj and k_proj flow through its backward."""
    _stream_against_reference(dev, True, monkeypatch)


def test_config1_chunk_stream_through_transformers_llama(dev, monkeypatch):
    """The Llama call site: LlamaAttention.forward's cache update and attention
    lookup, the model's own DynamicCache on the first chunk, and the HIP
    attention registered under "flex_attention"."""
    _stream_against_reference(dev, False, monkeypatch, family="llama")


def run_hip_package_lora(mga, chunks, dev):
    """The bf16 stream with the package's own Gated LoRA: apply_lora_to_model
    on q/k/v/o (rank 8, alpha 16), each chunk's clamped gate_mask handed to
    every GatedLoRALinear (the reference's projections take it as their second
    argument, modeling_qwen3.py:247-251, 303; transformers' stock attention
    calls them with one, so a forward pre-hook supplies it). lora_B gets
    random values (the reference initialises it to zero) so that every LoRA
    gradient is non-trivial. Returns logits, LoRA gradients and the initial
    weights under the test GatedLoRA's names."""
    model, _ = build_model("mtp_hip", torch.bfloat16, dev, lora=False)
    mga.apply_lora_to_model(model, target_modules=["q_proj", "k_proj", "v_proj", "o_proj"], rank=RANK,
                            alpha=2 * RANK, dropout=0.0)
    gen = torch.Generator().manual_seed(3)
    mods = [getattr(layer.self_attn, n) for layer in model.model.layers for n in ("q_proj", "k_proj", "v_proj",
                                                                                   "o_proj")]
    assert all(isinstance(m, mga.GatedLoRALinear) for m in mods)
    current_gate = [None]
    for m in mods:
        with torch.no_grad():
            m.lora_B.weight.copy_(torch.randn(m.lora_B.weight.shape, generator=gen) * 0.05)
        m.register_forward_pre_hook(lambda mod, args, kwargs: (args, {"gate_mask": current_gate[0]}),
                                    with_kwargs=True)
    rename = {".base_layer.weight": ".base.weight", ".lora_A.weight": ".A", ".lora_B.weight": ".B"}
    state = {}
    for k, v in model.state_dict().items():
        for a, b in rename.items():
            if k.endswith(a):
                k = k[: -len(a)] + b
        state[k] = v.detach().double().cpu()
    mgr = mga.StreamingKVCacheManager(capacity=4096)
    mgr.reset_cache()
    pkv = mgr.new_cache(num_layers=2)
    logits_out = []
    for c, (seq, ids, labels) in enumerate(chunks):
        chunk = {"input_ids": torch.tensor(ids, device=dev)[None],
                 "gate_mask": torch.tensor(seq.gate, device=dev)[None],
                 "regular_token_mask": torch.tensor(seq.regular, device=dev)[None],
                 "position_ids": torch.tensor(seq.position, device=dev)[None]}
        chunk = mgr.prepare_data_with_kv_cache(chunk)
        current_gate[0] = chunk["gate_mask"]
        out = model(input_ids=chunk["input_ids"], attention_mask=chunk["attention_mask"],
                    position_ids=chunk["position_ids"], past_key_values=pkv, use_cache=True)
        assert out.logits.dtype == torch.bfloat16
        chunk_loss(out.logits, torch.tensor(labels, device=dev)).backward()
        logits_out.append(out.logits.detach().double().cpu())
        if c + 1 < len(chunks):
            pkv = mgr.extract_regular_kv_cache_for_next_chunk(chunk, out.past_key_values)
    torch.cuda.synchronize()
    grads = [torch.cat([m.lora_A.weight.grad.flatten(), m.lora_B.weight.grad.flatten()]).double().cpu()
             for m in mods]
    return logits_out, grads, state


def test_config1_bf16_stream_with_package_gated_lora(dev):
    """Config 1's model in bf16 with the package's apply_lora_to_model /
    GatedLoRALinear, the HIP attention, StreamingKVCache and the manager,
    against the reference's procedure in float64 on the same (bf16) weights.
    Yardstick: the reference's procedure run in bf16 on the GPU with torch ops
    and flex-like attention (fp32 softmax, P rounded to bf16), i.e. what the
    reference's own bf16 run deviates from float64 by. The HIP stream's max-
    and mean-abs deviation of the logits (all chunks) and of each LoRA
    gradient (relative to its largest entry) must stay within 2x the
    yardstick's."""
    mga = importlib.import_module("mtp-glora_amd")
    mga.register("mtp_hip")
    AttentionInterface.register("mtp_dense_ref", dense_masked_attention)
    AttentionInterface.register("mtp_flex_like", flex_like_attention)
    chunks = make_sequence(1)
    hip_logits, hip_grads, state = run_hip_package_lora(mga, chunks, dev)
    ref_logits, ref_grads = run_reference(chunks, state=state)
    y_logits, y_grads = run_reference(chunks, dtype=torch.bfloat16, device=dev, attn="mtp_flex_like", state=state)
    H, R, Y = (torch.cat([t.flatten() for t in x]) for x in (hip_logits, ref_logits, y_logits))

    def within(name, got, ref, yard):
        e, ey = (got - ref).abs(), (yard - ref).abs()
        print(f"  {name}: max-abs {e.max().item():.3e} mean-abs {e.mean().item():.3e} "
              f"(bf16 reference run: {ey.max().item():.3e} / {ey.mean().item():.3e})", flush=True)
        assert e.max().item() <= 2 * ey.max().item() and e.mean().item() <= 2 * ey.mean().item(), name

    within("logits", H, R, Y)
    for i, (g, r, y) in enumerate(zip(hip_grads, ref_grads, y_grads)):
        scale = r.abs().max().item()
        assert scale > 0
        within(f"lora grad {i}", g / scale, r / scale, y / scale)
