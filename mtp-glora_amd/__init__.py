"""MI355X-native streaming KV cache + MTP block-masked attention for
MTP-GLoRA's chunked training.

The package mirrors the reference's operator boundaries for this path:

* ``StreamingKVCacheManager``   - mtp_glora/data_utils/collator.py:178-363
* ``StreamingKVCache``          - the transformers ``Cache`` the adapters call
  (``update`` / ``get_seq_length`` / legacy tuple access)
* ``mtp_attention_forward``     - the ``ALL_ATTENTION_FUNCTIONS`` entry
  (signature of [tf]integrations/flex_attention.py:262)
* ``build_mtp_block_mask``      - the BlockMask of collator.py:290-363
* ``StableSoftCrossEntropy``    - the sampler's soft cross-entropy,
  mtp_glora/core/loss.py:259-330
* ``GatedLoRALinear`` / ``apply_lora_to_model`` - the gated LoRA layers,
  mtp_glora/models/layers/gated_lora.py
* ``qk_norm_rope`` / ``qwen3_attention_forward`` - q_norm, k_norm and
  apply_rotary_pos_emb of Qwen3Attention.forward
  (mtp_glora/models/modeling_qwen3.py:254-305), fused

All arithmetic runs in libmtp_glora_amd.so (HIP, gfx950) through the C ABI in
include/mtp_glora_amd.h. The directory name is not a Python identifier; import
it with ``importlib.import_module("mtp-glora_amd")``.
"""
from . import _lib, ops
from .attention import mtp_attention, mtp_attention_forward, register
from .block_mask import MTPBlockMask, build_mtp_block_mask
from .cache import StreamingKVCache
from .lora import GatedLoRALinear, apply_lora_to_model, gated_lora_linear
from .loss import StableSoftCrossEntropy
from .manager import StreamingKVCacheManager
from .rope import qk_norm_rope, qwen3_attention_forward

__all__ = [
    "StreamingKVCache", "StreamingKVCacheManager", "MTPBlockMask", "build_mtp_block_mask",
    "mtp_attention", "mtp_attention_forward", "register", "ops", "StableSoftCrossEntropy",
    "qk_norm_rope", "qwen3_attention_forward", "GatedLoRALinear", "apply_lora_to_model", "gated_lora_linear",
]


def library_path() -> str:
    return str(_lib.LIB_PATH)


def load_library():
    """Load libmtp_glora_amd.so (raises if it is not built)."""
    return _lib.load()
