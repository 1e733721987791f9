"""MI355X-native host runtime for the DeepSeek-V2-Lite decode step (HIP kernels via triton_kernels._hip)."""

from .config import DSV2Config
from .cache import CompressedKVCache
from .weights import LayerWeights, ModelWeights, init_weights, pack_hf_layer, quantize_experts_fp8
from .engine import DecodeEngine, FAMILIES, plan_splits, moe_tile_tokens
from .checkpoint import Checkpoint, config_from_hf, load_tokenizer, load_weights

__all__ = ["DSV2Config", "CompressedKVCache", "LayerWeights", "ModelWeights", "init_weights", "pack_hf_layer",
           "quantize_experts_fp8",
           "DecodeEngine", "FAMILIES", "plan_splits", "moe_tile_tokens", "Checkpoint", "config_from_hf",
           "load_tokenizer", "load_weights"]
