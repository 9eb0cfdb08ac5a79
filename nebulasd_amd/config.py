"""Model and engine configuration read by the attention path.

Duck-type compatible with swiftLLM's ``LlamaModelConfig``
(swiftLLM/swiftllm/model_config.py:19-36) and the ``EngineConfig`` fields the
kernels read (swiftLLM/swiftllm/engine_config.py:14-19): the wrappers only
touch ``num_layers``, ``num_q_heads``, ``num_kv_heads``, ``head_dim``,
``rms_norm_eps``, ``rope_theta``, ``rope_scaling``, ``has_qk_norm``,
``block_size`` and ``max_blocks_per_seq``, so the reference's own config
objects can be passed unchanged.
"""

from __future__ import annotations

import dataclasses


class ModelConfig:
    """Attention-relevant part of a HF-style config dict.

    Field derivation follows swiftLLM/swiftllm/model_config.py:19-36.
    """

    def __init__(self, cfg: dict):
        if cfg["model_type"] not in {"llama", "qwen3"}:
            raise ValueError(f"unsupported model_type {cfg['model_type']!r}")
        self.model_type = cfg["model_type"]
        self.has_qk_norm = self.model_type == "qwen3"
        self.num_layers = cfg["num_hidden_layers"]
        self.num_q_heads = cfg["num_attention_heads"]
        self.num_kv_heads = cfg.get("num_key_value_heads", self.num_q_heads)
        self.hidden_size = cfg["hidden_size"]
        self.head_dim = cfg.get("head_dim", self.hidden_size // self.num_q_heads)
        self.vocab_size = cfg["vocab_size"]
        self.max_position_embeddings = cfg["max_position_embeddings"]
        self.ffn_inter_dim = cfg["intermediate_size"]
        self.rms_norm_eps = cfg["rms_norm_eps"]
        self.rope_theta = cfg.get("rope_theta", 10000)
        self.rope_scaling = cfg.get("rope_scaling", 1.0) or 1.0

    def get_kvslot_size(self, itemsize: int = 2) -> int:
        """Bytes of K+V of one token over all layers (model_config.py:38-42)."""
        return 2 * self.num_layers * self.num_kv_heads * self.head_dim * itemsize


@dataclasses.dataclass
class EngineConfig:
    """The paged-attention fields of swiftLLM's EngineConfig (engine_config.py:14-19)."""

    block_size: int = 16
    max_blocks_per_seq: int = 2048
    max_seqs_in_block_table: int = 128
    num_gpu_blocks: int = 24576


# Public Qwen3 shapes.  Qwen3-8B: swiftLLM/tests/test_qwen3_qk_norm.py:6-19
# (36 layers as deployed); Qwen3-0.6B: 28 layers, 16 q / 8 kv heads, d=128.
QWEN3_8B = {
    "model_type": "qwen3", "num_hidden_layers": 36, "num_attention_heads": 32,
    "num_key_value_heads": 8, "hidden_size": 4096, "head_dim": 128, "vocab_size": 151936,
    "max_position_embeddings": 40960, "intermediate_size": 12288, "rope_theta": 1000000,
    "rms_norm_eps": 1e-6, "hidden_act": "silu",
}
QWEN3_0_6B = {
    "model_type": "qwen3", "num_hidden_layers": 28, "num_attention_heads": 16,
    "num_key_value_heads": 8, "hidden_size": 1024, "head_dim": 128, "vocab_size": 151936,
    "max_position_embeddings": 40960, "intermediate_size": 3072, "rope_theta": 1000000,
    "rms_norm_eps": 1e-6, "hidden_act": "silu",
}
