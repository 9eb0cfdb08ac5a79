"""MI355X (gfx950) verify/decode paged-attention path for NebulaSD's swiftLLM backend.

Hand-written HIP kernels behind a C-ABI (``include/nsd_attn.h``), called from
Python wrappers with swiftLLM's kernel signatures (``nebulasd_amd.kernels``).
"""

from .config import EngineConfig, ModelConfig, QWEN3_0_6B, QWEN3_8B
from .infer_state import LlamaInferState, build_infer_state, rope_cache

__all__ = ["EngineConfig", "ModelConfig", "QWEN3_0_6B", "QWEN3_8B", "LlamaInferState",
           "build_infer_state", "rope_cache"]
__version__ = "0.1.0"
