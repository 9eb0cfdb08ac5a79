"""Native decoder stack for decode/verify rows (``nsd_decoder_forward``).

The reference runs its layers from Python (swiftLLM/swiftllm/worker/model.py:
280-289, each ``LlamaTransformerLayer.forward``, layers/transformer_layer.py:
83-201), a dozen kernel and GEMM calls per layer.  At the draft's and the
target's decode/verify batches the GPU finishes a layer faster than Python
issues it.  ``DecoderStack`` hands the whole stack of a forward to one C++
call that enqueues the same sequence on the current stream: fused
add-RMSNorm, one q/k/v projection, the fused QK-norm + RoPE + KV-store
prologue and paged attention (one launch for decode batches), the O
projection, fused add-RMSNorm, the fused
up/gate + SiLU-and-mul, the down projection (the projections are this
library's split-k GEMM, whose fp32 split partials the next kernel sums where
it reads them).  The embedding lookup and the post-layer stay in Python.
"""

from __future__ import annotations

import ctypes
from ctypes import c_void_p

import torch

from . import _lib
from .kernels._util import cache_dims, check_block_table, ptr, require, require_cuda, stream_of
from .plan import plan_for

__all__ = ["DecoderStack", "MAX_ROWS"]

MAX_ROWS = 128  # rows of one forward (the fused up/gate kernel's single pass)


class _Layer(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("w_qkv", "w_o", "w_up_gate", "w_down", "norm_in", "norm_post",
                                        "q_norm", "k_norm")]


class DecoderStack:
    """Every layer of a decoder for the decode/verify rows of a forward.

    ``layers``: one dict per layer with fp16 device tensors ``wqkv``
    [(Hq + 2 Hkv) d, hidden] (q, k, v projections stacked), ``wo``
    [hidden, Hq d], ``wug`` [2 I, hidden] (up rows, then gate), ``wd``
    [hidden, I], ``n_in`` / ``n_post`` [hidden] and optionally ``q_norm`` /
    ``k_norm`` [d].  The tensors are referenced, not copied: they must stay
    unchanged while the stack is in use.
    """

    def __init__(self, model_config, layers: list, max_rows: int = MAX_ROWS):
        mc = model_config
        if len(layers) != mc.num_layers:
            raise ValueError(f"{len(layers)} layer weight sets for a {mc.num_layers}-layer model")
        H, I, hq, hkv, d = mc.hidden_size, mc.ffn_inter_dim, mc.num_q_heads, mc.num_kv_heads, mc.head_dim
        shapes = {"wqkv": ((hq + 2 * hkv) * d, H), "wo": (H, hq * d), "wug": (2 * I, H), "wd": (H, I),
                  "n_in": (H,), "n_post": (H,), "q_norm": (d,), "k_norm": (d,)}
        for i, lw in enumerate(layers):
            for name, shape in shapes.items():
                t = lw.get(name)
                if t is None and name in ("q_norm", "k_norm"):
                    continue
                if t is None:
                    raise ValueError(f"layer {i}: missing {name}")
                require_cuda(t)
                require(t, torch.float16, f"layer {i} {name}")
                if tuple(t.shape) != shape:
                    raise ValueError(f"layer {i}: {name} is {tuple(t.shape)}, expected {shape}")
        self.mc = mc
        self.max_rows = max_rows
        self._layers = layers  # keeps the weights referenced by the native stack alive
        arr = (_Layer * len(layers))(*[
            _Layer(lw["wqkv"].data_ptr(), lw["wo"].data_ptr(), lw["wug"].data_ptr(), lw["wd"].data_ptr(),
                   lw["n_in"].data_ptr(), lw["n_post"].data_ptr(), ptr(lw.get("q_norm")), ptr(lw.get("k_norm")))
            for lw in layers])
        handle = c_void_p()
        _lib.call("nsd_decoder_create", mc.num_layers, H, I, hq, hkv, d, float(mc.rms_norm_eps),
                  ctypes.addressof(arr), max_rows, ctypes.byref(handle))
        self._handle = handle

    def close(self) -> None:
        h, self._handle = getattr(self, "_handle", None), None
        if h is not None and h.value:
            _lib.call("nsd_decoder_destroy", h)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, x: torch.Tensor, residual: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                block_table: torch.Tensor, engine_config, infer_state, cos_cache: torch.Tensor,
                sin_cache: torch.Tensor, probe_layer: int = -1):
        """Runs every layer for the forward's decode/verify rows on the
        current stream.  ``x`` [rows, hidden]: the embeddings, replaced by
        the last layer's output (add ``residual`` for the final hidden
        state, model.py:292); ``residual`` must be zero on entry.  With
        ``probe_layer`` >= 0 returns that layer's attention (q, o, lse), else
        None."""
        mc = self.mc
        if self._handle is None:
            raise RuntimeError("the decoder stack was closed")
        require_cuda(x, residual, k_cache, v_cache, block_table, cos_cache, sin_cache)
        require(x, torch.float16, "x")
        require(residual, torch.float16, "residual")
        require(k_cache, torch.float16, "k_cache")
        require(v_cache, torch.float16, "v_cache")
        check_block_table(block_table, engine_config)
        rows = int(infer_state.num_decoding_seqs)
        if infer_state.num_prefill_seqs:
            raise ValueError("the decoder stack serves forwards of decode/verify rows only")
        if rows < 1 or rows > self.max_rows:
            raise ValueError(f"{rows} rows: the decoder stack serves 1..{self.max_rows}")
        if tuple(x.shape) != (rows, mc.hidden_size) or residual.shape != x.shape:
            raise ValueError(f"x and residual must be [{rows}, {mc.hidden_size}]")
        n_blocks, n_layers, hkv, bs, d = cache_dims(k_cache)
        if v_cache.shape != k_cache.shape or n_layers != mc.num_layers or hkv != mc.num_kv_heads or bs != 16:
            raise ValueError("KV caches do not match the model ([blocks, layers, kv heads, 16, head_dim])")
        if cos_cache.dim() != 2 or cos_cache.shape[1] != d // 2 or sin_cache.shape != cos_cache.shape:
            raise ValueError("cos/sin caches must be [max_positions, head_dim/2]")
        if getattr(infer_state, "ignore_kvcache", False):
            raise ValueError("infer_state.ignore_kvcache is set but the forward has decode rows")
        plan = plan_for(infer_state, mc, engine_config, block_table)
        if plan.n_rows != rows:
            raise ValueError(f"the forward's attention plan covers {plan.n_rows} rows, not {rows}")
        probe = None
        if probe_layer >= 0:
            probe = (torch.empty((rows, mc.num_q_heads, d), dtype=torch.float16, device=x.device),
                     torch.empty((rows, mc.num_q_heads, d), dtype=torch.float16, device=x.device),
                     torch.empty((rows, mc.num_q_heads), dtype=torch.float32, device=x.device))
        _lib.call("nsd_decoder_forward", self._handle, x.data_ptr(), residual.data_ptr(), rows,
                  k_cache.data_ptr(), v_cache.data_ptr(), n_blocks, block_table.data_ptr(), block_table.shape[0],
                  block_table.shape[1], infer_state.seq_ids.data_ptr(), infer_state.decoding_seq_lens.data_ptr(),
                  cos_cache.data_ptr(), sin_cache.data_ptr(), cos_cache.shape[0], plan.host_ptr(),
                  plan.dev.data_ptr(), plan.workspace.data_ptr(), plan.workspace.numel(),
                  float(infer_state.softmax_scale), int(probe_layer),
                  *(t.data_ptr() for t in probe) if probe else (None, None, None), None, stream_of(x))
        return probe
