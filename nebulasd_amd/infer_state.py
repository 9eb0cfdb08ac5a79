"""Per-forward metadata of the attention path.

``LlamaInferState`` keeps the fields of swiftLLM's dataclass
(swiftLLM/swiftllm/worker/infer_state.py:4-29) and adds the host copies of
the decode rows (which swiftLLM's ``model.forward`` already holds as
Python lists, model.py:304-341) plus the lazily built attention plan.
``build_infer_state`` restates the metadata section of
``LlamaModel.forward`` (model.py:325-430).
"""

from __future__ import annotations

import dataclasses
import math

import torch

from .plan import AttnPlan, build_attn_plan


@dataclasses.dataclass
class LlamaInferState:
    batch_size: int
    num_tokens: int

    seq_ids: torch.Tensor            # [batch_size] int32
    softmax_scale: float             # head_dim ** -0.5

    num_prefill_seqs: int
    num_prefill_tokens: int
    prefill_seq_start_locs: torch.Tensor
    prefill_seq_start_locs_with_end: torch.Tensor
    prefill_seq_lens: torch.Tensor
    max_prefill_len: int

    num_decoding_seqs: int
    decoding_seq_lens: torch.Tensor  # [num_decoding_seqs] int32
    max_decoding_len: int

    seq_block_size: int
    num_seq_blocks: int

    position_cos: torch.Tensor       # [num_tokens, head_dim/2] fp16
    position_sin: torch.Tensor

    ignore_kvcache: bool = False

    # host copies of the decode rows (seq_ids[num_prefill_seqs:], decoding_seq_lens)
    seq_ids_list: list | None = None
    decoding_seq_lens_list: list | None = None
    # verify grouping: 0 = pack up to 48 rows per (group, kv head); 1 = row-wise
    max_group_rows: int = 0
    attn_plan: AttnPlan | None = None

    def decode_rows_host(self):
        """(seq_ids, seq_lens) of the decode rows as host lists (one D2H copy if absent)."""
        if self.seq_ids_list is None:
            self.seq_ids_list = self.seq_ids[self.num_prefill_seqs:].cpu().tolist()
        if self.decoding_seq_lens_list is None:
            self.decoding_seq_lens_list = self.decoding_seq_lens.cpu().tolist()
        return self.seq_ids_list, self.decoding_seq_lens_list

    def get_attn_plan(self, model_config, engine_config, block_table: torch.Tensor) -> AttnPlan:
        """The plan of this forward's decode rows (built on first use, reused by all layers)."""
        plan = self.attn_plan
        if plan is None or not plan.fits(model_config.num_q_heads, model_config.num_kv_heads,
                                         block_table):
            sids, slens = self.decode_rows_host()
            plan = build_attn_plan(
                sids, slens, model_config.num_q_heads, model_config.num_kv_heads,
                model_config.head_dim, engine_config.block_size, block_table.shape[0],
                block_table.shape[1], block_table.device, max_group_rows=self.max_group_rows)
            self.attn_plan = plan
        return plan


def reference_seq_block_size(num_kv_heads: int, decoding_seq_lens_list) -> int:
    """swiftLLM's split-size heuristic (model.py:380-384), kept for the metadata fields."""
    sbs = 2048
    total = sum(decoding_seq_lens_list)
    max_len = max(decoding_seq_lens_list) if decoding_seq_lens_list else 0
    while num_kv_heads * (total / sbs) < 1024 and sbs // 2 >= 64 and max_len / (sbs // 2) <= 128:
        sbs //= 2
    return sbs


def host_to_device(values, dtype, device) -> torch.Tensor:
    """A device tensor of host values without synchronising the host: the
    values are copied into pinned memory (torch's caching host allocator
    keeps the block until the copy has run) and sent with a non-blocking
    copy on the current stream.  (``torch.tensor(values, device=cuda)``
    waits for the stream: every kernel enqueued before it must finish.)"""
    dev = torch.device(device)
    t = torch.tensor(values, dtype=dtype)
    if dev.type != "cuda":
        return t.to(dev)
    return t.pin_memory().to(dev, non_blocking=True)


def build_infer_state(seq_ids_list, decoding_seq_lens_list, prefill_lens_list, model_config,
                      cos_cache: torch.Tensor, sin_cache: torch.Tensor, device,
                      max_group_rows: int = 0, ignore_kvcache: bool = False) -> LlamaInferState:
    """Metadata of one forward (swiftLLM/swiftllm/worker/model.py:325-430).

    ``seq_ids_list`` covers prefill sequences first, then decode rows;
    ``prefill_lens_list`` gives the prompt length of each prefill sequence.
    ``ignore_kvcache`` marks a prefill-only forward that must not write the
    cache (transformer_layer.py:133); decode rows cannot use it (:171).
    """
    num_prefill = len(prefill_lens_list)
    if ignore_kvcache and decoding_seq_lens_list:
        raise ValueError("ignore_kvcache needs a forward without decode rows (they attend the cache)")
    if len(seq_ids_list) != num_prefill + len(decoding_seq_lens_list):
        raise ValueError("seq_ids_list must list prefill sequences then decode rows")
    dev = torch.device(device)
    i32 = torch.int32
    num_tokens = sum(prefill_lens_list) + len(decoding_seq_lens_list)
    prefill_lens = host_to_device(prefill_lens_list, i32, dev)
    starts = torch.cumsum(prefill_lens, 0, dtype=torch.int32) - prefill_lens
    dec_lens = host_to_device(decoding_seq_lens_list, i32, dev)
    positions = [p for n in prefill_lens_list for p in range(n)] + [s - 1 for s in decoding_seq_lens_list]
    pos = host_to_device(positions, torch.long, dev)
    max_dec = max(decoding_seq_lens_list) if decoding_seq_lens_list else 0
    sbs = reference_seq_block_size(model_config.num_kv_heads, decoding_seq_lens_list)
    return LlamaInferState(
        batch_size=len(seq_ids_list),
        num_tokens=num_tokens,
        seq_ids=host_to_device(seq_ids_list, i32, dev),
        softmax_scale=model_config.head_dim ** -0.5,
        num_prefill_seqs=num_prefill,
        num_prefill_tokens=num_tokens - len(decoding_seq_lens_list),
        prefill_seq_start_locs=starts,
        prefill_seq_start_locs_with_end=torch.cat([starts, host_to_device([num_tokens], i32, dev)]),
        prefill_seq_lens=prefill_lens,
        max_prefill_len=max(prefill_lens_list) if prefill_lens_list else 0,
        num_decoding_seqs=len(decoding_seq_lens_list),
        decoding_seq_lens=dec_lens,
        max_decoding_len=max_dec,
        seq_block_size=sbs,
        num_seq_blocks=math.ceil(max_dec / sbs) if max_dec else 0,
        position_cos=cos_cache[pos],
        position_sin=sin_cache[pos],
        seq_ids_list=list(seq_ids_list[num_prefill:]),
        decoding_seq_lens_list=list(decoding_seq_lens_list),
        max_group_rows=max_group_rows,
        ignore_kvcache=ignore_kvcache,
    )


def rope_cache(head_dim: int, theta: float, max_positions: int, device, scaling=1.0):
    """fp16 cos/sin caches [max_positions, head_dim/2] (model.py:209-252).

    ``scaling`` is the config's ``rope_scaling``: a number divides every
    position (model.py:242-246); a dict (Llama 3.2 style, model.py:209-240)
    splits the frequencies at ``int(d/2 * lf / (lf + hf))`` and divides the
    positions by ``low_freq_factor`` (lf) below the split and by
    ``high_freq_factor`` (hf) above it.  Positions are the table rows, so
    ``max_positions`` only sets the length.
    """
    dev = torch.device(device)
    f32 = dict(device=dev, dtype=torch.float32)
    t = torch.arange(max_positions, **f32)
    if isinstance(scaling, dict):
        lf = float(scaling.get("low_freq_factor", 1.0))
        hf = float(scaling.get("high_freq_factor", 1.0))
        split = int((head_dim // 2) * lf / (lf + hf))
        inv_low = 1.0 / (theta ** (torch.arange(0, split * 2, 2, **f32) / head_dim))
        inv_high = 1.0 / (theta ** (torch.arange(split * 2, head_dim, 2, **f32) / head_dim))
        freqs = torch.cat([torch.outer(t / lf, inv_low), torch.outer(t / hf, inv_high)], dim=-1)
    else:
        inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, **f32) / head_dim))
        freqs = torch.outer(t / float(scaling), inv_freq)
    return torch.cos(freqs).to(torch.float16), torch.sin(freqs).to(torch.float16)


def model_rope_cache(model_config, max_positions: int, device):
    """The cos/sin caches of ``model_config`` (its rope_theta, head_dim and
    rope_scaling, number or dict), ``max_positions`` rows."""
    return rope_cache(model_config.head_dim, model_config.rope_theta, max_positions, device,
                      getattr(model_config, "rope_scaling", 1.0) or 1.0)