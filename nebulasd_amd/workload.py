"""Seeded synthetic workloads of the attention path.

Each spec describes one layer call of decode or verify attention on the
reference's cache layout: per-request contexts drawn from a seeded
distribution, a block table made of consecutive ids of a seeded permutation
of the pool, and fp16 Q/K/V drawn from N(0, scale^2).  The same seed gives
the same contexts, block tables and tensors on every machine.
"""

from __future__ import annotations

import itertools
import math
from dataclasses import dataclass, field

import torch

from .config import QWEN3_0_6B, QWEN3_8B
from .speculative import expand_verify_rows


@dataclass(frozen=True)
class WorkloadSpec:
    name: str
    model: dict
    batch: int
    q_len: int                  # rows per request (proposal depth + 1; 1 for decode)
    ctx: tuple                  # ("uniform", lo, hi) or ("loguniform", lo, hi)
    pool_blocks: int
    scale: float = 1.0          # std of Q/K/V
    force_max_ctx: bool = False # make one request use the upper context bound
    block_size: int = 16

    @property
    def num_q_heads(self) -> int:
        return self.model["num_attention_heads"]

    @property
    def num_kv_heads(self) -> int:
        return self.model["num_key_value_heads"]

    @property
    def num_layers(self) -> int:
        return self.model["num_hidden_layers"]

    @property
    def head_dim(self) -> int:
        return self.model["head_dim"]

    def bt_stride(self, ctxs=None) -> int:
        """Block-table row length: enough blocks for the largest possible context."""
        hi = self.ctx[2] if ctxs is None else max(max(ctxs), self.ctx[2])
        return math.ceil((hi + self.q_len) / self.block_size)


SPECS = {
    # One layer of Qwen3-0.6B-shape decode, small enough for the CPU oracle.
    "cpu_plumbing": WorkloadSpec("cpu_plumbing", QWEN3_0_6B, 4, 1, ("uniform", 64, 256), 256,
                                 scale=128 ** -0.5),
    # Draft decode: Qwen3-0.6B shape, B=64, contexts U[512, 2048].
    "draft_decode": WorkloadSpec("draft_decode", QWEN3_0_6B, 64, 1, ("uniform", 512, 2048), 24576),
    # Target verify: Qwen3-8B shape, B=16, q_len=5, contexts U[256, 4096].
    "target_verify": WorkloadSpec("target_verify", QWEN3_8B, 16, 5, ("uniform", 256, 4096), 24576),
    # Ragged long-context verify: q_len=9, contexts log-U[1024, 32768], one 32k request.
    "ragged_verify": WorkloadSpec("ragged_verify", QWEN3_8B, 16, 9, ("loguniform", 1024, 32768),
                                  24576, force_max_ctx=True),
}


@dataclass
class Workload:
    spec: WorkloadSpec
    seed: int
    ctxs: list                   # per request: tokens already in the cache
    seq_ids: list                # per row
    seq_lens: list               # per row
    block_table: torch.Tensor    # [batch, bt_stride] int32 (device)
    q: torch.Tensor              # [rows, Hq, d] fp16
    k_cache: torch.Tensor        # [pool, L, Hkv, 16, d] fp16
    v_cache: torch.Tensor
    extra: dict = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return len(self.seq_lens)

    def kv_tokens(self) -> int:
        """Unique KV tokens read per layer call (each request's last seq_len)."""
        return sum(c + self.spec.q_len for c in self.ctxs)

    def algorithmic_bytes(self, with_lse: bool = False) -> int:
        """HBM bytes one layer call must move: K+V once per request and kv head,
        Q in, O out, block-table entries (and the LSE if exported)."""
        s = self.spec
        kv = self.kv_tokens() * s.num_kv_heads * s.head_dim * 2 * 2
        qo = 2 * self.rows * s.num_q_heads * s.head_dim * 2
        bt = sum(math.ceil((c + s.q_len) / s.block_size) for c in self.ctxs) * 4
        return kv + qo + bt + (self.rows * s.num_q_heads * 4 if with_lse else 0)

    def prologue_bytes(self) -> int:
        """HBM bytes of the fused prologue: q/k/v read, q/k written back in
        place, k/v written to their cache slots, plus the per-row metadata,
        block-table entry and RoPE table rows (gamma vectors are negligible)."""
        s = self.spec
        d2 = s.head_dim * 2
        qkv = self.rows * (s.num_q_heads + 2 * s.num_kv_heads) * d2
        back = self.rows * (s.num_q_heads + s.num_kv_heads) * d2
        store = self.rows * 2 * s.num_kv_heads * d2
        meta = self.rows * (4 + 4 + 4 + 2 * s.head_dim)  # seq_id, seq_len, block id, cos+sin rows
        return qkv + back + store + meta

    def flops(self) -> int:
        """2 flops per multiply-add of QK^T and PV over the attended tokens."""
        s = self.spec
        g = s.num_q_heads
        return sum(4 * g * s.head_dim * sl for sl in self.seq_lens)


def draw_contexts(spec: WorkloadSpec, gen: torch.Generator) -> list:
    kind, lo, hi = spec.ctx
    if kind == "uniform":
        ctxs = torch.randint(lo, hi + 1, (spec.batch,), generator=gen).tolist()
    elif kind == "loguniform":
        u = torch.rand(spec.batch, generator=gen, dtype=torch.float64)
        ctxs = [int(round(math.exp(math.log(lo) + float(x) * (math.log(hi) - math.log(lo))))) for x in u]
    else:
        raise ValueError(kind)
    if spec.force_max_ctx:
        ctxs[int(torch.randint(0, spec.batch, (1,), generator=gen))] = hi
    return ctxs


def make_block_table(spec: WorkloadSpec, ctxs: list, gen: torch.Generator):
    """Request r takes the next ceil((ctx_r + q_len)/16) ids of a seeded pool
    permutation; unused entries point at a pool block no request owns."""
    perm = torch.randperm(spec.pool_blocks, generator=gen).to(torch.int32)
    need = [math.ceil((c + spec.q_len) / spec.block_size) for c in ctxs]
    if sum(need) >= spec.pool_blocks:
        raise ValueError(f"pool of {spec.pool_blocks} blocks too small for {sum(need)}")
    poison = int(perm[-1])
    bt = torch.full((len(ctxs), spec.bt_stride(ctxs)), poison, dtype=torch.int32)
    at = 0
    for r, n in enumerate(need):
        bt[r, :n] = perm[at:at + n]
        at += n
    return bt, poison


def make_workload(spec: WorkloadSpec | str, seed: int = 0, device="cuda",
                  pool_blocks: int | None = None, num_layers: int | None = None,
                  ctxs: list | None = None, q_len: int | None = None,
                  model: dict | None = None) -> Workload:
    """Build one seeded workload on ``device``.

    ``pool_blocks`` / ``num_layers`` shrink the cache for quick tests (the
    defaults are the spec's full pool and the model's layer count);
    ``ctxs`` / ``q_len`` / ``model`` replace the drawn contexts, the rows
    per request and the model shape.
    """
    if isinstance(spec, str):
        spec = SPECS[spec]
    if any(x is not None for x in (pool_blocks, num_layers, q_len, model)) or ctxs is not None:
        m = dict(model or spec.model)
        if num_layers is not None:
            m["num_hidden_layers"] = num_layers
        spec = WorkloadSpec(spec.name, m, len(ctxs) if ctxs is not None else spec.batch,
                            q_len or spec.q_len, spec.ctx, pool_blocks or spec.pool_blocks,
                            spec.scale, spec.force_max_ctx and ctxs is None, spec.block_size)
    gen = torch.Generator().manual_seed(seed)
    drawn = draw_contexts(spec, gen)
    ctxs = list(ctxs) if ctxs is not None else drawn
    bt, poison = make_block_table(spec, ctxs, gen)
    reqs = [(r, c, 0, [0] * (spec.q_len - 1)) for r, c in enumerate(ctxs)]
    _, seq_ids, seq_lens = expand_verify_rows(reqs)
    dev = torch.device(device)
    dgen = torch.Generator(device=dev).manual_seed(seed + 1000)
    shape = (spec.pool_blocks, spec.num_layers, spec.num_kv_heads, spec.block_size, spec.head_dim)
    k_cache = torch.empty(shape, dtype=torch.float16, device=dev)
    v_cache = torch.empty(shape, dtype=torch.float16, device=dev)
    for cache in (k_cache, v_cache):
        for chunk in cache.split(max(1, 2048 * 28 // spec.num_layers)):  # bounded temporaries
            chunk.normal_(0.0, spec.scale, generator=dgen)
    q = torch.empty((len(seq_lens), spec.num_q_heads, spec.head_dim), dtype=torch.float16, device=dev)
    q.normal_(0.0, spec.scale, generator=dgen)
    return Workload(spec, seed, ctxs, seq_ids, seq_lens, bt.to(dev), q, k_cache, v_cache,
                    extra={"poison_block": poison})


# --------------------------------------------------------------------------
# Prefill (prompt) attention workloads
# --------------------------------------------------------------------------

@dataclass(frozen=True)
class PrefillSpec:
    name: str
    model: dict
    batch: int
    lens: tuple                 # ("uniform", lo, hi): prompt lengths
    scale: float = 1.0          # std of Q/K/V

    @property
    def num_q_heads(self) -> int:
        return self.model["num_attention_heads"]

    @property
    def num_kv_heads(self) -> int:
        return self.model["num_key_value_heads"]

    @property
    def num_layers(self) -> int:
        return self.model["num_hidden_layers"]

    @property
    def head_dim(self) -> int:
        return self.model.get("head_dim", self.model["hidden_size"] // self.num_q_heads)


PREFILL_SPECS = {
    # One prefill chunk of the speculative loop: 16 prompts of U[128, 1024] tokens.
    "prefill_target": PrefillSpec("prefill_target", QWEN3_8B, 16, ("uniform", 128, 1024)),
    "prefill_draft": PrefillSpec("prefill_draft", QWEN3_0_6B, 16, ("uniform", 128, 1024)),
}


@dataclass
class PrefillWorkload:
    spec: PrefillSpec
    seed: int
    lens: list                   # prompt lengths
    cu_seqlens: torch.Tensor     # [batch + 1] int32 (device)
    q: torch.Tensor              # [tokens, Hq, d] fp16
    k: torch.Tensor              # [tokens, Hkv, d] fp16
    v: torch.Tensor

    @property
    def tokens(self) -> int:
        return sum(self.lens)

    def flops(self) -> int:
        """2 flops per multiply-add of QK^T and PV over the causal triangle."""
        s = self.spec
        return sum(4 * s.num_q_heads * s.head_dim * n * (n + 1) // 2 for n in self.lens)

    def algorithmic_bytes(self) -> int:
        """q, k, v read once and o written once."""
        s = self.spec
        return self.tokens * (2 * s.num_q_heads + 2 * s.num_kv_heads) * s.head_dim * 2


def make_prefill_workload(spec: PrefillSpec | str, seed: int = 0, device="cuda",
                          lens: list | None = None, model: dict | None = None) -> PrefillWorkload:
    """Seeded prompts of ``spec`` (or the given ``lens`` / ``model`` shape) on ``device``."""
    if isinstance(spec, str):
        spec = PREFILL_SPECS[spec]
    if model is not None or lens is not None:
        spec = PrefillSpec(spec.name, model or spec.model, len(lens) if lens is not None else spec.batch,
                           spec.lens, spec.scale)
    gen = torch.Generator().manual_seed(seed)
    if lens is None:
        _, lo, hi = spec.lens
        lens = torch.randint(lo, hi + 1, (spec.batch,), generator=gen).tolist()
    lens = [int(n) for n in lens]
    dev = torch.device(device)
    cu = torch.tensor([0] + list(itertools.accumulate(lens)), dtype=torch.int32, device=dev)
    t = sum(lens)
    dgen = torch.Generator(device=dev).manual_seed(seed + 2000)
    q = torch.empty((t, spec.num_q_heads, spec.head_dim), dtype=torch.float16, device=dev)
    k = torch.empty((t, spec.num_kv_heads, spec.head_dim), dtype=torch.float16, device=dev)
    v = torch.empty_like(k)
    for x in (q, k, v):
        x.normal_(0.0, spec.scale, generator=dgen)
    return PrefillWorkload(spec, seed, lens, cu, q, k, v)
