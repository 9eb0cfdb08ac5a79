"""Single-GPU speculative decoding loop on random-init Qwen3 models.

This drives the attention path the way NebulaSD's swiftLLM backend does, at
real model shapes, so that every layer call of a speculative run goes through
this package's gfx950 kernels:

* decode / verify rows: QK-RMSNorm + RoPE + KV store and paged attention in
  one launch (``paged_attention_fused``), or, on a sampled-check layer or
  with the forward-phase ranges on, the prologue in one launch
  (``qk_norm_rope_store``) then paged attention, in the order of
  swiftLLM/swiftllm/worker/layers/transformer_layer.py:105-185;
* prefill: ``rmsnorm_inplace`` on q/k, ``rotary_embedding_inplace``, the
  prefill ``store_kvcache`` and the prompts' causal attention in one launch
  (``flash_attn_varlen_func``, the entry point of transformer_layer.py:7-32
  and :151-164);
* the rest of the layer in the reference's order
  (transformer_layer.py:83-201, model.py:266-301): the residual buffer with
  ``fused_add_rmsnorm_inplace`` before attention and before the FFN, the
  stacked up/gate projection and SiLU-and-mul in one pass over the weight
  (``up_gate_silu_and_mul``) for decode and verify batches (the library GEMM
  and ``silu_and_mul_inplace`` for prompts), one fused q/k/v GEMM (the
  reference runs three) whose row slices the prologue reads, and the
  post-layer's last-token norm with the fused lm_head + argmax
  (``post_layer_forward``); the other GEMMs are library GEMMs through
  ``F.linear`` as in the reference (kernels/linear.py:3-12).  Weights are
  random (no checkpoints are available offline).

The loop is NebulaSD's linear speculation: the draft proposes ``depth``
tokens with single-token decode steps (nebulasd workers/draft/backend.py:52-70);
the target verifies anchor + proposal as q_len = depth+1 rows
(workers/target/backend.py:101-127, swiftLLM/swiftllm/speculative.py:75-89);
greedy acceptance (speculative.py:122-156) appends the accepted proposal and
the target's bonus token.  When a whole proposal is accepted the draft has not
seen its last token; its next step then runs that token and the new anchor as
one two-row group (the reconcile of workers/draft/inputs.py:59-85).

Every ``check_every``-th forward of either model hands one mid-depth attention
layer call (q, o, LSE, rows) to the caller's ``make_check`` callback; the tests
compare those calls with the numpy oracle (tests/spec_checks.py,
tests/run_spec_loop.py for the full 512-request configuration).
"""

from __future__ import annotations

import argparse
import contextlib
import json
import math
import time

import numpy as np
import torch
import torch.nn.functional as F

from .config import QWEN3_0_6B, QWEN3_8B, EngineConfig, ModelConfig
from .infer_state import build_infer_state, host_to_device, model_rope_cache
from .kernels import (FUSED_UP_GATE_MAX_ROWS, flash_attn_varlen_func, fused_add_rmsnorm_inplace, paged_attention,
                      paged_attention_fused, post_layer_forward, qk_norm_rope_store, rmsnorm_inplace,
                      rotary_embedding_inplace, silu_and_mul_inplace, store_kvcache, up_gate_silu_and_mul)
from .decoder import MAX_ROWS as DECODER_MAX_ROWS
from .decoder import DecoderStack
from .phases import ENABLED as PHASE_RANGES
from .plan import plan_for
from .phases import forward_phase_range
from .speculative import compute_greedy_acceptance


class RandomQwen3:
    """A random-init Qwen3 decoder with a paged KV cache of its own.

    ``native``: decode/verify forwards of up to 128 rows run their layers in
    one call of the native decoder stack (``DecoderStack``), the same kernels
    and GEMMs enqueued from C++; otherwise (and always for prompts, or with
    the forward-phase ranges on) the layers run from Python as below."""

    def __init__(self, cfg: dict, seq_blocks: list, device, seed: int, std: float = 0.02, native: bool = True):
        self.mc = mc = ModelConfig(cfg)
        self.dev = dev = torch.device(device)
        g = torch.Generator(device=dev).manual_seed(seed)
        H, I, V = mc.hidden_size, mc.ffn_inter_dim, mc.vocab_size
        hq, hkv, d = mc.num_q_heads, mc.num_kv_heads, mc.head_dim

        def w(*shape, scale=std):
            return (torch.randn(shape, device=dev, generator=g) * scale).half()

        self.embed = w(V, H, scale=1.0)
        self.lm_head = w(V, H)
        self.final_norm = (torch.rand(H, device=dev, generator=g) + 0.5).half()
        self.layers = []
        for _ in range(mc.num_layers):
            self.layers.append(dict(
                wqkv=w((hq + 2 * hkv) * d, H), wo=w(H, hq * d),  # q, k, v projections stacked
                wug=w(2 * I, H), wd=w(H, I),  # up rows first, then gate (weight.py:151)
                n_in=(torch.rand(H, device=dev, generator=g) + 0.5).half(),
                n_post=(torch.rand(H, device=dev, generator=g) + 0.5).half(),
                q_norm=(torch.rand(d, device=dev, generator=g) + 0.5).half(),
                k_norm=(torch.rand(d, device=dev, generator=g) + 0.5).half()))
        # one block-table row per sequence: its blocks drawn from a shuffled pool
        n_blocks = sum(seq_blocks)
        perm = torch.randperm(n_blocks, generator=torch.Generator().manual_seed(seed))
        width = max(seq_blocks)
        bt = torch.zeros((len(seq_blocks), width), dtype=torch.int32)
        pos = 0
        for r, nb in enumerate(seq_blocks):
            bt[r, :nb] = perm[pos:pos + nb].to(torch.int32)
            pos += nb
        self.block_table = bt.to(dev)
        self.ec = EngineConfig(block_size=16, max_blocks_per_seq=width, num_gpu_blocks=n_blocks)
        shape = (n_blocks, mc.num_layers, hkv, 16, d)
        self.k_cache = torch.zeros(shape, dtype=torch.float16, device=dev)
        self.v_cache = torch.zeros(shape, dtype=torch.float16, device=dev)
        self.cos, self.sin = model_rope_cache(mc, width * 16 + 1, dev)
        self.check = None  # (layer, callback) of a sampled attention check
        self.native = native
        self.stacks = {}  # native decoder stacks by lane (one per concurrent stream), built on first use

    def _token_tensor(self, tokens) -> torch.Tensor:
        """Token ids as a device int64 tensor (a device tensor passes through;
        a host list is sent without waiting for the stream)."""
        if isinstance(tokens, torch.Tensor):
            return tokens
        return host_to_device(tokens, torch.long, self.dev)

    def _forward(self, st, token_ids, attention, as_tensor: bool = False):
        """transformer_layer.py:83-201 for every layer, then model.py:292 and
        the post-layer (post_layer.py:49-79); `attention(li, lw, q, k, v)`
        returns o [tokens, Hq, d].  Returns the greedy token of every request
        (every prompt's last token, then every decode row): a list, or with
        ``as_tensor`` the int64 device tensor (no host synchronisation)."""
        mc, dev = self.mc, self.dev
        eps, inter = mc.rms_norm_eps, mc.ffn_inter_dim
        hq, hkv, d = mc.num_q_heads, mc.num_kv_heads, mc.head_dim
        x = self.embed[self._token_tensor(token_ids)]
        res = torch.zeros_like(x)
        for li, lw in enumerate(self.layers):
            fused_add_rmsnorm_inplace(x, res, lw["n_in"], eps)
            with forward_phase_range(f"layer_{li}_qkv"):
                qkv = F.linear(x, lw["wqkv"])  # one GEMM for the reference's three (transformer_layer.py:107-109)
            q = qkv[:, :hq * d].view(-1, hq, d)
            k = qkv[:, hq * d:(hq + hkv) * d].view(-1, hkv, d)
            v = qkv[:, (hq + hkv) * d:].view(-1, hkv, d)
            o = attention(li, lw, q, k, v)
            with forward_phase_range(f"layer_{li}_o_proj"):
                o = F.linear(o.view(x.shape[0], -1), lw["wo"])
            fused_add_rmsnorm_inplace(o, res, lw["n_post"], eps)
            with forward_phase_range(f"layer_{li}_ffn"):
                if o.shape[0] <= FUSED_UP_GATE_MAX_ROWS:  # decode / verify batches: one pass over the weight
                    h = up_gate_silu_and_mul(o, lw["wug"])
                else:
                    up_gate = F.linear(o, lw["wug"])
                    silu_and_mul_inplace(up_gate)
                    h = up_gate[:, :inter]
                x = F.linear(h, lw["wd"])
        x += res
        with forward_phase_range("post_lm_head"):
            out = post_layer_forward(x, st, self.final_norm, self.lm_head, eps)
        return out if as_tensor else out.tolist()

    def prefill(self, seq_ids: list, prompts: list, ignore_kvcache: bool = False) -> list:
        """Run the prompts; returns each one's greedy next token.  With
        ``ignore_kvcache`` the forward leaves the cache untouched
        (transformer_layer.py:133)."""
        mc, dev = self.mc, self.dev
        lens = [len(p) for p in prompts]
        st = build_infer_state(seq_ids, [], lens, mc, self.cos, self.sin, dev,
                               ignore_kvcache=ignore_kvcache)
        d = mc.head_dim

        def attention(li, lw, q, k, v):
            q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
            rmsnorm_inplace(q.view(-1, d), lw["q_norm"], mc.rms_norm_eps)
            rmsnorm_inplace(k.view(-1, d), lw["k_norm"], mc.rms_norm_eps)
            rotary_embedding_inplace(q, k, st)
            if not st.ignore_kvcache:
                with forward_phase_range(f"layer_{li}_store_kvcache"):
                    store_kvcache(k, v, self.k_cache, self.v_cache, self.block_table, mc, self.ec, st, li)
            return flash_attn_varlen_func(q, k, v, st.prefill_seq_start_locs_with_end,
                                          st.prefill_seq_start_locs_with_end, st.max_prefill_len,
                                          st.max_prefill_len, softmax_scale=st.softmax_scale)
        return self._forward(st, [t for p in prompts for t in p], attention)

    def decode(self, seq_ids: list, seq_lens: list, tokens, as_tensor: bool = False, lane: int = 0):
        """Decode / verify rows (rows of one sequence contiguous, seq_lens
        rising by one); returns the greedy next token of every row.  `tokens`
        is a host list or an int64 device tensor; with ``as_tensor`` the result
        stays on the device (no host synchronisation).  Forwards that may run
        at the same time (other streams) take different ``lane`` numbers: each
        lane has its own native stack buffers (the weights are shared)."""
        mc, dev = self.mc, self.dev
        st = build_infer_state(seq_ids, seq_lens, [], mc, self.cos, self.sin, dev)
        if self.native and len(tokens) <= DECODER_MAX_ROWS and not PHASE_RANGES:
            return self._decode_native(st, seq_ids, seq_lens, tokens, as_tensor, lane)
        hq = mc.num_q_heads

        def attention(li, lw, q_rows, k, v):
            checked = self.check is not None and self.check[0] == li
            if not checked and not PHASE_RANGES and plan_for(st, mc, self.ec, self.block_table).keeps_sequences_whole:
                # the prologue inside the attention's launch: the two calls' results, one launch
                o = torch.empty(q_rows.shape, dtype=q_rows.dtype, device=dev)
                paged_attention_fused(q_rows, k, v, self.k_cache, self.v_cache, self.block_table, lw["q_norm"],
                                      lw["k_norm"], mc, self.ec, st, li, self.cos, self.sin, o)
                return o
            q = torch.empty(q_rows.shape, dtype=q_rows.dtype, device=dev)  # the prologue's contiguous q
            with forward_phase_range(f"layer_{li}_store_kvcache"):  # QK-norm + RoPE + store, one launch
                qk_norm_rope_store(q_rows, k, v, self.k_cache, self.v_cache, self.block_table,
                                   lw["q_norm"], lw["k_norm"], mc, self.ec, st, li, self.cos, self.sin,
                                   q_out=q)
            o = torch.empty_like(q)
            if self.check is not None and self.check[0] == li:
                lse = torch.empty((q.shape[0], hq), dtype=torch.float32, device=dev)
                paged_attention(q, self.k_cache, self.v_cache, self.block_table, mc, self.ec, st,
                                li, o, lse)
                self.check[1](self, li, q, o, lse, seq_ids, seq_lens)
                self.check = None
            else:
                with forward_phase_range(f"layer_{li}_paged_attention"):
                    paged_attention(q, self.k_cache, self.v_cache, self.block_table, mc, self.ec, st,
                                    li, o)
            return o
        return self._forward(st, tokens, attention, as_tensor)

    def _decode_native(self, st, seq_ids: list, seq_lens: list, tokens, as_tensor: bool = False, lane: int = 0):
        """decode() with every layer in one call of the native decoder stack;
        a sampled attention check receives its layer's q, o and LSE after
        the forward (later layers write only their own cache slots)."""
        mc, dev = self.mc, self.dev
        stack = self.stacks.get(lane)
        if stack is None:
            stack = self.stacks[lane] = DecoderStack(mc, self.layers)
        x = self.embed[self._token_tensor(tokens)]
        res = torch.zeros_like(x)
        probe_layer = self.check[0] if self.check is not None else -1
        probe = stack.forward(x, res, self.k_cache, self.v_cache, self.block_table, self.ec, st, self.cos,
                                   self.sin, probe_layer)
        if probe is not None:
            q, o, lse = probe
            self.check[1](self, probe_layer, q, o, lse, seq_ids, seq_lens)
            self.check = None
        x += res
        with forward_phase_range("post_lm_head"):
            out = post_layer_forward(x, st, self.final_norm, self.lm_head, mc.rms_norm_eps)
        return out if as_tensor else out.tolist()


def _sync(dev: torch.device) -> None:
    if dev.type == "cuda":
        torch.cuda.synchronize(dev)


def run(n_requests=512, prompt_lo=128, prompt_hi=1024, new_tokens=128, draft_batch=64,
        target_batch=16, depth=4, seed=0, check_every=0, make_check=None, device="cuda:0",
        draft_cfg=QWEN3_0_6B, target_cfg=QWEN3_8B, share_weights=False, return_outputs=False,
        log=None, native=True, sync_each_forward=False, overlap=True, target_streams=2) -> dict:
    """The speculative loop over `n_requests` synthetic requests; returns a summary.

    With ``check_every`` > 0, every check_every-th forward calls
    ``make_check()(model, layer, q, o, lse, seq_ids, seq_lens)`` for its
    mid-depth attention layer call.  ``share_weights`` builds the draft with
    the target's configuration and seed, so that it holds the same weights
    and its greedy proposals are accepted except where the two forwards'
    rounding splits a near-tie: this exercises multi-token acceptance and
    the draft's two-row reconcile step, which independent random models
    (acceptance 0) never reach.  ``return_outputs`` adds every request's
    generated tokens to the summary (key ``outputs``).

    A draft group's forwards are enqueued back to back: the draft's
    proposals stay on the device (each step's tokens are the next step's
    input), the target batches read them there, and the host reads the
    proposals and the target's tokens back once per draft group, so it
    builds the next forward's metadata while the GPU runs the previous one.
    ``sync_each_forward`` waits for every forward instead (same results:
    the kernels are deterministic; for tests and timing comparisons).

    ``overlap`` (on a GPU, without ``sync_each_forward``) runs the draft's
    forwards on one stream and the target's on another, the target's waiting
    for its group's proposals by an event, and reads a group's results back
    after the next group is enqueued: the next group's draft forwards then
    run beside this group's verifies.  A group's target batches alternate
    over ``target_streams`` streams (each with its own decoder-stack lane),
    so verifies of different batches run side by side too.  Results are the
    same either way.
    """
    dev = torch.device(device)
    rng = np.random.default_rng(seed)
    vocab = target_cfg["vocab_size"]
    plens = rng.integers(prompt_lo, prompt_hi + 1, n_requests).tolist()
    prompts = [rng.integers(0, vocab, n).tolist() for n in plens]
    # room for the prompt, the output and one proposal beyond it
    blocks = [math.ceil((p + new_tokens + depth + 2) / 16) for p in plens]
    target = RandomQwen3(target_cfg, blocks, dev, seed + 1, native=native)
    if share_weights:
        draft = RandomQwen3(target_cfg, blocks, dev, seed + 1, native=native)
    else:
        draft = RandomQwen3(draft_cfg, blocks, dev, seed + 2, native=native)
    n_checks = 0
    t0 = time.perf_counter()

    out = [[] for _ in range(n_requests)]
    chunk = 16
    for s in range(0, n_requests, chunk):
        ids = list(range(s, min(n_requests, s + chunk)))
        first = target.prefill(ids, [prompts[r] for r in ids])
        draft.prefill(ids, [prompts[r] for r in ids])
        for r, t in zip(ids, first):
            out[r].append(t)
        if log and (s // chunk) % 8 == 7:
            log(f"prefill: {ids[-1] + 1} of {n_requests} requests")
    _sync(dev)
    t_prefill = time.perf_counter() - t0
    # tokens of the output each cache holds: the target all but the anchor;
    # the draft the same, or one fewer after a fully accepted proposal
    draft_missing = [None] * n_requests  # accepted proposal token the draft has not run
    stats = {"target_forwards": 0, "draft_forwards": 0, "rounds": 0, "proposed": 0,
             "accepted": 0, "reconcile_groups": 0, "full_accepts": 0, "partial_accepts": 0,
             "multi_token_appends": 0}
    step = 0
    # draft forwards on one stream, target verifies on `target_streams` more:
    # a draft group's forwards run beside the previous group's verifies
    # (other requests, the other model), as the reference's draft and target
    # workers run side by side (streams at the default priority)
    overlap = overlap and not sync_each_forward and dev.type == "cuda"
    d_stream = torch.cuda.Stream(device=dev) if overlap else None
    t_streams = [torch.cuda.Stream(device=dev) for _ in range(max(1, target_streams))] if overlap else [None]

    def on(stream):
        return torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()

    def to_host(t: torch.Tensor) -> torch.Tensor:
        """Copy of `t` in pinned host memory, enqueued on the current stream."""
        if t.device.type != "cuda":
            return t
        h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
        h.copy_(t, non_blocking=True)
        return h

    def enqueue_group(dgroup: list):
        """The group's draft proposals and target verifies, enqueued; returns
        what finish_group reads back."""
        nonlocal step, n_checks
        with on(d_stream):
            # draft: `depth` proposals per request, kept on the device; step
            # j's tokens in request order ([len(dgroup)] int64)
            steps_dev = []
            for j in range(depth):
                sids, slens, toks, last_row = [], [], [], []
                for r in dgroup:
                    base = plens[r] + len(out[r]) - 1 + j  # tokens before this step's input
                    if j == 0 and draft_missing[r] is not None:
                        stats["reconcile_groups"] += 1
                        sids += [r, r]
                        slens += [base, base + 1]
                        toks += [draft_missing[r], out[r][-1]]
                    else:
                        sids.append(r)
                        slens.append(base + 1)
                        if j == 0:
                            toks.append(out[r][-1])
                    last_row.append(len(sids) - 1)
                if j > 0:  # one row per request: the previous step's proposals
                    toks = steps_dev[-1]
                if check_every and make_check and step % check_every == 0:
                    draft.check = (draft.mc.num_layers // 2, make_check())
                    n_checks += 1
                step += 1
                nxt = draft.decode(sids, slens, toks, as_tensor=True)
                stats["draft_forwards"] += 1
                if sync_each_forward:
                    _sync(dev)
                steps_dev.append(nxt if len(sids) == len(dgroup)
                                 else nxt[host_to_device(last_row, torch.long, dev)])
            for r in dgroup:
                draft_missing[r] = None
            # target rows per request: [anchor, proposals...]
            anchors = host_to_device([out[r][-1] for r in dgroup], torch.long, dev)
            props_dev = torch.stack(steps_dev, 1)
            rows_dev = torch.cat([anchors[:, None], props_dev], 1)
            drafted = torch.cuda.Event() if overlap else None
            if overlap:
                drafted.record(d_stream)
        if overlap:
            for ts_ in t_streams:
                ts_.wait_event(drafted)
                # made on the draft stream, read on the target streams
                props_dev.record_stream(ts_)
                rows_dev.record_stream(ts_)
        posts_h = []
        for b, ts in enumerate(range(0, len(dgroup), target_batch)):
            lane = b % len(t_streams)
            with on(t_streams[lane]):
                tgroup = dgroup[ts:ts + target_batch]
                sids, slens = [], []
                for r in tgroup:
                    base = plens[r] + len(out[r]) - 1
                    sids += [r] * (depth + 1)
                    slens += list(range(base + 1, base + 2 + depth))
                if check_every and make_check and step % check_every == 0:
                    target.check = (target.mc.num_layers // 2, make_check())
                    n_checks += 1
                step += 1
                post = target.decode(sids, slens, rows_dev[ts:ts + len(tgroup)].reshape(-1), as_tensor=True,
                                     lane=lane)
                stats["target_forwards"] += 1
                if sync_each_forward:
                    _sync(dev)
                # one read-back per draft group: the proposals, then each batch's tokens
                posts_h.append((tgroup, to_host(post)))
        with on(t_streams[0]):
            props_h = to_host(props_dev)
        done = []
        if dev.type == "cuda":
            for ts_ in t_streams:
                ev = torch.cuda.Event()
                ev.record(ts_ if ts_ is not None else torch.cuda.current_stream(dev))
                done.append(ev)
        return dgroup, props_h, posts_h, done

    def finish_group(pending) -> None:
        """Greedy acceptance of a group whose verifies were enqueued."""
        dgroup, props_h, posts_h, done = pending
        for ev in done:
            ev.synchronize()
        props_host = props_h.tolist()
        props = {r: props_host[i] for i, r in enumerate(dgroup)}
        for tgroup, post_h in posts_h:
            post = post_h.tolist()
            for i, r in enumerate(tgroup):
                p = post[i * (depth + 1):(i + 1) * (depth + 1)]
                acc, n_acc = compute_greedy_acceptance(props[r], p, new_tokens - len(out[r]))
                stats["proposed"] += depth
                stats["accepted"] += n_acc
                stats["full_accepts"] += n_acc == depth
                # a proposal token rejected after at least one accepted (not a
                # proposal cut short by the output limit: len(acc) == n_acc then)
                stats["partial_accepts"] += 0 < n_acc < depth and len(acc) == n_acc + 1
                stats["multi_token_appends"] += len(acc) > 1
                if n_acc == depth and len(acc) == depth + 1:
                    draft_missing[r] = props[r][-1]
                out[r] += acc

    early = None  # the next round's first group, enqueued before this round's last read-back
    while True:
        live = [r for r in range(n_requests) if len(out[r]) < new_tokens]
        if not live:
            break
        stats["rounds"] += 1
        groups = [live[ds:ds + draft_batch] for ds in range(0, len(live), draft_batch)]
        # group g's acceptance is read back after group g + 1 is enqueued
        pending = None
        for gi, dgroup in enumerate(groups):
            if gi == 0 and early is not None:
                if early[0] != dgroup:
                    raise RuntimeError("the round's first draft group changed after it was enqueued")
                nxt_pending, early = early, None
            else:
                nxt_pending = enqueue_group(dgroup)
            if pending is not None:
                finish_group(pending)
            pending = nxt_pending
        # The first group's requests are the lowest live ones: if none of
        # them has finished they open the next round too, and their results
        # are in, so their next proposals go out before the last group's
        # read-back (other requests: the same work in the same order).
        if len(groups) > 1 and all(len(out[r]) < new_tokens for r in groups[0]):
            early = enqueue_group(groups[0])
        finish_group(pending)
        if log:
            log(f"round {stats['rounds']}: {sum(min(len(o), new_tokens) for o in out)} tokens")
    _sync(dev)
    wall = time.perf_counter() - t0
    generated = sum(len(o) for o in out)
    extra = {"outputs": out} if return_outputs else {}
    return {
        "requests": n_requests, "new_tokens": new_tokens, "generated_tokens": generated,
        "prompt_tokens": int(sum(plens)), "wall_s": wall, "prefill_s": t_prefill,
        "decode_tokens_per_s": (generated - n_requests) / max(wall - t_prefill, 1e-9),
        "acceptance_rate": stats["accepted"] / max(stats["proposed"], 1), **stats,
        "attention_checks": n_checks, **extra,
    }


def main():
    p = argparse.ArgumentParser(description="Speculative loop on random-init Qwen3-0.6B / Qwen3-8B")
    p.add_argument("--requests", type=int, default=512)
    p.add_argument("--prompt-lo", type=int, default=128)
    p.add_argument("--prompt-hi", type=int, default=1024)
    p.add_argument("--new-tokens", type=int, default=128)
    p.add_argument("--draft-batch", type=int, default=64)
    p.add_argument("--target-batch", type=int, default=16)
    p.add_argument("--depth", type=int, default=4)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--share-weights", action="store_true",
                   help="draft = the target's model and weights (proposals accepted)")
    p.add_argument("--python-layers", action="store_true",
                   help="run decode/verify layers from Python instead of the native decoder stack")
    p.add_argument("--no-overlap", action="store_true",
                   help="draft and target forwards on one stream (no draft/verify overlap)")
    p.add_argument("--target-streams", type=int, default=2,
                   help="streams a draft group's target batches alternate over")
    a = p.parse_args()
    res = run(a.requests, a.prompt_lo, a.prompt_hi, a.new_tokens, a.draft_batch, a.target_batch,
              a.depth, a.seed, share_weights=a.share_weights, log=lambda m: print(m, flush=True),
              native=not a.python_layers, overlap=not a.no_overlap,
              target_streams=a.target_streams)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
