"""numpy restatement of swiftLLM's verify/decode attention path (the oracle).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg; never by the product package.

All reference citations are relative to the reference repository root.
``K = swiftLLM/swiftllm/worker/kernels``.

How each function is pinned (see ``tests/test_oracle.py``):

* ``build_linear_verification_rows``, ``expand_verify_rows``,
  ``aggregate_max_lens_by_seq_id``, ``compute_greedy_acceptance`` -- the
  reference's own literal cases from
  ``swiftLLM/tests/test_speculative_planning.py`` (committed as data in
  ``tests/golden/speculative_cases.json``).
* ``kv_slot_offset`` / ``store_kvcache`` / ``store_kvcache_prefill`` -- the
  closed-form flat offset checked against numpy's own 5-D indexing, and a
  canary pool in which every byte outside the written slots must survive.
* ``rmsnorm`` -- ``torch.nn.functional.rms_norm`` (library routine) and the
  constant-row closed form ``y = sign(c) * w``.
* ``rope_cache`` / ``rope`` -- identity at position 0, norm preservation of
  each (x0, x1) pair, equality with a complex-multiplication formulation,
  ``cos^2 + sin^2 = 1`` and the closed form ``cos(pos)`` for frequency 0;
  for dict ``rope_scaling``, equal factors give the number form, and
  unequal ones split the columns at the stated index, each side equal to
  the number form of its own factor.
* ``paged_attention`` -- ``torch.nn.functional.scaled_dot_product_attention``
  (library routine) on the gathered K/V, a pure-Python brute force on tiny
  inputs, the closed forms seq_len=1 -> v_0, identical keys -> mean(V),
  one dominant logit -> that V, and the grouped-vs-rowwise identity.
* ``paged_attention_two_phase`` -- equality with the unsplit
  ``paged_attention`` for several seq_block_size values (the split-KV
  combine must not depend on the partition).
* ``prefill_attention`` -- ``torch.nn.functional.scaled_dot_product_attention``
  with ``is_causal=True`` per prompt after ``repeat_interleave`` of K/V
  (the reference's own formulation, library routine), a pure-Python brute
  force on tiny inputs, the closed forms position 0 -> v_0 and identical
  keys -> running mean of V, and the identity prompt = verify group with
  ctx 0 and q_len = prompt length under the pinned ``paged_attention``.
"""

from __future__ import annotations

import math

import numpy as np

__all__ = [
    "LOG2E",
    "LN2",
    "build_linear_verification_rows",
    "expand_verify_rows",
    "aggregate_max_lens_by_seq_id",
    "compute_greedy_acceptance",
    "kv_slot_offset",
    "store_kvcache",
    "store_kvcache_prefill",
    "rmsnorm",
    "rope_cache",
    "rope",
    "qk_norm_rope_store",
    "gather_kv",
    "paged_attention",
    "paged_attention_two_phase",
    "reference_seq_block_size",
    "prefill_attention",
]

LOG2E = 1.4426950408889634
LN2 = 0.6931471805599453


# --------------------------------------------------------------------------
# Verify-row definition (host side of the path)
# --------------------------------------------------------------------------

def build_linear_verification_rows(prompt_len: int, output_token_ids, draft_token_ids):
    """Rows of one linear verify request.

    swiftLLM/swiftllm/speculative.py:75-89 -- tokens are ``[anchor] + draft``
    where the anchor is the last (unstored) output token; row i has
    ``seq_len = prompt_len + len(output) + i``.
    """
    if not output_token_ids:
        raise ValueError("linear speculative verification requires an unstored anchor token")
    tokens = [output_token_ids[-1]] + list(draft_token_ids)
    base = prompt_len + len(output_token_ids)
    return tokens, [base + i for i in range(len(tokens))]


def expand_verify_rows(requests):
    """Flatten verify requests into decode rows.

    nebulasd/src/nebulasd/workers/target/backend.py:101-110 -- each request
    ``(seq_id, logical, anchor, proposal)`` becomes ``q_len = 1+len(proposal)``
    rows with identical seq_id and ``seq_len = logical+1 .. logical+q_len``,
    contiguous in the batch.  Returns (input_ids, seq_ids, seq_lens).
    """
    input_ids, seq_ids, seq_lens = [], [], []
    for seq_id, logical, anchor, proposal in requests:
        tokens = [anchor, *proposal]
        input_ids.extend(tokens)
        seq_ids.extend([seq_id] * len(tokens))
        seq_lens.extend(range(logical + 1, logical + len(tokens) + 1))
    return input_ids, seq_ids, seq_lens


def aggregate_max_lens_by_seq_id(seq_ids_list, seq_lens_list):
    """swiftLLM/swiftllm/speculative.py:203-213."""
    if len(seq_ids_list) != len(seq_lens_list):
        raise ValueError("seq_ids_list and seq_lens_list must have the same length")
    out: dict[int, int] = {}
    for sid, sl in zip(seq_ids_list, seq_lens_list):
        out[sid] = max(out.get(sid, 0), sl)
    return out


def compute_greedy_acceptance(draft_token_ids, posterior_token_ids,
                              remaining_output_len=None, stop_token_ids=()):
    """swiftLLM/swiftllm/speculative.py:122-156 (greedy acceptance)."""
    if remaining_output_len is not None and remaining_output_len < 0:
        raise ValueError("remaining_output_len must be non-negative")
    if len(posterior_token_ids) < len(draft_token_ids) + 1:
        raise ValueError("posterior_token_ids must contain K+1 tokens for K draft tokens")
    n = 0
    while n < len(draft_token_ids) and posterior_token_ids[n] == draft_token_ids[n]:
        n += 1
    accepted = list(draft_token_ids[:n]) + [posterior_token_ids[n]]
    if remaining_output_len is not None:
        accepted = accepted[:remaining_output_len]
    stops = frozenset(int(t) for t in stop_token_ids)
    if any(t < 0 for t in stops):
        raise ValueError("stop_token_ids must be non-negative")
    for i, tok in enumerate(accepted):
        if tok in stops:
            accepted = accepted[: i + 1]
            break
    return accepted, min(n, len(accepted))


def reference_seq_block_size(num_kv_heads: int, decoding_seq_lens) -> int:
    """The reference's split-size heuristic, swiftLLM/swiftllm/worker/model.py:380-384."""
    sbs = 2048
    total = sum(decoding_seq_lens)
    max_len = max(decoding_seq_lens) if decoding_seq_lens else 0
    while num_kv_heads * (total / sbs) < 1024 and sbs // 2 >= 64 and max_len / (sbs // 2) <= 128:
        sbs //= 2
    return sbs


# --------------------------------------------------------------------------
# KV-cache placement
# --------------------------------------------------------------------------

def kv_slot_offset(block_table, seq_id, pos, layer, h, num_layers, num_kv_heads,
                   block_size, head_dim):
    """Flat element offset of (token ``pos`` of ``seq_id``, layer, kv head h).

    K/kvcache_mgmt.py:71-76 -- ``blk = block_table[seq_id, pos // bs]``,
    ``off = pos % bs``, offset ``((blk*L + layer)*Hkv + h)*bs*d + off*d``.
    """
    blk = int(block_table[seq_id, pos // block_size])
    off = pos % block_size
    return ((blk * num_layers + layer) * num_kv_heads + h) * block_size * head_dim + off * head_dim


def store_kvcache(k, v, k_cache, v_cache, block_table, seq_ids, seq_lens, layer):
    """Decode/verify KV store, in place on numpy caches.

    K/kvcache_mgmt.py:50-79 (kernel) and :124-132 (commented PyTorch loop):
    row r writes ``k[r]``/``v[r]`` ``[Hkv, d]`` to slot ``seq_len[r]-1`` of
    block ``block_table[seq_id[r], (seq_len[r]-1)//bs]`` at ``layer``.
    """
    bs = k_cache.shape[3]
    for r in range(k.shape[0]):
        pos = int(seq_lens[r]) - 1
        blk = int(block_table[int(seq_ids[r]), pos // bs])
        k_cache[blk, layer, :, pos % bs, :] = k[r]
        v_cache[blk, layer, :, pos % bs, :] = v[r]


def store_kvcache_prefill(k, v, k_cache, v_cache, block_table, seq_ids, prefill_lens, layer):
    """Prefill KV store, in place.  K/kvcache_mgmt.py:10-48: sequence s's
    tokens ``[start_s, start_s + len_s)`` of k/v go to positions 0..len_s-1."""
    bs = k_cache.shape[3]
    start = 0
    for sid, n in zip(seq_ids, prefill_lens):
        for pos in range(int(n)):
            blk = int(block_table[int(sid), pos // bs])
            k_cache[blk, layer, :, pos % bs, :] = k[start + pos]
            v_cache[blk, layer, :, pos % bs, :] = v[start + pos]
        start += int(n)


# --------------------------------------------------------------------------
# Prologue: QK-RMSNorm + RoPE
# --------------------------------------------------------------------------

def rmsnorm(x, w, eps):
    """K/rmsnorm.py:5-24: fp32 ``x * 1/sqrt(mean(x^2)+eps) * w`` -> fp16.

    ``x``: [..., hidden] fp16; ``w``: [hidden] fp16.
    """
    xf = x.astype(np.float32)
    var = np.mean(xf.astype(np.float64) ** 2, axis=-1, keepdims=True)
    rstd = (1.0 / np.sqrt(var + eps)).astype(np.float32)
    return (xf * rstd * w.astype(np.float32)).astype(np.float16)


def rope_cache(head_dim: int, theta: float, max_positions: int, scaling=1.0):
    """cos/sin tables, swiftLLM/swiftllm/worker/model.py:209-252.

    Number ``scaling`` (:242-246): ``inv_freq = 1/theta^(arange(0,d,2)/d)``
    and ``t = arange(n)/scaling`` in fp32, ``freqs = outer(t, inv_freq)``.
    Dict ``scaling`` (:209-240): frequencies below ``split = int(d/2 * lf /
    (lf + hf))`` use positions ``t/lf``, the rest ``t/hf`` (lf, hf = the
    dict's ``low_freq_factor``/``high_freq_factor``, default 1).  cos/sin
    cast to fp16.  Returns (cos, sin), each [max_positions, head_dim//2].
    """
    exps = np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)
    inv_freq = (np.float32(1.0) / np.power(np.float32(theta), exps, dtype=np.float32)).astype(np.float32)
    t = np.arange(max_positions, dtype=np.float32)
    if isinstance(scaling, dict):
        lf = np.float32(scaling.get("low_freq_factor", 1.0))
        hf = np.float32(scaling.get("high_freq_factor", 1.0))
        split = int((head_dim // 2) * float(lf) / (float(lf) + float(hf)))
        freqs = np.concatenate([np.outer((t / lf).astype(np.float32), inv_freq[:split]),
                                np.outer((t / hf).astype(np.float32), inv_freq[split:])], axis=1)
    else:
        freqs = np.outer((t / np.float32(scaling)).astype(np.float32), inv_freq)
    freqs = freqs.astype(np.float32)
    return np.cos(freqs).astype(np.float16), np.sin(freqs).astype(np.float16)


def rope(x, cos, sin):
    """Rotate-half RoPE of one tensor, K/rotary_emb.py:26-42.

    ``x``: [T, H, d] fp16; ``cos``/``sin``: [T, d/2] fp16 (row t = the
    token's position).  ``x0' = x0 cos - x1 sin``, ``x1' = x0 sin + x1 cos``
    on halves [0, d/2) and [d/2, d), evaluated in fp32 and rounded once to
    fp16 (the reference evaluates the same expression on fp16 operands).
    """
    half = x.shape[-1] // 2
    xf = x.astype(np.float32)
    c = cos.astype(np.float32)[:, None, :]
    s = sin.astype(np.float32)[:, None, :]
    x0, x1 = xf[..., :half], xf[..., half:]
    out = np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)
    return out.astype(np.float16)


def qk_norm_rope_store(q, k, v, q_w, k_w, eps, cos_cache, sin_cache, k_cache, v_cache,
                       block_table, seq_ids, seq_lens, layer):
    """The attention prologue of one decode/verify layer call.

    swiftLLM/swiftllm/worker/layers/transformer_layer.py:114-145 -- QK-RMSNorm
    per 128-wide head (:114-124), RoPE at position ``seq_len-1``
    (:127-131, positions from model.py:343-354,426-427), then the KV store
    (:133-143).  Returns (q', k') and updates the caches in place.
    """
    pos = np.asarray(seq_lens, dtype=np.int64) - 1
    qn = rmsnorm(q, q_w, eps)
    kn = rmsnorm(k, k_w, eps)
    qr = rope(qn, cos_cache[pos], sin_cache[pos])
    kr = rope(kn, cos_cache[pos], sin_cache[pos])
    store_kvcache(kr, v, k_cache, v_cache, block_table, seq_ids, seq_lens, layer)
    return qr, kr


# --------------------------------------------------------------------------
# Paged attention
# --------------------------------------------------------------------------

def gather_kv(k_cache, v_cache, block_table, seq_id, n_tokens, layer, dtype=np.float64):
    """K/V of tokens [0, n_tokens) of ``seq_id`` at ``layer`` as [Hkv, n, d].

    Block ``i`` of the sequence is ``block_table[seq_id, i]``
    (K/paged_attn.py:68-76; commented loop :227-236).
    """
    bs = k_cache.shape[3]
    nb = (n_tokens + bs - 1) // bs
    ids = np.asarray(block_table[seq_id, :nb], dtype=np.int64)
    kk = k_cache[ids, layer]  # [nb, Hkv, bs, d]
    vv = v_cache[ids, layer]
    hkv, d = kk.shape[1], kk.shape[3]
    kk = kk.transpose(1, 0, 2, 3).reshape(hkv, nb * bs, d)[:, :n_tokens].astype(dtype)
    vv = vv.transpose(1, 0, 2, 3).reshape(hkv, nb * bs, d)[:, :n_tokens].astype(dtype)
    return kk, vv


def _row_runs(seq_ids):
    """Maximal runs of consecutive rows with the same seq_id."""
    runs, start = [], 0
    n = len(seq_ids)
    for r in range(1, n + 1):
        if r == n or int(seq_ids[r]) != int(seq_ids[start]):
            runs.append((start, r))
            start = r
    return runs


def paged_attention(q, k_cache, v_cache, block_table, seq_ids, seq_lens, layer,
                    softmax_scale=None, dtype=np.float64):
    """Row-wise paged decode attention with natural-log LSE.

    K/paged_attn.py:33-108 (phase 1) and :125-149 (phase 2); the intended
    math is the commented PyTorch loop :224-259.  Row r, q-head qh attends
    tokens ``[0, seq_len[r])`` of ``block_table[seq_id[r]]`` in kv head
    ``qh // (Hq/Hkv)`` (:36) with scores ``q.k * softmax_scale`` (:72-73).

    ``q``: [R, Hq, d] (fp16 or float).  Returns (o [R, Hq, d], lse [R, Hq])
    in ``dtype``; ``lse = ln(sum_t exp(score_t))``.
    """
    rows, hq, d = q.shape
    hkv = k_cache.shape[2]
    g = hq // hkv
    if softmax_scale is None:
        softmax_scale = d ** -0.5
    seq_lens = np.asarray(seq_lens, dtype=np.int64)
    o = np.zeros((rows, hq, d), dtype=dtype)
    lse = np.zeros((rows, hq), dtype=dtype)
    for r0, r1 in _row_runs(seq_ids):
        n_tok = int(seq_lens[r0:r1].max())
        kk, vv = gather_kv(k_cache, v_cache, block_table, int(seq_ids[r0]), n_tok, layer, dtype)
        n = r1 - r0
        # [Hkv, n*G, d] x [Hkv, d, T]: q-head qh = kv*G + j uses kv head kv
        qq = q[r0:r1].astype(dtype).reshape(n, hkv, g, d).transpose(1, 0, 2, 3).reshape(hkv, n * g, d)
        s = np.matmul(qq, kk.transpose(0, 2, 1)) * dtype(softmax_scale)
        t = np.arange(n_tok)
        mask = np.repeat(t[None, :] >= seq_lens[r0:r1, None], g, axis=0)  # [n*G, T]
        s = np.where(mask[None], -np.inf, s)
        m = s.max(axis=-1, keepdims=True)
        p = np.exp(s - m)
        den = p.sum(axis=-1, keepdims=True)
        oo = np.matmul(p, vv) / den  # [Hkv, n*G, d]
        o[r0:r1] = oo.reshape(hkv, n, g, d).transpose(1, 0, 2, 3).reshape(n, hq, d)
        ll = (np.log(den) + m)[..., 0]  # [Hkv, n*G]
        lse[r0:r1] = ll.reshape(hkv, n, g).transpose(1, 0, 2).reshape(n, hq)
    return o, lse


def paged_attention_two_phase(q, k_cache, v_cache, block_table, seq_ids, seq_lens, layer,
                              seq_block_size, softmax_scale=None):
    """Split-KV restatement in the exp2 domain, mirroring the reference.

    Phase 1 (K/paged_attn.py:42-108): per (row, q-head, seq block of
    ``seq_block_size`` tokens) an online softmax with ``scale*log2(e)``
    (:195) gives normalised ``mid_o`` and ``log2(sum)+max`` (:105-108).
    Phase 2 (:128-149): LSE-weighted combine over ``cdiv(seq_len, sbs)``
    partials.  Returns (o, lse_natural), float64.
    """
    rows, hq, d = q.shape
    hkv = k_cache.shape[2]
    g = hq // hkv
    if softmax_scale is None:
        softmax_scale = d ** -0.5
    sc2 = softmax_scale * LOG2E
    o = np.zeros((rows, hq, d))
    lse = np.zeros((rows, hq))
    for r in range(rows):
        n_tok = int(seq_lens[r])
        kk, vv = gather_kv(k_cache, v_cache, block_table, int(seq_ids[r]), n_tok, layer)
        for qh in range(hq):
            kv = qh // g
            s2 = (kk[kv] @ q[r, qh].astype(np.float64)) * sc2
            mids, lses = [], []
            for start in range(0, n_tok, seq_block_size):
                part = s2[start:start + seq_block_size]
                mx = part.max()
                e = np.exp2(part - mx)
                mids.append((e @ vv[kv, start:start + seq_block_size]) / e.sum())
                lses.append(math.log2(e.sum()) + mx)
            mx = max(lses)
            w = np.exp2(np.asarray(lses) - mx)
            o[r, qh] = (w[:, None] * np.asarray(mids)).sum(0) / w.sum()
            lse[r, qh] = (math.log2(w.sum()) + mx) * LN2
    return o, lse


# --------------------------------------------------------------------------
# Prefill attention
# --------------------------------------------------------------------------

def prefill_attention(q, k, v, cu_seqlens, softmax_scale=None, dtype=np.float64):
    """Causal attention within each prompt of a packed batch, natural-log LSE.

    swiftLLM/swiftllm/worker/layers/transformer_layer.py:7-32 (the
    flash_attn_varlen_func the layer calls at :151-164 with
    cu_seqlens_q = cu_seqlens_k and causal=True): prompt i is tokens
    ``[cu[i], cu[i+1])``; K/V are repeated per q-head (:20-23, q-head qh
    reads kv head ``qh // (Hq/Hkv)``) and each position attends positions
    ``0..itself`` (``scaled_dot_product_attention(is_causal=True)``, :25-29).
    The Triton prefill_attention (K/prefill_attn.py:10-99) computes the same.

    ``q``: [T, Hq, d]; ``k``, ``v``: [T, Hkv, d].  Returns (o [T, Hq, d],
    lse [T, Hq]) in ``dtype``.
    """
    tokens, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    if softmax_scale is None:
        softmax_scale = d ** -0.5
    cu = [int(x) for x in cu_seqlens]
    o = np.zeros((tokens, hq, d), dtype=dtype)
    lse = np.zeros((tokens, hq), dtype=dtype)
    for s0, s1 in zip(cu[:-1], cu[1:]):
        n = s1 - s0
        if n <= 0:
            continue
        qq = q[s0:s1].astype(dtype).transpose(1, 0, 2)          # [Hq, n, d]
        kk = np.repeat(k[s0:s1].astype(dtype).transpose(1, 0, 2), g, axis=0)
        vv = np.repeat(v[s0:s1].astype(dtype).transpose(1, 0, 2), g, axis=0)
        sc = np.matmul(qq, kk.transpose(0, 2, 1)) * dtype(softmax_scale)   # [Hq, n, n]
        causal = np.arange(n)[None, :] > np.arange(n)[:, None]
        sc = np.where(causal[None], -np.inf, sc)
        m = sc.max(axis=-1, keepdims=True)
        p = np.exp(sc - m)
        den = p.sum(axis=-1, keepdims=True)
        o[s0:s1] = (np.matmul(p, vv) / den).transpose(1, 0, 2)
        lse[s0:s1] = (np.log(den) + m)[..., 0].T
    return o, lse
