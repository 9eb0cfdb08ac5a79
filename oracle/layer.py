"""numpy restatement of the rest of the layer around the attention path (the
oracle): fused add-RMSNorm, SiLU-and-multiply, the post-layer's last-token
gather, norm, lm_head and argmax, and one whole decode/verify layer
(``decoder_layer``) composed from them and the attention oracle.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``; never by the product package.

All reference citations are relative to ``swiftLLM/swiftllm/worker``.

How each function is pinned (``tests/test_oracle_layer.py``):

* ``fused_add_rmsnorm`` -- torch's fp16 add for the residual (bit-exact) and
  ``torch.nn.functional.rms_norm`` for the output; the constant-row closed
  form; a planted mistake (the norm taken over x instead of x + residual).
* ``silu_and_mul`` -- ``torch.nn.functional.silu`` on the gate half times
  the up half; closed forms (gate 0 -> 0, large gate -> up); planted mistake
  (halves swapped).
* ``argmax_first`` -- ``torch.argmax`` on fp16 rows, and known answers for
  ties (first index), NaN (counts as the maximum) and -0 == +0.
* ``last_token_indices`` -- hand-built infer states whose answer is known.
* ``lm_head_logits`` -- ``torch.nn.functional.linear`` in float64.
* ``linear`` -- ``torch.nn.functional.linear`` in float64.
* ``decoder_layer`` -- closed forms that fix its wiring: zero O and down
  projections (the output is 0 and the residual x + residual); every row the
  first token of its sequence (attention returns each q head's v row, so the
  O projection sees v repeated over its GQA group, checked against a
  hand-built product); the new cache slots equal ``qk_norm_rope_store``'s;
  a planted mistake (up and gate halves swapped) changes the output.
"""

from __future__ import annotations

import numpy as np

from .attention import paged_attention, qk_norm_rope_store

__all__ = ["fused_add_rmsnorm", "silu_and_mul", "argmax_first", "last_token_indices", "lm_head_logits",
           "post_layer", "rmsnorm_rows", "linear", "decoder_layer"]


def fused_add_rmsnorm(x, residual, weight, eps):
    """layers/../kernels/rmsnorm.py:39-72: r = x + r in fp16 (:57-59), then
    x = fp16(fp32(r) * 1/sqrt(mean(r^2) + eps) * w) (:61-67); computed here in
    float64.  Returns (x_out, residual_out)."""
    r = (x.astype(np.float32) + residual.astype(np.float32)).astype(np.float16)
    return rmsnorm_rows(r, weight, eps), r


def rmsnorm_rows(x, weight, eps):
    """kernels/rmsnorm.py:5-24 per row, float64 arithmetic, fp16 result."""
    xf = x.astype(np.float64)
    rstd = 1.0 / np.sqrt((xf * xf).mean(axis=-1, keepdims=True) + eps)
    return (xf * rstd * weight.astype(np.float64)).astype(np.float16)


def silu_and_mul(x):
    """kernels/silu_and_mul.py:5-23: up = x[:, :I], gate = x[:, I:] (:15-21),
    gate' = fp16(gate / (1 + exp(-gate))) in fp32 (here float64), out =
    fp16(up * gate').  Returns the [tokens, I] result (the reference writes
    it over x[:, :I])."""
    inter = x.shape[1] // 2
    up = x[:, :inter].astype(np.float64)
    g = x[:, inter:].astype(np.float64)
    with np.errstate(over="ignore"):
        sg = (g / (1.0 + np.exp(-g))).astype(np.float16).astype(np.float64)
    return (up * sg).astype(np.float16)


def argmax_first(logits):
    """torch.argmax(logits, dim=1) (layers/post_layer.py:69): the first
    maximum of every row, a NaN counting as the maximum, -0 equal to +0."""
    return np.argmax(logits, axis=1).astype(np.int64)


def last_token_indices(prefill_seq_start_locs, prefill_seq_lens, num_prefill_tokens, num_tokens):
    """layers/post_layer.py:53-59: each prompt's last token, then every decode row."""
    starts = np.asarray(prefill_seq_start_locs, np.int64)
    lens = np.asarray(prefill_seq_lens, np.int64)
    return np.concatenate([starts + lens - 1, np.arange(num_prefill_tokens, num_tokens, dtype=np.int64)])


def lm_head_logits(x, lm_head, dtype=np.float64):
    """layers/post_layer.py:68 (kernels/linear.py:3-12): x @ lm_head^T,
    sums in `dtype` (float64 for parity; float32 for the timed CPU baseline)
    rounded to fp16."""
    return (x.astype(dtype, copy=False) @ lm_head.astype(dtype, copy=False).T).astype(np.float16)


def post_layer(input_embds, indices, final_norm, lm_head, eps):
    """layers/post_layer.py:49-79: gather, RMSNorm, logits, argmax.
    Returns (tokens, logits)."""
    last = rmsnorm_rows(input_embds[np.asarray(indices)], final_norm, eps)
    logits = lm_head_logits(last, lm_head)
    return argmax_first(logits), logits


def linear(x, w):
    """kernels/linear.py:3-12 (F.linear without bias): x @ w^T with float64
    sums, rounded to fp16 as the reference's fp16 output."""
    return (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float16)


def decoder_layer(x, residual, weights, eps, cos_cache, sin_cache, k_cache, v_cache, block_table, seq_ids,
                  seq_lens, layer, num_q_heads, num_kv_heads):
    """One Qwen3 decoder layer over decode/verify rows,
    layers/transformer_layer.py:83-201: fused add-RMSNorm (:98-103), the q, k
    and v projections (:107-109; ``weights["wqkv"]`` stacks their rows),
    QK-RMSNorm + RoPE + KV store (:114-143), paged attention (:169-180), the
    O projection (:188-189), fused add-RMSNorm (:192), up/gate + SiLU-and-mul
    (:199-200; ``weights["wug"]`` holds the up rows, then the gate rows) and
    the down projection (:201).  Float64 arithmetic with the reference's
    fp16 tensors between the steps.  ``weights``: n_in, wqkv, q_norm, k_norm,
    wo, n_post, wug, wd (fp16).  Writes the rows' K/V to their cache slots of
    ``layer`` (in place) and returns (x_out, residual_out)."""
    d = weights["q_norm"].shape[0]
    hq, hkv = num_q_heads, num_kv_heads
    rows = x.shape[0]
    h, r1 = fused_add_rmsnorm(x, residual, weights["n_in"], eps)
    qkv = linear(h, weights["wqkv"])
    q = qkv[:, :hq * d].reshape(rows, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].reshape(rows, hkv, d)
    v = qkv[:, (hq + hkv) * d:].reshape(rows, hkv, d)
    q, _ = qk_norm_rope_store(q, k, v, weights["q_norm"], weights["k_norm"], eps, cos_cache, sin_cache,
                              k_cache, v_cache, block_table, seq_ids, seq_lens, layer)
    o, _ = paged_attention(q, k_cache, v_cache, block_table, seq_ids, seq_lens, layer)
    a = linear(o.astype(np.float16).reshape(rows, hq * d), weights["wo"])
    h2, r2 = fused_add_rmsnorm(a, r1, weights["n_post"], eps)
    y = linear(silu_and_mul(linear(h2, weights["wug"])), weights["wd"])
    return y, r2
