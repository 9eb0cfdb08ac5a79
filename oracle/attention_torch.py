"""PyTorch-CPU restatement of swiftLLM's verify/decode paged attention.

TEST INFRASTRUCTURE ONLY: the timed CPU baseline of ``bench.py``'s
``cpu_baseline`` legs and a cross-check in ``tests/``; never imported by the
product package.

It follows the row-wise PyTorch formulation that the reference keeps beside
its Triton kernels (swiftLLM/swiftllm/worker/kernels/paged_attn.py:224-259):
row r gathers blocks ``block_table[seq_id[r], :cdiv(seq_len[r], 16)]`` of
``cur_layer`` (:227-236), scores ``q . k * softmax_scale`` over its first
``seq_len[r]`` tokens (:242-252) and averages V with their softmax (:254-258);
q-head ``qh`` reads kv head ``qh // (Hq / Hkv)`` (:237-238).  Unlike that loop
it keeps the gathered K/V per kv head (no repeat over the group) and also
returns the natural-log LSE.  All arithmetic is fp32 on the CPU.

Pinned by ``tests/test_oracle_torch.py`` against the numpy oracle
(``oracle.paged_attention``, itself pinned by SDPA, brute force and closed
forms) on random, ragged and interleaved inputs.
"""

from __future__ import annotations

import torch

__all__ = ["paged_attention_rowwise"]


def paged_attention_rowwise(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                            block_table: torch.Tensor, seq_ids, seq_lens, layer: int,
                            softmax_scale: float | None = None):
    """(o [R, Hq, d], lse [R, Hq]) in fp32 for decode/verify rows.

    ``q`` [R, Hq, d]; ``k_cache``/``v_cache`` [blocks, layers, Hkv, 16, d];
    ``block_table`` [rows, width] integer; all CPU tensors.
    """
    rows, hq, d = q.shape
    hkv, bs = k_cache.shape[2], k_cache.shape[3]
    g = hq // hkv
    scale = d ** -0.5 if softmax_scale is None else softmax_scale
    o = torch.empty((rows, hq, d), dtype=torch.float32)
    lse = torch.empty((rows, hq), dtype=torch.float32)
    for r in range(rows):
        n = int(seq_lens[r])
        nb = (n + bs - 1) // bs
        ids = block_table[int(seq_ids[r]), :nb].long()
        kk = k_cache[ids, layer].float().permute(1, 0, 2, 3).reshape(hkv, nb * bs, d)[:, :n]
        vv = v_cache[ids, layer].float().permute(1, 0, 2, 3).reshape(hkv, nb * bs, d)[:, :n]
        qq = q[r].float().view(hkv, g, d)
        s = torch.bmm(qq, kk.transpose(1, 2)) * scale           # [Hkv, G, n]
        m = s.amax(dim=-1, keepdim=True)
        p = torch.exp(s - m)
        den = p.sum(dim=-1, keepdim=True)
        o[r] = (torch.bmm(p, vv) / den).reshape(hq, d)
        lse[r] = (torch.log(den) + m).reshape(hq)
    return o, lse
