"""The native decoder stack (nsd_decoder_forward) against the layers run from
Python (transformer_layer.py:83-201 in this package's kernels and F.linear).

Two models with the same seed (same weights, same block tables) prefill the
same prompts through Python (their caches then agree bit for bit) and decode
the same verify rows, one through the native stack, one from Python.  Every
layer's K/V for the new rows lands in the cache, and each layer's K depends
on the previous layers' outputs, so comparing the caches checks every
layer of the stack, not only the last.  The two paths issue the same kernels;
the projection GEMMs are hipBLASLt in both, chosen by this library's
heuristic query on one side and by torch's on the other, so values may sit
an fp16 rounding apart: caches within 2e-2 abs, tokens equal except at
float near-ties (at most one row).  Every case prints its name first.
"""

from __future__ import annotations

import pytest
import torch

from nebulasd_amd import _lib
from nebulasd_amd.config import QWEN3_0_6B, QWEN3_8B
from nebulasd_amd.decoder import DecoderStack
from nebulasd_amd.spec_loop import RandomQwen3

pytestmark = pytest.mark.gpu


def _pair(cfg, n_layers, gpu, prompt_lens, depth):
    cfg = dict(cfg, num_hidden_layers=n_layers)
    blocks = [(p + depth + 4) // 16 + 1 for p in prompt_lens]
    a = RandomQwen3(cfg, blocks, gpu, seed=3, native=True)
    b = RandomQwen3(cfg, blocks, gpu, seed=3, native=False)
    g = torch.Generator().manual_seed(4)
    prompts = [torch.randint(0, cfg["vocab_size"], (n,), generator=g).tolist() for n in prompt_lens]
    ids = list(range(len(prompt_lens)))
    ta, tb = a.prefill(ids, prompts), b.prefill(ids, prompts)
    assert ta == tb
    assert torch.equal(a.k_cache, b.k_cache) and torch.equal(a.v_cache, b.v_cache)
    return a, b, prompts


@pytest.mark.parametrize("cfg,n_layers,n_req,depth", [(QWEN3_0_6B, 4, 64, 0), (QWEN3_8B, 3, 16, 4),
                                                      (QWEN3_0_6B, 2, 3, 2)],
                         ids=["0.6b-decode64", "8b-verify16x5", "0.6b-verify3x3"])
def test_decoder_stack_equals_python_layers(gpu, cfg, n_layers, n_req, depth):
    print(f"decoder stack {n_layers} layers, {n_req} requests, depth {depth}", flush=True)
    g = torch.Generator().manual_seed(5)
    prompt_lens = torch.randint(20, 300, (n_req,), generator=g).tolist()
    a, b, prompts = _pair(cfg, n_layers, gpu, prompt_lens, depth)
    sids, slens, toks = [], [], []
    for r, p in enumerate(prompts):
        rows = [p[-1]] + torch.randint(0, cfg["vocab_size"], (depth,), generator=g).tolist()
        sids += [r] * len(rows)
        slens += list(range(len(p) + 1, len(p) + 1 + len(rows)))
        toks += rows
    seen = {}

    def probe(model, li, q, o, lse, seq_ids, seq_lens):
        seen[id(model)] = (li, q.clone(), o.clone(), lse.clone())
    a.check = (n_layers // 2, probe)
    b.check = (n_layers // 2, probe)
    out_a = a.decode(sids, slens, toks)
    out_b = b.decode(sids, slens, toks)
    torch.cuda.synchronize()
    assert a.stacks and not b.stacks, "expected one native and one Python forward"
    for x, y, what in ((a.k_cache, b.k_cache, "k_cache"), (a.v_cache, b.v_cache, "v_cache")):
        err = (x.float() - y.float()).abs().max().item()
        print(f"  {what}: max |native - python| = {err:.2e}", flush=True)
        assert err <= 2e-2, what
    (la, qa, oa, sa), (lb, qb, ob, sb) = seen[id(a)], seen[id(b)]
    assert la == lb == n_layers // 2
    for x, y, what in ((qa, qb, "probe q"), (oa, ob, "probe o"), (sa, sb, "probe lse")):
        assert (x.float() - y.float()).abs().max().item() <= 2e-2, what
    diff = sum(u != v for u, v in zip(out_a, out_b))
    print(f"  tokens differing: {diff} of {len(out_a)}", flush=True)
    assert diff <= 1


def test_decoder_stack_rejects_bad_calls(gpu):
    cfg = dict(QWEN3_0_6B, num_hidden_layers=2)
    m = RandomQwen3(cfg, [4, 4], gpu, seed=1)
    with pytest.raises(ValueError, match="layer weight sets"):
        DecoderStack(m.mc, m.layers * 2)
    bad = [dict(lw) for lw in m.layers]
    bad[1]["wo"] = bad[1]["wo"][:, :64].contiguous()
    with pytest.raises(ValueError, match="layer 1: wo"):
        DecoderStack(m.mc, bad)
    with pytest.raises(_lib.NativeLibraryError, match="max_rows"):
        DecoderStack(m.mc, m.layers, max_rows=129)
    stack = DecoderStack(m.mc, m.layers, max_rows=2)
    from nebulasd_amd.infer_state import build_infer_state

    st = build_infer_state([0, 1, 1], [10, 11, 12], [], m.mc, m.cos, m.sin, gpu)
    x = torch.zeros((3, m.mc.hidden_size), dtype=torch.float16, device=gpu)
    with pytest.raises(ValueError, match="1..2"):
        stack.forward(x, torch.zeros_like(x), m.k_cache, m.v_cache, m.block_table, m.ec, st, m.cos, m.sin)
    st = build_infer_state([0, 1], [5], [4], m.mc, m.cos, m.sin, gpu)
    x = torch.zeros((1, m.mc.hidden_size), dtype=torch.float16, device=gpu)
    with pytest.raises(ValueError, match="decode/verify rows only"):
        stack.forward(x, torch.zeros_like(x), m.k_cache, m.v_cache, m.block_table, m.ec, st, m.cos, m.sin)
    stack.close()
    with pytest.raises(RuntimeError, match="closed"):
        stack.forward(x, torch.zeros_like(x), m.k_cache, m.v_cache, m.block_table, m.ec, st, m.cos, m.sin)
