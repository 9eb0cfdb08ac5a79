"""The native decoder stack (nsd_decoder_forward) against the layers run from
Python (transformer_layer.py:83-201 in this package's kernels and F.linear).

Two models with the same seed (same weights, same block tables) prefill the
same prompts through Python (their caches then agree bit for bit) and decode
the same verify rows, one through the native stack, one from Python.  Every
layer's K/V for the new rows lands in the cache, and each layer's K depends
on the previous layers' outputs, so comparing the caches checks every
layer of the stack, not only the last.  The two paths share the attention,
prologue, norm and fused up/gate kernels; the stack's q/k/v, O and down
projections are this library's split-k GEMM (fp32 partials that the next
kernel sums), the Python layers' are torch's F.linear (hipBLASLt, fp16
output), so values may sit an fp16 rounding apart: caches within 2e-2 abs,
tokens equal except at float near-ties (at most one row).

One layer of the stack is also checked against the float64 layer oracle
(oracle.decoder_layer, composed from the oracle's norm, projection,
prologue, attention and SiLU-and-mul) at the two speculative shapes: 80
verify rows (Qwen3-8B, 16 requests x q_len 5) and 64 draft rows (Qwen3-0.6B
decode): the layer's output and residual, and the new K/V cache slots.
Every case prints its name first.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

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


@pytest.mark.parametrize("cfg,n_req,depth", [(QWEN3_8B, 16, 4), (QWEN3_0_6B, 64, 0)],
                         ids=["8b-verify80", "0.6b-decode64"])
def test_decoder_layer_matches_float64_oracle(gpu, cfg, n_req, depth):
    """One native decoder layer against oracle.decoder_layer.  The stack
    keeps the projections' sums in fp32 where the reference rounds them to
    fp16 and fuses SiLU-and-mul into the up/gate GEMM, so each step sits
    within a few fp16 roundings of the oracle: the output and residual
    within 1e-2 x their RMS at worst (2e-3 x RMS on average), new K/V
    slots within 2e-2 abs (their values are O(1) after the norm)."""
    print(f"decoder layer vs float64 oracle: {n_req} requests, q_len {depth + 1}", flush=True)
    cfg = dict(cfg, num_hidden_layers=1)
    g = torch.Generator().manual_seed(7)
    prompt_lens = torch.randint(20, 300, (n_req,), generator=g).tolist()
    blocks = [(p + depth + 4) // 16 + 1 for p in prompt_lens]
    m = RandomQwen3(cfg, blocks, gpu, seed=8, native=True)
    prompts = [torch.randint(0, cfg["vocab_size"], (n,), generator=g).tolist() for n in prompt_lens]
    m.prefill(list(range(n_req)), prompts)
    sids, slens, toks = [], [], []
    for r, p in enumerate(prompts):
        rows = [p[-1]] + torch.randint(0, cfg["vocab_size"], (depth,), generator=g).tolist()
        sids += [r] * len(rows)
        slens += list(range(len(p) + 1, len(p) + 1 + len(rows)))
        toks += rows
    assert len(sids) == n_req * (depth + 1)
    mc = m.mc
    from nebulasd_amd.infer_state import build_infer_state

    st = build_infer_state(sids, slens, [], mc, m.cos, m.sin, gpu)
    x = m.embed[torch.tensor(toks, device=gpu)]
    res = torch.zeros_like(x)
    x0 = x.cpu().numpy()
    kc, vc = m.k_cache.cpu().numpy(), m.v_cache.cpu().numpy()
    stack = DecoderStack(mc, m.layers)
    stack.forward(x, res, m.k_cache, m.v_cache, m.block_table, m.ec, st, m.cos, m.sin)
    torch.cuda.synchronize()
    stack.close()
    weights = {k: v.cpu().numpy() for k, v in m.layers[0].items()}
    want_y, want_r = oracle.decoder_layer(x0, np.zeros_like(x0), weights, mc.rms_norm_eps, m.cos.cpu().numpy(),
                                          m.sin.cpu().numpy(), kc, vc, m.block_table.cpu().numpy(), sids, slens,
                                          0, mc.num_q_heads, mc.num_kv_heads)
    for got, want, what in ((x, want_y, "output"), (res, want_r, "residual")):
        d = np.abs(got.float().cpu().numpy().astype(np.float64) - want.astype(np.float64))
        rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
        print(f"  {what}: rms {rms:.3g}, max |native - oracle| / rms {d.max() / rms:.2e}, "
              f"mean {d.mean() / rms:.2e}", flush=True)
        assert d.max() <= 1e-2 * rms and d.mean() <= 2e-3 * rms, what
    bt = m.block_table.cpu().numpy()
    got_k, got_v = m.k_cache.cpu().numpy(), m.v_cache.cpu().numpy()
    for r, (sid, n) in enumerate(zip(sids, slens)):
        blk, off = int(bt[sid, (n - 1) // 16]), (n - 1) % 16
        for got, want, what in ((got_k, kc, "k"), (got_v, vc, "v")):
            err = np.abs(got[blk, 0, :, off].astype(np.float64) - want[blk, 0, :, off].astype(np.float64)).max()
            assert err <= 2e-2, (what, r, err)
    # and nothing else of the caches moved
    mask = np.ones(kc.shape[:1] + kc.shape[2:4], bool)
    for sid, n in zip(sids, slens):
        mask[int(bt[sid, (n - 1) // 16]), :, (n - 1) % 16] = False
    assert np.array_equal(got_k[:, 0][mask], kc[:, 0][mask]) and np.array_equal(got_v[:, 0][mask], vc[:, 0][mask])


@pytest.mark.parametrize("cfg,n_req,depth", [(QWEN3_8B, 16, 0), (QWEN3_0_6B, 64, 0), (QWEN3_0_6B, 16, 4)],
                         ids=["8b-decode16", "0.6b-decode64", "0.6b-verify16x5"])
def test_decoder_fused_layers_equal_two_launch_layers(gpu, cfg, n_req, depth):
    """At batches whose groups fit one 16-row tile per kv head, a layer runs
    its prologue inside the attention's launch unless it is the probe layer,
    which runs them as two launches.  Two layers from the same state, with
    no probe (both fused), a probe on layer 1 and a probe on layer 0: the
    outputs, residuals and caches are the same bits."""
    print(f"decoder fused vs two-launch layers: {n_req} requests, q_len {depth + 1}", flush=True)
    cfg = dict(cfg, num_hidden_layers=2)
    g = torch.Generator().manual_seed(11)
    prompt_lens = torch.randint(20, 300, (n_req,), generator=g).tolist()
    blocks = [(p + depth + 4) // 16 + 1 for p in prompt_lens]
    m = RandomQwen3(cfg, blocks, gpu, seed=12, native=True)
    prompts = [torch.randint(0, cfg["vocab_size"], (n,), generator=g).tolist() for n in prompt_lens]
    m.prefill(list(range(n_req)), prompts)
    sids, slens, toks = [], [], []
    for r, p in enumerate(prompts):
        rows = [p[-1]] + torch.randint(0, cfg["vocab_size"], (depth,), generator=g).tolist()
        sids += [r] * len(rows)
        slens += list(range(len(p) + 1, len(p) + 1 + len(rows)))
        toks += rows
    from nebulasd_amd.infer_state import build_infer_state

    st = build_infer_state(sids, slens, [], m.mc, m.cos, m.sin, gpu)
    x0 = m.embed[torch.tensor(toks, device=gpu)]
    kc0, vc0 = m.k_cache.clone(), m.v_cache.clone()
    stack = DecoderStack(m.mc, m.layers)
    runs = []
    for probe in (-1, 1, 0):
        m.k_cache.copy_(kc0)
        m.v_cache.copy_(vc0)
        x, res = x0.clone(), torch.zeros_like(x0)
        stack.forward(x, res, m.k_cache, m.v_cache, m.block_table, m.ec, st, m.cos, m.sin, probe_layer=probe)
        torch.cuda.synchronize()
        runs.append((x, res, m.k_cache.clone(), m.v_cache.clone()))
    stack.close()
    assert st.attn_plan.rows_max <= 16, "a batch the stack runs fused"
    assert not torch.equal(runs[0][2], kc0), "the new K rows were written"
    for probe, run in zip((1, 0), runs[1:]):
        for a, b, what in zip(runs[0], run, ("output", "residual", "k cache", "v cache")):
            assert torch.equal(a, b), (probe, what)


@pytest.mark.parametrize("cfg,n_req,depth", [(QWEN3_0_6B, 64, 0), (QWEN3_8B, 16, 4)],
                         ids=["0.6b-decode64", "8b-verify16x5"])
def test_decoder_stack_graph_replay_bit_identical(gpu, cfg, n_req, depth):
    """The stack's forward captured in a HIP graph replays to the eager
    forward bit for bit (output, residual, caches), three replays from the
    same inputs, with an eager forward between them: the decode batch runs
    the prologue inside the attention launch, the verify batch as two."""
    print(f"decoder stack graph replay: {n_req} requests, q_len {depth + 1}", flush=True)
    cfg = dict(cfg, num_hidden_layers=2)
    g = torch.Generator().manual_seed(21)
    prompt_lens = torch.randint(20, 300, (n_req,), generator=g).tolist()
    blocks = [(p + depth + 4) // 16 + 1 for p in prompt_lens]
    m = RandomQwen3(cfg, blocks, gpu, seed=22, native=True)
    prompts = [torch.randint(0, cfg["vocab_size"], (n,), generator=g).tolist() for n in prompt_lens]
    m.prefill(list(range(n_req)), prompts)
    sids, slens, toks = [], [], []
    for r, p in enumerate(prompts):
        rows = [p[-1]] + torch.randint(0, cfg["vocab_size"], (depth,), generator=g).tolist()
        sids += [r] * len(rows)
        slens += list(range(len(p) + 1, len(p) + 1 + len(rows)))
        toks += rows
    from nebulasd_amd.infer_state import build_infer_state

    st = build_infer_state(sids, slens, [], m.mc, m.cos, m.sin, gpu)
    x0 = m.embed[torch.tensor(toks, device=gpu)]
    kc0, vc0 = m.k_cache.clone(), m.v_cache.clone()
    x, res = x0.clone(), torch.zeros_like(x0)
    stack = DecoderStack(m.mc, m.layers)

    def reset():
        x.copy_(x0)
        res.zero_()
        m.k_cache.copy_(kc0)
        m.v_cache.copy_(vc0)

    def fwd():
        stack.forward(x, res, m.k_cache, m.v_cache, m.block_table, m.ec, st, m.cos, m.sin)

    fwd()
    torch.cuda.synchronize()
    want = (x.clone(), res.clone(), m.k_cache.clone(), m.v_cache.clone())
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    reset()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            fwd()
    torch.cuda.synchronize()
    for rep in range(3):
        reset()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, exp, what in zip((x, res, m.k_cache, m.v_cache), want, ("output", "residual", "k cache", "v cache")):
            assert torch.equal(got, exp), (rep, what)
        reset()
        fwd()  # eager work between replays
        torch.cuda.synchronize()
    del graph
    stack.close()
