"""GPU parity of the paged verify/decode attention against the numpy oracle.

Every case prints its name first (pytest -v) so a failing GPU step is named.
Tolerances (written in tests/helpers.py): o within 2e-3 abs + 1e-2 rel,
natural-log LSE within 1e-4 abs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from helpers import ATOL_LSE, ATOL_O, RTOL_O, assert_close, compact_cache
from nebulasd_amd import _lib
from nebulasd_amd import plan as planmod
from nebulasd_amd.config import QWEN3_0_6B, QWEN3_8B, EngineConfig, ModelConfig
from nebulasd_amd.infer_state import build_infer_state, rope_cache
from nebulasd_amd.kernels import paged_attention
from nebulasd_amd.workload import make_workload

pytestmark = pytest.mark.gpu


def run_attention(w, layer, max_group_rows=0, validate=True):
    mc = ModelConfig(w.spec.model)
    ec = EngineConfig(block_size=16, max_blocks_per_seq=w.block_table.shape[1])
    cos, sin = rope_cache(mc.head_dim, mc.rope_theta, max(w.seq_lens) + 1, w.q.device)
    st = build_infer_state(w.seq_ids, w.seq_lens, [], mc, cos, sin, w.q.device, max_group_rows)
    o = torch.empty_like(w.q)
    lse = torch.empty(w.q.shape[:2], dtype=torch.float32, device=w.q.device)
    paged_attention(w.q, w.k_cache, w.v_cache, w.block_table, mc, ec, st, layer, o, lse,
                    validate=validate)
    torch.cuda.synchronize()
    return o, lse, st


def oracle_attention(w, layer):
    kc, vc, bt = compact_cache(w.k_cache, w.v_cache, w.block_table, w.seq_ids, w.seq_lens, layer)
    return oracle.paged_attention(w.q.cpu().numpy(), kc, vc, bt, w.seq_ids, w.seq_lens, 0)


def check_against_oracle(w, layer, o, lse, what):
    wo, wl = oracle_attention(w, layer)
    e_o = assert_close(o.float().cpu().numpy(), wo, ATOL_O, RTOL_O, f"{what} o")
    e_l = assert_close(lse.cpu().numpy(), wl, ATOL_LSE, 0.0, f"{what} lse")
    print(f"{what}: max|do|={e_o:.2e} max|dlse|={e_l:.2e}", flush=True)


CASES = [("cpu_plumbing", 0), ("cpu_plumbing", 1), ("cpu_plumbing", 2)] + \
    [(n, s) for n in ("draft_decode", "target_verify", "ragged_verify") for s in range(5)]


@pytest.mark.parametrize("name,seed", CASES, ids=[f"{n}-s{s}" for n, s in CASES])
def test_attention_matches_oracle(gpu, name, seed):
    w = make_workload(name, seed, device=gpu)
    layer = w.spec.num_layers // 2
    o, lse, st = run_attention(w, layer)
    check_against_oracle(w, layer, o, lse, f"{name} seed {seed}")
    if name == "target_verify":
        # the reference's row-wise launch (no verify grouping) gives the same result
        o1, l1, _ = run_attention(w, layer, max_group_rows=1)
        check_against_oracle(w, layer, o1, l1, f"{name} seed {seed} row-wise")
    del w
    torch.cuda.empty_cache()


EDGE_CTXS = [0, 1, 14, 15, 16, 17, 30, 31, 32, 33, 47, 63, 64, 65, 100, 127, 128, 257]


@pytest.mark.parametrize("model,q_len", [(QWEN3_8B, 1), (QWEN3_8B, 5), (QWEN3_8B, 9),
                                         (QWEN3_8B, 16), (QWEN3_8B, 17), (QWEN3_0_6B, 1),
                                         (QWEN3_0_6B, 5), (QWEN3_0_6B, 32)],
                         ids=["8b-q1", "8b-q5", "8b-q9", "8b-q16", "8b-q17", "06b-q1", "06b-q5",
                              "06b-q32"])
def test_attention_chunk_boundaries(gpu, model, q_len):
    """Contexts on both sides of the 16-token block and 32-token chunk edges."""
    w = make_workload("target_verify", 3, device=gpu, pool_blocks=600, num_layers=3,
                      ctxs=EDGE_CTXS, q_len=q_len, model=model)
    o, lse, _ = run_attention(w, 2)
    check_against_oracle(w, 2, o, lse, f"edges q_len={q_len}")


@pytest.mark.parametrize("hq,hkv,q_len", [(8, 8, 5), (40, 8, 5), (40, 8, 1), (64, 8, 5), (64, 8, 9), (32, 4, 1)],
                         ids=["gqa1-q5", "gqa5-q5", "gqa5-q1", "gqa8-q5", "gqa8-q9", "32x4-q1"])
def test_attention_gqa_ratios(gpu, hq, hkv, q_len):
    """Head layouts beyond the two benchmark models: one q-head per kv head,
    the Qwen3-14B (40/8) and Qwen3-32B (64/8) groups, and four kv heads.
    With 8 q-heads per kv head a 9-row verify group is 72 rows, more than one
    64-row MFMA group holds, so the planner splits it into 8 + 1 rows."""
    model = dict(QWEN3_8B, num_attention_heads=hq, num_key_value_heads=hkv)
    w = make_workload("target_verify", 4, device=gpu, num_layers=2, q_len=q_len, model=model)
    o, lse, _ = run_attention(w, 1)
    check_against_oracle(w, 1, o, lse, f"gqa {hq}/{hkv} q_len={q_len}")
    del w
    torch.cuda.empty_cache()


@pytest.mark.parametrize("q_len", [12, 16], ids=["48rows", "64rows"])
def test_attention_long_contexts_wide_groups(gpu, q_len):
    """48- and 64-row groups over log-uniform contexts up to 32k: segments cut
    into pieces whose wave merge runs in two 64-dim rounds and whose fp32
    partials are combined across workgroups."""
    w = make_workload("ragged_verify", 1, device=gpu, num_layers=2, q_len=q_len)
    o, lse, st = run_attention(w, 1)
    assert st.attn_plan.host[6] > 0, "expected split segments"
    check_against_oracle(w, 1, o, lse, f"ragged q_len={q_len}")
    del w
    torch.cuda.empty_cache()


def test_attention_every_layer_and_repeatable(gpu):
    """Every layer checks against the oracle; a repeated call gives the same
    bits (every output is summed in a fixed order, whatever the timing)."""
    w = make_workload("target_verify", 4, device=gpu, pool_blocks=2048, num_layers=4,
                      ctxs=[300, 1000, 77, 2500])
    for layer in range(4):
        o, lse, _ = run_attention(w, layer)
        check_against_oracle(w, layer, o, lse, f"layer {layer}")
    for _ in range(3):
        o2, lse2, _ = run_attention(w, 3)
        assert torch.equal(o, o2) and torch.equal(lse, lse2)


def test_attention_reused_plan_split_segments(gpu):
    """One plan and workspace across calls and layers: long contexts cut into
    many pieces, whose partials every call rewrites before merging them."""
    w = make_workload("target_verify", 7, device=gpu, pool_blocks=4096, num_layers=3,
                      ctxs=[20000, 33, 9000, 1], q_len=5)
    mc = ModelConfig(w.spec.model)
    ec = EngineConfig(block_size=16, max_blocks_per_seq=w.block_table.shape[1])
    cos, sin = rope_cache(mc.head_dim, mc.rope_theta, max(w.seq_lens) + 1, w.q.device)
    st = build_infer_state(w.seq_ids, w.seq_lens, [], mc, cos, sin, w.q.device)
    o = torch.empty_like(w.q)
    lse = torch.empty(w.q.shape[:2], dtype=torch.float32, device=w.q.device)
    for layer in (2, 0, 1, 2):
        paged_attention(w.q, w.k_cache, w.v_cache, w.block_table, mc, ec, st, layer, o, lse,
                        validate=True)
        torch.cuda.synchronize()
        assert int(st.attn_plan.host[6]) > 0, "the long contexts should be split across workgroups"
        check_against_oracle(w, layer, o, lse, f"reused plan layer {layer}")


def test_attention_reference_style_infer_state(gpu):
    """A bare object with only the reference infer state's fields works as the
    drop-in does (the plan is attached on first use and reused)."""
    import types

    w = make_workload("target_verify", 8, device=gpu, pool_blocks=1024, num_layers=2,
                      ctxs=[100, 700, 3], q_len=5)
    mc = ModelConfig(w.spec.model)
    ec = EngineConfig(block_size=16, max_blocks_per_seq=w.block_table.shape[1])
    st = types.SimpleNamespace(
        num_prefill_seqs=0, num_decoding_seqs=w.rows, softmax_scale=128 ** -0.5,
        seq_ids=torch.tensor(w.seq_ids, dtype=torch.int32, device=gpu),
        decoding_seq_lens=torch.tensor(w.seq_lens, dtype=torch.int32, device=gpu))
    o = torch.empty_like(w.q)
    lse = torch.empty(w.q.shape[:2], dtype=torch.float32, device=gpu)
    for layer in (1, 0):
        paged_attention(w.q, w.k_cache, w.v_cache, w.block_table, mc, ec, st, layer, o, lse)
        torch.cuda.synchronize()
        check_against_oracle(w, layer, o, lse, f"reference-style state layer {layer}")
    assert st.nsd_attn_plan.n_rows == w.rows


def test_attention_closed_form_single_token(gpu):
    """seq_len = 1: the output is V of token 0 and the LSE its score."""
    w = make_workload("target_verify", 5, device=gpu, pool_blocks=64, num_layers=2,
                      ctxs=[0, 0, 0], q_len=1)
    o, lse, _ = run_attention(w, 1)
    blk = w.block_table[:, 0].long()
    v0 = w.v_cache[blk, 1, :, 0].float()  # [3, Hkv, d]
    k0 = w.k_cache[blk, 1, :, 0].float()
    g = w.spec.num_q_heads // w.spec.num_kv_heads
    want_o = v0.repeat_interleave(g, dim=1)
    want_l = (w.q.float() * k0.repeat_interleave(g, dim=1)).sum(-1) * 128 ** -0.5
    assert_close(o.float().cpu().numpy(), want_o.cpu().numpy(), 1e-3, 0, "seq_len=1 o")
    assert_close(lse.cpu().numpy(), want_l.cpu().numpy(), ATOL_LSE, 0, "seq_len=1 lse")


def test_attention_bad_block_is_flagged(gpu):
    """An out-of-range block id is skipped by the kernel and reported, not faulted on."""
    w = make_workload("target_verify", 6, device=gpu, pool_blocks=256, num_layers=2,
                      ctxs=[40, 90], q_len=5)
    w.block_table[1, 2] = w.k_cache.shape[0] + 5
    with pytest.raises(RuntimeError, match="block id outside the pool"):
        run_attention(w, 0, validate=True)


def test_attention_no_rows(gpu):
    mc = ModelConfig(QWEN3_8B)
    ec = EngineConfig(max_blocks_per_seq=4)
    cos, sin = rope_cache(128, 1e6, 8, gpu)
    st = build_infer_state([], [], [], mc, cos, sin, gpu)
    kc = torch.zeros((4, 1, 8, 16, 128), dtype=torch.float16, device=gpu)
    q = torch.empty((0, 32, 128), dtype=torch.float16, device=gpu)
    paged_attention(q, kc, kc, torch.zeros((1, 4), dtype=torch.int32, device=gpu), mc, ec, st, 0,
                    torch.empty_like(q))


@pytest.mark.parametrize("q_len", [5, 1, 9], ids=["verify-bound", "decode-claimed", "q9-claimed"])
def test_attention_graph_replay_bit_identical(gpu, q_len, monkeypatch):
    """A HIP graph of attention calls over every layer replays to the eager
    results bit for bit, replay after replay, with eager work in between.
    The decode and 9-row cases ask the planner for two pieces per workgroup
    slot, so their later workgroups claim pieces from the workspace's
    counter, which every call (replayed or eager) must leave at zero."""
    print(f"graph replay, q_len {q_len}", flush=True)
    if q_len != 5:
        monkeypatch.setattr(planmod, "PIECES_PER_SLOT", 2.0)
    w = make_workload("target_verify", 9, device=gpu, pool_blocks=4096, num_layers=3,
                      ctxs=[6000, 40, 3000, 1400, 9], q_len=q_len)
    mc = ModelConfig(w.spec.model)
    ec = EngineConfig(block_size=16, max_blocks_per_seq=w.block_table.shape[1])
    cos, sin = rope_cache(mc.head_dim, mc.rope_theta, max(w.seq_lens) + 1, w.q.device)
    st = build_infer_state(w.seq_ids, w.seq_lens, [], mc, cos, sin, w.q.device)
    outs = [torch.empty_like(w.q) for _ in range(3)]
    lses = [torch.empty(w.q.shape[:2], dtype=torch.float32, device=gpu) for _ in range(3)]

    def calls():
        for layer in range(3):
            paged_attention(w.q, w.k_cache, w.v_cache, w.block_table, mc, ec, st, layer,
                            outs[layer], lses[layer])

    calls()
    torch.cuda.synchronize()
    eager = [(o.clone(), l.clone()) for o, l in zip(outs, lses)]
    assert int(st.attn_plan.host[_lib.PLAN_COMBINES]) > 0, "expected split segments (the partial merge launch)"
    if q_len != 5:
        assert int(st.attn_plan.host[_lib.PLAN_CLAIMED]) > 0, "expected claimed pieces"
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            calls()
    torch.cuda.synchronize()
    for rep in range(3):
        for o, l in zip(outs, lses):
            o.zero_()
            l.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for layer in range(3):
            assert torch.equal(outs[layer], eager[layer][0]), f"replay {rep} layer {layer} o"
            assert torch.equal(lses[layer], eager[layer][1]), f"replay {rep} layer {layer} lse"
        calls()  # eager work between replays
        torch.cuda.synchronize()
    check_against_oracle(w, 2, outs[2], lses[2], "graph replay layer 2")


def test_attention_mixed_prefill_forward(gpu):
    """A forward with prefill sequences first: the wrapper is given the decode
    rows' slices ``q[num_prefill_tokens:]`` / ``o[num_prefill_tokens:]`` and
    reads ``seq_ids[num_prefill_seqs:]`` (transformer_layer.py:171-179,
    paged_attn.py:197); the prefill part of ``o`` is left alone."""
    w = make_workload("target_verify", 10, device=gpu, pool_blocks=2048, num_layers=2,
                      ctxs=[900, 12, 2000, 333, 50, 1], q_len=5)
    mc = ModelConfig(w.spec.model)
    ec = EngineConfig(block_size=16, max_blocks_per_seq=w.block_table.shape[1])
    prefill_lens = [37, 5, 120]
    prefill_ids = [3, 0, 5]  # rows of the block table, as the engine assigns them
    npt = sum(prefill_lens)
    cos, sin = rope_cache(mc.head_dim, mc.rope_theta, max(w.seq_lens) + 1, w.q.device)
    st = build_infer_state(prefill_ids + list(w.seq_ids), w.seq_lens, prefill_lens, mc, cos, sin,
                           w.q.device)
    assert st.num_prefill_seqs == 3 and st.num_prefill_tokens == npt
    hq, d = w.q.shape[1:]
    q = torch.randn((npt + w.rows, hq, d), device=gpu).half()
    q[npt:] = w.q
    o = torch.full((npt + w.rows, hq * d), 7.0, dtype=torch.float16, device=gpu)
    lse = torch.empty((w.rows, hq), dtype=torch.float32, device=gpu)
    paged_attention(q[npt:], w.k_cache, w.v_cache, w.block_table, mc, ec, st, 1, o[npt:], lse,
                    validate=True)
    torch.cuda.synchronize()
    assert bool((o[:npt] == 7.0).all()), "the prefill rows of o were written"
    check_against_oracle(w, 1, o[npt:].view(w.rows, hq, d), lse, "mixed forward")


def test_attention_interleaved_rows(gpu):
    """Rows of one sequence that are not adjacent (a, b, a, b ...) are valid
    reference input; each row attends to its own seq_len prefix."""
    w = make_workload("target_verify", 11, device=gpu, pool_blocks=2048, num_layers=2,
                      ctxs=[700, 1500, 64], q_len=1)
    ctx = w.ctxs
    seq_ids = [0, 1, 0, 1, 2, 0, 2, 1]
    nth = {}
    seq_lens = []
    for s in seq_ids:
        nth[s] = nth.get(s, 0) + 1
        seq_lens.append(ctx[s] - 3 + nth[s])  # rising by one per row of the sequence
    hq, d = w.q.shape[1:]
    w.q = torch.randn((len(seq_ids), hq, d), device=gpu).half()
    w.seq_ids, w.seq_lens = seq_ids, seq_lens
    o, lse, st = run_attention(w, 1)
    check_against_oracle(w, 1, o, lse, "interleaved rows")
    # the same rows, grouped per sequence, give the same per-row results
    order = sorted(range(len(seq_ids)), key=lambda i: (seq_ids[i], seq_lens[i]))
    q_interleaved = w.q
    w.q = q_interleaved[order].contiguous()
    w.seq_ids, w.seq_lens = [seq_ids[i] for i in order], [seq_lens[i] for i in order]
    o2, lse2, _ = run_attention(w, 1)
    check_against_oracle(w, 1, o2, lse2, "same rows grouped")
