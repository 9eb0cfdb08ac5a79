"""GPU parity of the fused prologue + attention launch (nsd_paged_attention_fused).

The reference runs QK-RMSNorm, RoPE and the K/V store (transformer_layer.py
:114-145), then paged attention (:169-180).  The fused launch must give the
same bits as this build's two calls that restate them (qk_norm_rope_store,
then paged_attention, both checked against the oracle in their own tests):
o, lse and the whole K and V pools (so the new rows land in the same slots
and nothing else is written).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from nebulasd_amd import _lib
from nebulasd_amd import plan as planmod
from nebulasd_amd.config import QWEN3_0_6B, QWEN3_8B, EngineConfig, ModelConfig
from nebulasd_amd.infer_state import build_infer_state, rope_cache
from nebulasd_amd.kernels import paged_attention, paged_attention_fused, qk_norm_rope_store
from nebulasd_amd.kernels import qk_norm_rope_store_partials
from nebulasd_amd.kernels._util import stream_of
from nebulasd_amd.workload import make_workload
import oracle

from helpers import ATOL_O, RTOL_O, assert_close

pytestmark = pytest.mark.gpu

# contexts on both sides of block edges, so that the new rows of a group
# fall in one or two blocks, at the start of a block or across its edge;
# short ones give pieces whose new rows sit in a wave's first two blocks
CTXS = [0, 1, 11, 12, 15, 16, 27, 30, 31, 47, 100, 255, 1000, 2047, 3000, 4090]


def _setup(gpu, model, q_len, seed, ctxs=CTXS):
    w = make_workload("target_verify", seed, device=gpu, pool_blocks=3072, num_layers=3, ctxs=ctxs,
                      q_len=q_len, model=model)
    mc = ModelConfig(w.spec.model)
    ec = EngineConfig(block_size=16, max_blocks_per_seq=w.block_table.shape[1])
    cos, sin = rope_cache(128, mc.rope_theta, max(w.seq_lens) + 1, gpu)
    st = build_infer_state(w.seq_ids, w.seq_lens, [], mc, cos, sin, gpu)
    g = torch.Generator(device=gpu).manual_seed(seed + 77)
    hkv = mc.num_kv_heads
    k = torch.randn((w.rows, hkv, 128), device=gpu, generator=g).half()
    v = torch.randn((w.rows, hkv, 128), device=gpu, generator=g).half()
    qn = (torch.rand(128, device=gpu, generator=g) + 0.5).half()
    kn = (torch.rand(128, device=gpu, generator=g) + 0.5).half()
    return w, mc, ec, st, cos, sin, k, v, qn, kn


def _outputs(w, mc):
    o = torch.full_like(w.q, float("nan"))
    lse = torch.full(w.q.shape[:2], float("nan"), dtype=torch.float32, device=w.q.device)
    return o, lse


@pytest.mark.parametrize("model,q_len,claims", [
    (QWEN3_8B, 5, False), (QWEN3_8B, 1, False), (QWEN3_8B, 9, False), (QWEN3_0_6B, 1, False),
    (QWEN3_0_6B, 5, False), (QWEN3_8B, 1, True), (QWEN3_8B, 12, False),
    (dict(QWEN3_8B, num_attention_heads=40), 5, False), (dict(QWEN3_8B, num_attention_heads=64), 5, False),
    (dict(QWEN3_8B, num_attention_heads=8), 16, False), (dict(QWEN3_8B, num_key_value_heads=4), 1, False)],
    ids=["8b-q5", "8b-q1", "8b-q9", "06b-q1", "06b-q5", "8b-q1-claimed", "8b-q12", "gqa5-q5", "gqa8-q5",
         "gqa1-q16", "32x4-q1"])
def test_fused_equals_prologue_then_attention(gpu, model, q_len, claims, monkeypatch):
    print(f"fused vs unfused, q_len {q_len}, claims {claims}", flush=True)
    if claims:
        monkeypatch.setattr(planmod, "PIECES_PER_SLOT", 2.0)
    w, mc, ec, st, cos, sin, k, v, qn, kn = _setup(gpu, model, q_len, seed=21 + q_len)
    layer = 1
    kc0, vc0 = w.k_cache.clone(), w.v_cache.clone()
    # the two calls
    qa = w.q.clone()
    qk_norm_rope_store(qa, k.clone(), v, w.k_cache, w.v_cache, w.block_table, qn, kn, mc, ec, st, layer, cos, sin,
                       validate=True)
    oa, la = _outputs(w, mc)
    paged_attention(qa, w.k_cache, w.v_cache, w.block_table, mc, ec, st, layer, oa, la, validate=True)
    torch.cuda.synchronize()
    kca, vca = w.k_cache.clone(), w.v_cache.clone()
    # the fused launch, from the same pools
    w.k_cache.copy_(kc0)
    w.v_cache.copy_(vc0)
    ob, lb = _outputs(w, mc)
    qb = w.q.clone()
    paged_attention_fused(qb, k, v, w.k_cache, w.v_cache, w.block_table, qn, kn, mc, ec, st, layer, cos, sin,
                          ob, lb, validate=True)
    torch.cuda.synchronize()
    if claims:
        assert int(st.attn_plan.host[_lib.PLAN_CLAIMED]) > 0, "expected claimed pieces"
    assert torch.equal(qb, w.q), "the fused launch does not write q"
    assert torch.equal(ob, oa), f"o: max |d| {float((ob.float() - oa.float()).abs().max())}"
    assert torch.equal(lb, la), "lse"
    assert torch.equal(w.k_cache, kca), "k pool"
    assert torch.equal(w.v_cache, vca), "v pool"
    assert not torch.equal(kca, kc0), "the new rows were written"


@pytest.mark.parametrize("model,q_len,splits", [(QWEN3_8B, 5, 5), (QWEN3_0_6B, 1, 2)], ids=["8b-q5", "06b-q1"])
def test_fused_from_projection_partials(gpu, model, q_len, splits):
    """q, k and v as the fused q/k/v projection's fp32 split partials (the
    native decoder stack's input): the same bits as the partials prologue
    then attention."""
    print(f"fused from partials, q_len {q_len}, splits {splits}", flush=True)
    w, mc, ec, st, cos, sin, _, _, qn, kn = _setup(gpu, model, q_len, seed=40 + q_len)
    hq, hkv, layer = mc.num_q_heads, mc.num_kv_heads, 2
    g = torch.Generator(device=gpu).manual_seed(5)
    part = torch.randn((splits, w.rows, (hq + 2 * hkv) * 128), device=gpu, generator=g) * 0.5
    kc0, vc0 = w.k_cache.clone(), w.v_cache.clone()
    qa = torch.empty_like(w.q)
    qk_norm_rope_store_partials(part, qa, w.k_cache, w.v_cache, w.block_table, qn, kn, mc, ec, st, layer, cos, sin,
                                validate=True)
    oa, la = _outputs(w, mc)
    paged_attention(qa, w.k_cache, w.v_cache, w.block_table, mc, ec, st, layer, oa, la, validate=True)
    torch.cuda.synchronize()
    kca, vca = w.k_cache.clone(), w.v_cache.clone()
    w.k_cache.copy_(kc0)
    w.v_cache.copy_(vc0)
    ob, lb = _outputs(w, mc)
    plan = st.attn_plan
    _lib.call("nsd_paged_attention_fused", None, 0, None, 0, None, 0, part.data_ptr(), splits, qn.data_ptr(),
              kn.data_ptr(), float(mc.rms_norm_eps), cos.data_ptr(), sin.data_ptr(), cos.shape[0], ob.data_ptr(),
              lb.data_ptr(), w.k_cache.data_ptr(), w.v_cache.data_ptr(), w.k_cache.shape[0], w.k_cache.shape[1],
              layer, hq, hkv, 128, 16, w.block_table.data_ptr(), w.block_table.shape[0], w.block_table.shape[1],
              plan.host.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), plan.dev.data_ptr(),
              plan.workspace.data_ptr(), plan.workspace.numel(), float(st.softmax_scale), None, stream_of(w.q))
    torch.cuda.synchronize()
    assert torch.equal(ob, oa), f"o: max |d| {float((ob.float() - oa.float()).abs().max())}"
    assert torch.equal(lb, la), "lse"
    assert torch.equal(w.k_cache, kca), "k pool"
    assert torch.equal(w.v_cache, vca), "v pool"


def test_fused_refuses_sequences_split_over_groups(gpu):
    """17 verify rows of one request at GQA 4 are 68 rows, more than one
    48-row group: the plan splits the request, and the fused launch refuses
    it before any launch (the two calls serve it)."""
    w, mc, ec, st, cos, sin, k, v, qn, kn = _setup(gpu, QWEN3_8B, 17, seed=3, ctxs=[500, 40])
    o, lse = _outputs(w, mc)
    with pytest.raises(_lib.NativeLibraryError, match="several verify groups"):
        paged_attention_fused(w.q, k, v, w.k_cache, w.v_cache, w.block_table, qn, kn, mc, ec, st, 0, cos, sin, o,
                              lse)


def test_fused_matches_oracle(gpu):
    """The fused launch against the oracle directly: QK-RMSNorm + RoPE +
    K/V store (transformer_layer.py:114-145), then paged attention
    (:169-180), on host copies.  The oracle's q and new K rows are rounded
    to fp16 (the reference's q tensor and cache are fp16); a 1-ulp flip of
    an fp16 norm output can move a rotated element by ~2 ulp, which moves
    scores by up to ~1e-3, hence lse to 1e-3 here (1e-4 with a shared q)."""
    ctxs = [0, 11, 31, 300, 1000]
    w, mc, ec, st, cos, sin, k, v, qn, kn = _setup(gpu, QWEN3_8B, 5, seed=61, ctxs=ctxs)
    layer = 1
    kc_h, vc_h = w.k_cache.cpu().numpy(), w.v_cache.cpu().numpy()
    o, lse = _outputs(w, mc)
    paged_attention_fused(w.q, k, v, w.k_cache, w.v_cache, w.block_table, qn, kn, mc, ec, st, layer, cos, sin,
                          o, lse, validate=True)
    torch.cuda.synchronize()
    bt = w.block_table.cpu().numpy()
    qr, kr = oracle.qk_norm_rope_store(w.q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), qn.cpu().numpy(),
                                       kn.cpu().numpy(), float(mc.rms_norm_eps), cos.cpu().numpy(),
                                       sin.cpu().numpy(), kc_h, vc_h, bt, w.seq_ids, w.seq_lens, layer)
    wo, wl = oracle.paged_attention(qr.astype(np.float16), kc_h, vc_h, bt, w.seq_ids, w.seq_lens, layer)
    e_o = assert_close(o.float().cpu().numpy(), wo, ATOL_O, RTOL_O, "fused o")
    e_l = assert_close(lse.cpu().numpy(), wl, 1e-3, 0.0, "fused lse")
    print(f"fused vs oracle: max|do|={e_o:.2e} max|dlse|={e_l:.2e}", flush=True)
    # the new rows: V bit for bit, K to the prologue's tolerance, nothing else written
    kg, vg = w.k_cache.cpu().numpy(), w.v_cache.cpu().numpy()
    assert np.array_equal(vg.view(np.uint16), vc_h.view(np.uint16))
    diff = kg.view(np.uint16) != kc_h.view(np.uint16)
    new = np.zeros(kg.shape, bool)
    for sid, n in zip(w.seq_ids, w.seq_lens):
        blk = bt[sid, (n - 1) // 16]
        new[blk, layer, :, (n - 1) % 16, :] = True
    assert not (diff & ~new).any(), "only the new K rows may differ from the oracle's pool"
    np.testing.assert_allclose(kg[new].astype(np.float64), kc_h[new].astype(np.float64), atol=1e-3, rtol=2e-3)


@pytest.mark.parametrize("col", [2, 5], ids=["mid-context", "new-rows"])
def test_fused_bad_block_is_flagged(gpu, col):
    """An out-of-range block id, inside a sequence's context or where its new
    rows go, is skipped and reported, not faulted on: the fused launch gives
    the two calls' o, lse and pools (both skip the block) and its status word
    names the bad block."""
    print(f"fused, bad block id at column {col}", flush=True)
    w, mc, ec, st, cos, sin, k, v, qn, kn = _setup(gpu, QWEN3_8B, 5, seed=71, ctxs=[40, 90])
    w.block_table[1, col] = w.k_cache.shape[0] + 5  # ctx 90: new rows at 90..94, block 5
    layer = 1
    kc0, vc0 = w.k_cache.clone(), w.v_cache.clone()
    qa = w.q.clone()
    qk_norm_rope_store(qa, k.clone(), v, w.k_cache, w.v_cache, w.block_table, qn, kn, mc, ec, st, layer, cos, sin)
    oa, la = _outputs(w, mc)
    paged_attention(qa, w.k_cache, w.v_cache, w.block_table, mc, ec, st, layer, oa, la)
    torch.cuda.synchronize()
    kca, vca = w.k_cache.clone(), w.v_cache.clone()
    w.k_cache.copy_(kc0)
    w.v_cache.copy_(vc0)
    ob, lb = _outputs(w, mc)
    with pytest.raises(RuntimeError, match="block id outside the pool"):
        paged_attention_fused(w.q, k, v, w.k_cache, w.v_cache, w.block_table, qn, kn, mc, ec, st, layer, cos, sin,
                              ob, lb, validate=True)
    assert torch.equal(ob, oa) and torch.equal(lb, la)
    assert torch.equal(w.k_cache, kca) and torch.equal(w.v_cache, vca)


@pytest.mark.parametrize("q_len", [5, 1], ids=["verify", "decode"])
def test_fused_graph_replay_bit_identical(gpu, q_len):
    """A HIP graph of fused launches over every layer replays to the eager
    results bit for bit, replay after replay, with eager calls in between:
    o, lse and both pools (the new rows written again to the same slots)."""
    print(f"fused graph replay, q_len {q_len}", flush=True)
    w, mc, ec, st, cos, sin, k, v, qn, kn = _setup(gpu, QWEN3_8B, q_len, seed=81)
    layers = w.k_cache.shape[1]
    outs = [_outputs(w, mc) for _ in range(layers)]

    def calls():
        for layer in range(layers):
            paged_attention_fused(w.q, k, v, w.k_cache, w.v_cache, w.block_table, qn, kn, mc, ec, st, layer, cos,
                                  sin, outs[layer][0], outs[layer][1])

    calls()
    torch.cuda.synchronize()
    eager = [(o.clone(), l.clone()) for o, l in outs]
    kc, vc = w.k_cache.clone(), w.v_cache.clone()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            calls()
    torch.cuda.synchronize()
    for rep in range(3):
        for o, l in outs:
            o.zero_()
            l.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for layer in range(layers):
            assert torch.equal(outs[layer][0], eager[layer][0]), f"replay {rep} layer {layer} o"
            assert torch.equal(outs[layer][1], eager[layer][1]), f"replay {rep} layer {layer} lse"
        assert torch.equal(w.k_cache, kc) and torch.equal(w.v_cache, vc), f"replay {rep} pools"
        calls()  # eager work between replays
        torch.cuda.synchronize()


def test_fused_no_rows(gpu):
    """A forward with no decode rows returns without a launch and writes nothing."""
    mc = ModelConfig(QWEN3_8B)
    ec = EngineConfig(max_blocks_per_seq=4)
    cos, sin = rope_cache(128, 1e6, 8, gpu)
    st = build_infer_state([], [], [], mc, cos, sin, gpu)
    kc = torch.zeros((4, 1, 8, 16, 128), dtype=torch.float16, device=gpu)
    vc = torch.zeros_like(kc)
    q = torch.empty((0, 32, 128), dtype=torch.float16, device=gpu)
    kv = torch.empty((0, 8, 128), dtype=torch.float16, device=gpu)
    w = torch.ones(128, dtype=torch.float16, device=gpu)
    paged_attention_fused(q, kv, kv, kc, vc, torch.zeros((1, 4), dtype=torch.int32, device=gpu), w, w, mc, ec, st,
                          0, cos, sin, torch.empty_like(q))
    torch.cuda.synchronize()
    assert not kc.any() and not vc.any()
