"""GPU parity of the prologue kernels (QK-RMSNorm, RoPE, KV store) against the oracle.

KV placement is checked bit-exactly over the whole pool: the expected pool is
the old pool with the oracle's slots (closed-form offsets) overwritten.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from nebulasd_amd.config import QWEN3_0_6B, QWEN3_8B, EngineConfig, ModelConfig
from nebulasd_amd.infer_state import build_infer_state, rope_cache
from nebulasd_amd.kernels import (qk_norm_rope_store, rmsnorm_inplace, rotary_embedding_inplace,
                                  store_kvcache)
from nebulasd_amd.workload import make_workload

pytestmark = pytest.mark.gpu


def ulp_close(got, want, what, ulps=1):
    """fp16 results within `ulps` units in the last place of the expected value."""
    g = np.asarray(got, np.float64)
    wv = np.asarray(want, np.float16)
    spacing = np.spacing(np.abs(wv)).astype(np.float64)
    bad = np.abs(g - wv.astype(np.float64)) > ulps * spacing + 1e-7
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} values off by more than {ulps} ulp"


def expected_pool(cache: torch.Tensor, offsets: np.ndarray, rows: torch.Tensor) -> torch.Tensor:
    """Old pool with rows [n, d] written at flat element offsets [n] (on the GPU)."""
    d = rows.shape[-1]
    exp = cache.clone()
    idx = torch.from_numpy(offsets).to(cache.device)[:, None] + torch.arange(d, device=cache.device)
    exp.view(-1)[idx.reshape(-1)] = rows.reshape(-1)
    return exp


def slot_offsets(bt, seq_ids, seq_lens, layer, L, hkv):
    return np.array([oracle.kv_slot_offset(bt, s, n - 1, layer, h, L, hkv, 16, 128)
                     for s, n in zip(seq_ids, seq_lens) for h in range(hkv)], dtype=np.int64)


def _state(w, mc, device, prefill=()):
    cos, sin = rope_cache(128, mc.rope_theta, max(w.seq_lens) + 1, device)
    return build_infer_state(list(range(len(prefill))) + w.seq_ids if prefill else w.seq_ids,
                             w.seq_lens, list(prefill), mc, cos, sin, device), cos, sin


def test_store_kvcache_full_pool_bit_exact(gpu):
    """Qwen3-8B pool of 24,576 blocks (14.5 G elements: 64-bit offsets)."""
    w = make_workload("target_verify", 0, device=gpu)
    mc, ec = ModelConfig(w.spec.model), EngineConfig(max_blocks_per_seq=w.block_table.shape[1])
    st, _, _ = _state(w, mc, gpu)
    layer = 35
    k = torch.randn((w.rows, 8, 128), device=gpu).half()
    v = torch.randn((w.rows, 8, 128), device=gpu).half()
    offs = slot_offsets(w.block_table.cpu().numpy(), w.seq_ids, w.seq_lens, layer, 36, 8)
    want_k = expected_pool(w.k_cache, offs, k)
    want_v = expected_pool(w.v_cache, offs, v)
    store_kvcache(k, v, w.k_cache, w.v_cache, w.block_table, mc, ec, st, layer, validate=True)
    assert torch.equal(w.k_cache, want_k)
    assert torch.equal(w.v_cache, want_v)


def test_store_kvcache_prefill_and_decode(gpu):
    """Mixed forward: two prefill sequences then decode rows (kvcache_mgmt.py:104-122)."""
    w = make_workload("draft_decode", 1, device=gpu, pool_blocks=4096, num_layers=2,
                      ctxs=[40, 600, 17])
    mc, ec = ModelConfig(QWEN3_0_6B), EngineConfig(max_blocks_per_seq=w.block_table.shape[1])
    prefill = [37, 70]
    bt_np = w.block_table.cpu().numpy()
    # prefill sequences use block-table rows 0 and 1 (their own rows of the table)
    st, _, _ = _state(w, mc, gpu, prefill=prefill)
    n_tok = sum(prefill) + w.rows
    k = torch.randn((n_tok, 8, 128), device=gpu).half()
    v = torch.randn((n_tok, 8, 128), device=gpu).half()
    kc0, vc0 = w.k_cache.clone(), w.v_cache.clone()
    store_kvcache(k, v, w.k_cache, w.v_cache, w.block_table, mc, ec, st, 1, validate=True)
    # oracle on the touched blocks only
    ids = sorted({int(b) for b in bt_np[:3].reshape(-1)})
    remap = {b: i for i, b in enumerate(ids)}
    bt_s = np.vectorize(remap.get)(bt_np[:3])
    sel = torch.tensor(ids, device=gpu)
    ko, vo = kc0[sel].cpu().numpy(), vc0[sel].cpu().numpy()
    kn, vn = k.cpu().numpy(), v.cpu().numpy()
    oracle.store_kvcache_prefill(kn, vn, ko, vo, bt_s, [0, 1], prefill, 1)
    oracle.store_kvcache(kn[sum(prefill):], vn[sum(prefill):], ko, vo, bt_s, w.seq_ids,
                         w.seq_lens, 1)
    assert np.array_equal(w.k_cache[sel].cpu().numpy().view(np.uint16), ko.view(np.uint16))
    assert np.array_equal(w.v_cache[sel].cpu().numpy().view(np.uint16), vo.view(np.uint16))
    # nothing outside those blocks changed
    mask = torch.ones(w.k_cache.shape[0], dtype=torch.bool, device=gpu)
    mask[sel] = False
    assert torch.equal(w.k_cache[mask], kc0[mask]) and torch.equal(w.v_cache[mask], vc0[mask])


def test_rmsnorm_matches_oracle(gpu):
    g = torch.Generator(device=gpu).manual_seed(3)
    x = (torch.randn((777, 128), device=gpu, generator=g) * 3).half()
    w = (torch.rand(128, device=gpu, generator=g) + 0.5).half()
    want = oracle.rmsnorm(x.cpu().numpy(), w.cpu().numpy(), 1e-6)
    rmsnorm_inplace(x, w, 1e-6)
    ulp_close(x.cpu().numpy(), want, "rmsnorm")


def test_rope_matches_oracle(gpu):
    g = torch.Generator(device=gpu).manual_seed(4)
    cos_c, sin_c = rope_cache(128, 1e6, 40960, gpu)
    pos = torch.randint(0, 40960, (300,), device=gpu, generator=g)
    q = torch.randn((300, 32, 128), device=gpu, generator=g).half()
    k = torch.randn((300, 8, 128), device=gpu, generator=g).half()

    class S:
        position_cos = cos_c[pos].contiguous()
        position_sin = sin_c[pos].contiguous()

    wq = oracle.rope(q.cpu().numpy(), S.position_cos.cpu().numpy(), S.position_sin.cpu().numpy())
    wk = oracle.rope(k.cpu().numpy(), S.position_cos.cpu().numpy(), S.position_sin.cpu().numpy())
    rotary_embedding_inplace(q, k, S)
    ulp_close(q.cpu().numpy(), wq, "rope q")
    ulp_close(k.cpu().numpy(), wk, "rope k")


def test_rope_table_matches_oracle(gpu):
    """The table is built in fp32 (model.py:242-252): the argument t*inv_freq
    carries up to ~2 fp32 roundings of |t| (and pow may differ by an ulp
    between libraries), so the bound grows with the position."""
    n = 40960
    cos_c, sin_c = rope_cache(128, 1e6, n, gpu)
    oc, os_ = oracle.rope_cache(128, 1e6, n)
    t = np.arange(n, dtype=np.float64)[:, None]
    bound = 2.0 ** -11 + t * 2.0 ** -21
    for got, want, what in ((cos_c, oc, "cos"), (sin_c, os_, "sin")):
        err = np.abs(got.cpu().numpy().astype(np.float64) - want.astype(np.float64))
        assert (err <= bound).all(), f"{what} table: max excess {(err - bound).max():.3g}"


@pytest.mark.parametrize("name,model", [("draft_decode", QWEN3_0_6B), ("target_verify", QWEN3_8B),
                                        ("target_verify", dict(QWEN3_8B, num_attention_heads=40))],
                         ids=["0.6b", "8b", "40q-8kv"])
def test_fused_prologue_matches_oracle(gpu, name, model):
    """QK-RMSNorm (gamma ~ U[0.5,1.5]) + RoPE (theta 1e6) + KV store for the new rows."""
    w = make_workload(name, 2, device=gpu)
    mc, ec = ModelConfig(model), EngineConfig(max_blocks_per_seq=w.block_table.shape[1])
    st, _, _ = _state(w, mc, gpu)
    cos_c, sin_c = rope_cache(128, mc.rope_theta, 40960, gpu)
    g = torch.Generator(device=gpu).manual_seed(5)
    hq, hkv = mc.num_q_heads, mc.num_kv_heads
    q = torch.randn((w.rows, hq, 128), device=gpu, generator=g).half()
    k = torch.randn((w.rows, hkv, 128), device=gpu, generator=g).half()
    v = torch.randn((w.rows, hkv, 128), device=gpu, generator=g).half()
    qw = (torch.rand(128, device=gpu, generator=g) + 0.5).half()
    kw = (torch.rand(128, device=gpu, generator=g) + 0.5).half()
    layer = mc.num_layers - 1
    # oracle on host copies
    bt_np = w.block_table.cpu().numpy()
    pos = np.asarray(w.seq_lens) - 1
    qn, kn = oracle.rmsnorm(q.cpu().numpy(), qw.cpu().numpy(), 1e-6), oracle.rmsnorm(
        k.cpu().numpy(), kw.cpu().numpy(), 1e-6)
    oc, os_ = cos_c.cpu().numpy(), sin_c.cpu().numpy()
    want_q, want_k = oracle.rope(qn, oc[pos], os_[pos]), oracle.rope(kn, oc[pos], os_[pos])
    offs = slot_offsets(bt_np, w.seq_ids, w.seq_lens, layer, mc.num_layers, hkv)
    kc0 = w.k_cache.clone()
    want_v = expected_pool(w.v_cache, offs, v)  # V is a bit-exact copy
    qk_norm_rope_store(q, k, v, w.k_cache, w.v_cache, w.block_table, qw, kw, mc, ec, st, layer,
                       cos_c, sin_c, validate=True)
    torch.cuda.synchronize()
    # a 1-ulp flip of the fp16 norm output can move the rotated value by ~2 ulp
    np.testing.assert_allclose(q.cpu().numpy().astype(np.float64), want_q.astype(np.float64),
                               atol=1e-3, rtol=2e-3, err_msg="fused q")
    np.testing.assert_allclose(k.cpu().numpy().astype(np.float64), want_k.astype(np.float64),
                               atol=1e-3, rtol=2e-3, err_msg="fused k")
    # placement: K pool = old pool with the kernel's own rotated k rows at the oracle's slots
    assert torch.equal(w.k_cache, expected_pool(kc0, offs, k))
    assert torch.equal(w.v_cache, want_v)


@pytest.mark.parametrize("name,model", [("draft_decode", QWEN3_0_6B), ("target_verify", QWEN3_8B)])
def test_strided_prologue_equals_contiguous(gpu, name, model):
    """q/k/v as row-strided slices of one fused projection output: the q
    written to q_out, the rotated k (in place) and both cache pools are
    bit-identical to the contiguous entry point's on copies; q is untouched."""
    w = make_workload(name, 3, device=gpu)
    mc, ec = ModelConfig(model), EngineConfig(max_blocks_per_seq=w.block_table.shape[1])
    st, _, _ = _state(w, mc, gpu)
    cos_c, sin_c = rope_cache(128, mc.rope_theta, 40960, gpu)
    g = torch.Generator(device=gpu).manual_seed(6)
    hq, hkv, d = mc.num_q_heads, mc.num_kv_heads, 128
    qkv = torch.randn((w.rows, (hq + 2 * hkv) * d), device=gpu, generator=g).half()
    q = qkv[:, :hq * d].view(w.rows, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(w.rows, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(w.rows, hkv, d)
    qc, kc_, vc_ = q.contiguous(), k.contiguous(), v.contiguous()
    q_in = q.clone()
    qw = (torch.rand(d, device=gpu, generator=g) + 0.5).half()
    kw = (torch.rand(d, device=gpu, generator=g) + 0.5).half()
    layer = 1
    kpool, vpool = w.k_cache.clone(), w.v_cache.clone()
    qk_norm_rope_store(qc, kc_, vc_, kpool, vpool, w.block_table, qw, kw, mc, ec, st, layer, cos_c, sin_c,
                       validate=True)
    q_out = torch.empty_like(qc)
    qk_norm_rope_store(q, k, v, w.k_cache, w.v_cache, w.block_table, qw, kw, mc, ec, st, layer, cos_c, sin_c,
                       validate=True, q_out=q_out)
    torch.cuda.synchronize()
    assert torch.equal(q_out, qc)
    assert torch.equal(k, kc_)
    assert torch.equal(q, q_in)
    assert torch.equal(w.k_cache, kpool) and torch.equal(w.v_cache, vpool)
    with pytest.raises(ValueError, match="q_out"):
        qk_norm_rope_store(q, k, v, w.k_cache, w.v_cache, w.block_table, qw, kw, mc, ec, st, layer, cos_c, sin_c)


def test_fused_equals_unfused(gpu):
    """One launch gives the result of rmsnorm -> rmsnorm -> rope -> store (to fp16 rounding),
    and each path's cache slots hold exactly the k/v that path produced."""
    w = make_workload("target_verify", 3, device=gpu, pool_blocks=2048, num_layers=2,
                      ctxs=[100, 2000, 5])
    mc, ec = ModelConfig(QWEN3_8B), EngineConfig(max_blocks_per_seq=w.block_table.shape[1])
    st, cos_c, sin_c = _state(w, mc, gpu)
    g = torch.Generator(device=gpu).manual_seed(6)
    q = torch.randn((w.rows, 32, 128), device=gpu, generator=g).half()
    k = torch.randn((w.rows, 8, 128), device=gpu, generator=g).half()
    v = torch.randn((w.rows, 8, 128), device=gpu, generator=g).half()
    qw = (torch.rand(128, device=gpu, generator=g) + 0.5).half()
    kw = (torch.rand(128, device=gpu, generator=g) + 0.5).half()
    q2, k2 = q.clone(), k.clone()
    kc2, vc2 = w.k_cache.clone(), w.v_cache.clone()
    qk_norm_rope_store(q, k, v, w.k_cache, w.v_cache, w.block_table, qw, kw, mc, ec, st, 1,
                       cos_c, sin_c)
    rmsnorm_inplace(q2.view(-1, 128), qw, mc.rms_norm_eps)
    rmsnorm_inplace(k2.view(-1, 128), kw, mc.rms_norm_eps)
    rotary_embedding_inplace(q2, k2, st)
    store_kvcache(k2, v, kc2, vc2, w.block_table, mc, ec, st, 1)
    for a, b, what in ((q, q2, "q"), (k, k2, "k")):
        diff = (a.float() - b.float()).abs()
        n_diff = int((a != b).sum())
        print(f"fused vs unfused {what}: {n_diff} differing of {a.numel()}, max |d|={diff.max().item():.3g}",
              flush=True)
        # both paths are fp32 math with fp16 stores; a rare 1-ulp flip of the fp16 norm
        # output is amplified relative to a rotated value that nearly cancels, so the
        # bound is absolute at the scale of the inputs (|x| <~ 8: fp16 ulp <= 2^-8)
        np.testing.assert_allclose(a.float().cpu().numpy(), b.float().cpu().numpy(),
                                   atol=2 ** -8, rtol=2 ** -9, err_msg=f"fused vs unfused {what}")
    # the cache holds exactly the k/v each path produced
    bt_np = w.block_table.cpu().numpy()
    offs = torch.from_numpy(slot_offsets(bt_np, w.seq_ids, w.seq_lens, 1, 2, 8)).to(gpu)
    idx = offs[:, None] + torch.arange(128, device=gpu)
    assert torch.equal(w.k_cache.view(-1)[idx], k.reshape(-1, 128))
    assert torch.equal(kc2.view(-1)[idx], k2.reshape(-1, 128))
    assert torch.equal(w.v_cache, vc2)


def test_prologue_bad_seq_is_flagged(gpu):
    w = make_workload("target_verify", 7, device=gpu, pool_blocks=256, num_layers=2, ctxs=[10, 20])
    mc, ec = ModelConfig(QWEN3_8B), EngineConfig(max_blocks_per_seq=w.block_table.shape[1])
    st, cos_c, sin_c = _state(w, mc, gpu)
    st.seq_ids[1] = 50  # outside the block table
    k = torch.randn((w.rows, 8, 128), device=gpu).half()
    with pytest.raises(RuntimeError, match="outside the block table"):
        store_kvcache(k, k.clone(), w.k_cache, w.v_cache, w.block_table, mc, ec, st, 0,
                      validate=True)
