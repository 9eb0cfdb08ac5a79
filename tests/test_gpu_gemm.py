"""GPU parity of the split-k projection GEMM (nsd_linear_partials) and the
kernels that consume its partials.

- The fp16 projection (the splits summed in split order, one rounding)
  against the oracle's float64 GEMM rounded to fp16
  (``oracle.lm_head_logits``): within rtol 2e-3 / atol 1e-3 (fp32 sums in a
  different order can land one fp16 rounding away) and at least 95% equal;
  and against F.linear on the same GPU, within the same bound.
- The split partials' sum against the float64 GEMM within fp32 summation
  error (rtol 1e-4, atol 1e-4 x sqrt(k) scale).
- Rows past n_rows in the partials are never written (sentinel).
- The consumers take the partials where they would read the fp16
  projection: add-RMSNorm and the strided prologue over
  ``sum_partials``' output are bit-identical to the partial-reading entries.

Every case prints its name first.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from nebulasd_amd import _lib
from nebulasd_amd.config import QWEN3_0_6B, QWEN3_8B, EngineConfig, ModelConfig
from nebulasd_amd.infer_state import build_infer_state, rope_cache
from nebulasd_amd.kernels import (fused_add_rmsnorm_inplace, fused_add_rmsnorm_partials, linear, linear_partials,
                                  linear_splits, qk_norm_rope_store, qk_norm_rope_store_partials, sum_partials)
from nebulasd_amd.workload import make_workload

pytestmark = pytest.mark.gpu


def _randn(gpu, *shape, scale=1.0, seed=0):
    g = torch.Generator(device=gpu).manual_seed(seed)
    return (torch.randn(shape, device=gpu, generator=g) * scale).half()


# (rows, n_out, n_in): Qwen3-8B q/k/v, O, down at the verify batch (80), the
# Qwen3-0.6B draft's at 64 rows, one row, a full 128-row pass, a ragged row
# count, and narrow / short shapes (one 16-column tile, one k step).
SHAPES = [(80, 6144, 4096), (80, 4096, 4096), (80, 4096, 12288), (64, 4096, 1024), (64, 1024, 2048),
          (64, 1024, 3072), (1, 4096, 4096), (128, 4096, 4096), (37, 1024, 3072), (5, 48, 256), (3, 16, 128)]


@pytest.mark.parametrize("rows,n,k", SHAPES, ids=[f"{r}x{n}x{k}" for r, n, k in SHAPES])
def test_linear_matches_oracle(gpu, rows, n, k):
    print(f"linear {rows} x {n} x {k}", flush=True)
    x = _randn(gpu, rows, k, seed=21)
    w = _randn(gpu, n, k, seed=22, scale=0.03)
    splits = linear_splits(rows, n, k)
    assert 1 <= splits <= 8
    # partials [splits][rows][n] followed by a sentinel row
    part_c = torch.full((splits * rows * n + n,), 7.0, dtype=torch.float32, device=gpu)
    got_part = linear_partials(x, w, part_c[:splits * rows * n].view(splits, rows, n))
    y = sum_partials(got_part)
    torch.cuda.synchronize()
    assert bool((part_c[splits * rows * n:] == 7.0).all()), "the kernel wrote past the partials"
    ref64 = x.double().cpu() @ w.double().cpu().T
    tot = got_part.double().sum(0).cpu()
    np.testing.assert_allclose(tot.numpy(), ref64.numpy(), rtol=1e-4, atol=1e-4 * max(1.0, (k / 128) ** 0.5))
    want = oracle.lm_head_logits(x.cpu().numpy(), w.cpu().numpy()).astype(np.float64)
    got = y.float().cpu().numpy().astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=2e-3, atol=1e-3)
    exact = float(np.mean(got == want))
    assert exact >= 0.95, exact
    lib = F.linear(x, w).float().cpu().numpy()
    np.testing.assert_allclose(got, lib, rtol=2e-3, atol=1e-3)
    # the convenience entry is the same computation
    assert torch.equal(linear(x, w), y)
    print(f"  {splits} splits; exact vs oracle {exact:.4f}, vs F.linear {float(np.mean(got == lib)):.4f}",
          flush=True)


def test_linear_rejects_bad_shapes(gpu):
    x = torch.zeros(2, 256, dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.NativeLibraryError, match="n_out=40"):
        linear_partials(x, torch.zeros(40, 256, dtype=torch.float16, device=gpu))
    x = torch.zeros(2, 200, dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.NativeLibraryError, match="n_in=200"):
        linear_partials(x, torch.zeros(32, 200, dtype=torch.float16, device=gpu))
    x = torch.zeros(129, 256, dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.NativeLibraryError, match="n_rows=129"):
        linear_partials(x, torch.zeros(32, 256, dtype=torch.float16, device=gpu))


@pytest.mark.parametrize("rows,hidden,k", [(80, 4096, 4096), (64, 1024, 3072), (7, 4096, 12288)])
def test_add_rmsnorm_over_partials_is_bit_identical(gpu, rows, hidden, k):
    """fused_add_rmsnorm_partials == sum_partials then fused_add_rmsnorm_inplace."""
    print(f"add-rmsnorm over partials {rows} x {hidden} (k {k})", flush=True)
    part = linear_partials(_randn(gpu, rows, k, seed=31), _randn(gpu, hidden, k, seed=32, scale=0.03))
    res = _randn(gpu, rows, hidden, seed=33, scale=2.0)
    wt = (torch.rand(hidden, device=gpu) + 0.5).half()
    x_ref, r_ref = sum_partials(part), res.clone()
    fused_add_rmsnorm_inplace(x_ref, r_ref, wt, 1e-6)
    out = torch.full_like(res, 3.0)
    fused_add_rmsnorm_partials(part, out, res, wt, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(res, r_ref) and torch.equal(out, x_ref)


@pytest.mark.parametrize("name,model", [("draft_decode", QWEN3_0_6B), ("target_verify", QWEN3_8B)])
def test_prologue_over_partials_is_bit_identical(gpu, name, model):
    """qk_norm_rope_store_partials == sum_partials then the strided prologue:
    q_out and both cache pools bit-identical."""
    print(f"prologue over partials, {name}", flush=True)
    w = make_workload(name, 4, device=gpu)
    mc, ec = ModelConfig(model), EngineConfig(max_blocks_per_seq=w.block_table.shape[1])
    cos_c, sin_c = rope_cache(128, mc.rope_theta, 40960, gpu)
    st = build_infer_state(w.seq_ids, w.seq_lens, [], mc, cos_c, sin_c, gpu)
    hq, hkv, d, hidden = mc.num_q_heads, mc.num_kv_heads, 128, mc.hidden_size
    x = _randn(gpu, w.rows, hidden, seed=41)
    wqkv = _randn(gpu, (hq + 2 * hkv) * d, hidden, seed=42, scale=0.03)
    part = linear_partials(x, wqkv)
    qkv = sum_partials(part)
    qw = (torch.rand(d, device=gpu) + 0.5).half()
    kw = (torch.rand(d, device=gpu) + 0.5).half()
    layer = 2
    kpool, vpool = w.k_cache.clone(), w.v_cache.clone()
    q_ref = torch.empty((w.rows, hq, d), dtype=torch.float16, device=gpu)
    qkv3 = qkv.view(w.rows, hq + 2 * hkv, d)
    qk_norm_rope_store(qkv3[:, :hq], qkv3[:, hq:hq + hkv], qkv3[:, hq + hkv:], kpool, vpool, w.block_table, qw, kw,
                       mc, ec, st, layer, cos_c, sin_c, validate=True, q_out=q_ref)
    q_out = torch.full_like(q_ref, 5.0)
    qk_norm_rope_store_partials(part, q_out, w.k_cache, w.v_cache, w.block_table, qw, kw, mc, ec, st, layer,
                                cos_c, sin_c, validate=True)
    torch.cuda.synchronize()
    assert torch.equal(q_out, q_ref)
    assert torch.equal(w.k_cache, kpool) and torch.equal(w.v_cache, vpool)
