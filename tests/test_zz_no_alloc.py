"""The allocation-free attention entry point against the workspace one.

``nsd_paged_attention_noalloc`` keeps the partials of segments cut into
several pieces (normalised O and log-sum-exp per slot) in a static device
array instead of a caller workspace.  Two calls in a row (the
second with fewer rows and shorter contexts, so it reuses what the first left
in the array) must give the workspace entry point's results, within the
path's tolerance (o 2e-3 abs + 1e-2 rel, LSE 1e-4), and match the oracle.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from helpers import ATOL_LSE, ATOL_O, RTOL_O, assert_close
from nebulasd_amd import _lib
from nebulasd_amd import plan as planmod
from nebulasd_amd.config import EngineConfig, ModelConfig
from nebulasd_amd.infer_state import build_infer_state, rope_cache
from nebulasd_amd.kernels import paged_attention
from nebulasd_amd.kernels._util import stream_of
from nebulasd_amd.workload import make_workload
from test_gpu_attention import check_against_oracle

pytestmark = pytest.mark.gpu


def noalloc_call(w, st, mc, layer, o, lse):
    plan = st.attn_plan
    _lib.call("nsd_paged_attention_noalloc",
              w.q.data_ptr(), o.data_ptr(), lse.data_ptr(), w.k_cache.data_ptr(),
              w.v_cache.data_ptr(), w.k_cache.shape[0], w.k_cache.shape[1], layer,
              mc.num_q_heads, mc.num_kv_heads, 128, 16, w.block_table.data_ptr(),
              w.block_table.shape[0], w.block_table.shape[1],
              plan.host.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
              plan.dev.data_ptr(), float(st.softmax_scale), None, stream_of(w.q))


@pytest.mark.parametrize("case", [
    # long contexts: segments cut across workgroups (partials and counters in use)
    dict(ctxs=[20000, 33, 9000, 1, 4000], q_len=5, seed=11),
    # the smaller second call: fewer rows, shorter contexts
    dict(ctxs=[700, 2500, 64], q_len=5, seed=12),
    # decode rows cut into two pieces per workgroup slot: the later ones
    # claimed through the counter at the start of the static array
    dict(ctxs=[20000, 33, 9000, 1, 4000], q_len=1, seed=13),
], ids=["first-long", "second-smaller", "third-decode-claimed"])
def test_noalloc_matches_workspace_entry(gpu, case, monkeypatch):
    if case["seed"] == 13:
        monkeypatch.setattr(planmod, "PIECES_PER_SLOT", 2.0)
    w = make_workload("target_verify", case["seed"], device=gpu, pool_blocks=4096, num_layers=2,
                      ctxs=case["ctxs"], q_len=case["q_len"])
    mc = ModelConfig(w.spec.model)
    ec = EngineConfig(block_size=16, max_blocks_per_seq=w.block_table.shape[1])
    cos, sin = rope_cache(128, mc.rope_theta, max(w.seq_lens) + 1, gpu)
    st = build_infer_state(w.seq_ids, w.seq_lens, [], mc, cos, sin, gpu)
    layer = 1
    o1 = torch.empty_like(w.q)
    l1 = torch.empty(w.q.shape[:2], dtype=torch.float32, device=gpu)
    paged_attention(w.q, w.k_cache, w.v_cache, w.block_table, mc, ec, st, layer, o1, l1,
                    validate=True)
    o2 = torch.full_like(w.q, float("nan"))
    l2 = torch.full_like(l1, float("nan"))
    noalloc_call(w, st, mc, layer, o2, l2)
    torch.cuda.synchronize()
    if case["seed"] == 11:
        assert int(st.attn_plan.host[_lib.PLAN_COMBINES]) > 0, "expected split segments"
    if case["seed"] == 13:
        assert int(st.attn_plan.host[_lib.PLAN_CLAIMED]) > 0, "expected claimed pieces"
    e_o = assert_close(o2.float().cpu().numpy(), o1.float().cpu().numpy(), ATOL_O, RTOL_O,
                       "noalloc o vs workspace entry")
    e_l = assert_close(l2.cpu().numpy(), l1.cpu().numpy(), ATOL_LSE, 0.0,
                       "noalloc lse vs workspace entry")
    print(f"noalloc vs workspace entry: max|do|={e_o:.2e} max|dlse|={e_l:.2e}", flush=True)
    check_against_oracle(w, layer, o2, l2, "noalloc")
