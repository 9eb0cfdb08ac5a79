"""The speculative loop on random-init Qwen3-0.6B (draft) + Qwen3-8B (target).

Runs the full single-GPU speculative configuration (512 requests x 128
generated tokens, draft batch 64, target batch 16, depth 4, prompts
U[128, 1024]), the same shapes with fewer requests and tokens, a reduced run,
and a run in which the draft holds the target's weights, so that proposals
are accepted and the multi-token append and the draft's two-row reconcile
step execute.
Attention layer calls sampled from both models are checked against the
oracle; every request must finish with exactly the requested tokens.
"""

from __future__ import annotations

import pytest

from nebulasd_amd.spec_loop import run
from spec_checks import make_checker

pytestmark = pytest.mark.gpu


def progress(msg):
    print(msg, flush=True)


def test_speculative_loop_small(gpu):
    results = []
    res = run(n_requests=6, prompt_lo=40, prompt_hi=90, new_tokens=10, draft_batch=4,
              target_batch=2, depth=4, seed=3, check_every=3, make_check=make_checker(results),
              device=gpu)
    print({k: v for k, v in res.items()}, flush=True)
    assert res["generated_tokens"] == 6 * 10
    assert res["target_forwards"] > 0 and res["draft_forwards"] > 0
    assert results and all(r["ok"] for r in results), results
    # both models' calls were checked, verify rows (q_len 5) included
    assert {r["layers"] for r in results} == {28, 36}
    assert max(r["max_q_len"] for r in results if r["layers"] == 36) == 5


def test_speculative_loop_full_configuration(gpu):
    """The full single-GPU speculative configuration: 512 requests, prompts
    U[128, 1024], 128 generated tokens each, draft batch 64, target batch 16,
    depth 4, greedy.  Every 251st forward (a stride co-prime with the eight
    forwards of a draft group, so draft decodes and target verifies are both
    sampled) hands its mid-depth attention layer call to the oracle; every
    request ends with exactly 128 tokens."""
    results = []
    res = run(n_requests=512, new_tokens=128, draft_batch=64, target_batch=16, depth=4, seed=0,
              check_every=251, make_check=make_checker(results), device=gpu, return_outputs=True)
    outputs = res.pop("outputs")
    print({k: v for k, v in res.items()}, flush=True)
    assert res["requests"] == 512 and res["generated_tokens"] == 512 * 128
    assert len(outputs) == 512 and all(len(o) == 128 for o in outputs)
    assert res["rounds"] <= 127 and res["target_forwards"] > 0 and res["draft_forwards"] > 0
    assert len(results) == res["attention_checks"] >= 30
    assert all(r["ok"] for r in results), [r for r in results if not r["ok"]]
    assert {r["layers"] for r in results} == {28, 36}
    assert max(r["rows"] for r in results if r["layers"] == 36) == 16 * 5
    assert max(r["rows"] for r in results if r["layers"] == 28) == 64


def test_speculative_loop_config_shape(gpu):
    """Draft batch 64 / target batch 16 / depth 4 over 64 prompts of U[128, 1024] tokens."""
    results = []
    res = run(n_requests=64, prompt_lo=128, prompt_hi=1024, new_tokens=16, draft_batch=64,
              target_batch=16, depth=4, seed=5, check_every=5, make_check=make_checker(results),
              device=gpu, log=progress)
    print({k: v for k, v in res.items()}, flush=True)
    assert res["generated_tokens"] == 64 * 16
    assert results and all(r["ok"] for r in results), [r for r in results if not r["ok"]]
    assert {r["layers"] for r in results} == {28, 36}
    draft_rows = {r["rows"] for r in results if r["layers"] == 28}
    target_rows = {r["rows"] for r in results if r["layers"] == 36}
    assert max(draft_rows) == 64 and max(target_rows) == 16 * 5
    assert max(r["max_seq_len"] for r in results) > 900


def test_speculative_loop_shared_weights_accepts(gpu):
    """The draft holds the target's weights: proposals are accepted, the
    draft reconciles after fully accepted proposals, and the sampled calls
    (two-row draft groups among them) still match the oracle."""
    results = []
    res = run(n_requests=64, prompt_lo=128, prompt_hi=1024, new_tokens=16, draft_batch=64,
              target_batch=16, depth=4, seed=6, check_every=2, make_check=make_checker(results),
              device=gpu, share_weights=True, log=progress)
    print({k: v for k, v in res.items()}, flush=True)
    assert res["generated_tokens"] == 64 * 16
    assert res["acceptance_rate"] > 0.5
    assert res["full_accepts"] > 0 and res["reconcile_groups"] > 0
    assert res["multi_token_appends"] > 0
    assert results and all(r["ok"] for r in results), [r for r in results if not r["ok"]]
    # a checked draft forward held two-row reconcile groups
    assert any(r["max_q_len"] == 2 and r["rows"] < 5 * 64 for r in results)


def test_speculative_loop_pipelined_equals_synchronous(gpu):
    """Forwards enqueued back to back with device-resident proposals, with
    the draft and target on two streams (two draft groups per round, so a
    group's draft forwards run beside the previous group's verifies), a
    group's target batches on two streams or one, and all on one stream, give the same tokens and counters as waiting for every forward
    (deterministic kernels), with proposals accepted and two-row reconcile
    groups present."""
    kw = dict(n_requests=24, prompt_lo=64, prompt_hi=400, new_tokens=12, draft_batch=16, target_batch=8,
              depth=4, seed=8, device=gpu, share_weights=True, return_outputs=True)
    a = run(**kw)
    b = run(**kw, sync_each_forward=True)
    c = run(**kw, overlap=False)
    d = run(**kw, target_streams=1)
    print({k: v for k, v in a.items() if k != "outputs"}, flush=True)
    assert a["reconcile_groups"] > 0 and a["accepted"] > 0
    assert a["outputs"] == b["outputs"] == c["outputs"] == d["outputs"]
    for key in ("accepted", "proposed", "reconcile_groups", "full_accepts", "partial_accepts", "rounds",
                "target_forwards", "draft_forwards"):
        assert a[key] == b[key] == c[key] == d[key], key


def test_prefill_ignore_kvcache_leaves_cache(gpu):
    """A prefill forward with ignore_kvcache writes no cache slot and returns
    the same tokens (prefill attention reads k/v directly), as the reference's
    layer skips store_kvcache then (transformer_layer.py:133)."""
    import torch

    from nebulasd_amd.config import QWEN3_0_6B
    from nebulasd_amd.spec_loop import RandomQwen3

    m = RandomQwen3(QWEN3_0_6B, [4, 4], gpu, seed=9)
    prompts = [list(range(100, 140)), list(range(7, 40))]
    t_ignored = m.prefill([0, 1], prompts, ignore_kvcache=True)
    torch.cuda.synchronize()
    assert int(m.k_cache.count_nonzero()) == 0 and int(m.v_cache.count_nonzero()) == 0
    t_stored = m.prefill([0, 1], prompts)
    torch.cuda.synchronize()
    assert t_ignored == t_stored
    assert int(m.k_cache.count_nonzero()) > 0


def test_prologue_refuses_ignore_kvcache_with_decode_rows(gpu):
    import types

    import torch

    from nebulasd_amd.config import QWEN3_0_6B, EngineConfig, ModelConfig
    from nebulasd_amd.infer_state import rope_cache
    from nebulasd_amd.kernels import qk_norm_rope_store

    mc = ModelConfig(QWEN3_0_6B)
    cos, sin = rope_cache(128, mc.rope_theta, 64, gpu)
    st = types.SimpleNamespace(num_prefill_seqs=0, num_decoding_seqs=1, ignore_kvcache=True,
                               seq_ids=torch.zeros(1, dtype=torch.int32, device=gpu),
                               decoding_seq_lens=torch.full((1,), 5, dtype=torch.int32, device=gpu))
    kc = torch.zeros((4, mc.num_layers, 8, 16, 128), dtype=torch.float16, device=gpu)
    q = torch.zeros((1, 16, 128), dtype=torch.float16, device=gpu)
    k = torch.zeros((1, 8, 128), dtype=torch.float16, device=gpu)
    with pytest.raises(ValueError, match="ignore_kvcache"):
        qk_norm_rope_store(q, k, k.clone(), kc, kc.clone(), torch.zeros((1, 4), dtype=torch.int32, device=gpu),
                           None, None, mc, EngineConfig(max_blocks_per_seq=4), st, 0, cos, sin)
    assert int(kc.count_nonzero()) == 0
