"""The speculative loop on random-init Qwen3-0.6B (draft) + Qwen3-8B (target).

A reduced run of the single-GPU speculative configuration: full model
shapes and depth 4, few short requests.  Attention layer calls sampled from
both models are checked against the oracle; the loop must finish every
request with exactly the requested number of tokens.
"""

from __future__ import annotations

import pytest

from nebulasd_amd.spec_loop import run
from spec_checks import make_checker

pytestmark = pytest.mark.gpu


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
