"""Bookkeeping of the speculative loop, on the CPU with scripted models.

``spec_loop.run`` is driven with a stand-in for ``RandomQwen3`` whose greedy
token is a fixed function of the tokens the model has stored so far (its
"KV cache": one token per position).  The stand-in asserts that every row
writes the next free position or rewrites an earlier one, so a forward that
skips a token fails at once, and the target's output is known in closed form:

* with the draft equal to the target, no proposal token is rejected, and
  the draft goes through its two-row reconcile step after fully accepted
  proposals (workers/draft/inputs.py:59-85);
* with a draft that deviates at some positions, proposals are accepted in
  part (speculative.py:122-156);
* with a draft that never agrees, every round commits the bonus token only;

and in every case each request's output is the target's greedy continuation.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nebulasd_amd import spec_loop
from nebulasd_amd.config import QWEN3_8B, ModelConfig

VOCAB = QWEN3_8B["vocab_size"]
SEED, PROMPT_LO, PROMPT_HI = 11, 5, 40


def next_token(seq: list) -> int:
    """The target's greedy token after `seq`: a function of its last three
    tokens and its length."""
    a, b, c = ([0, 0] + seq)[-3:]
    return (a * 7 + b * 131 + c * 8191 + len(seq) * 31 + 17) % VOCAB


class ScriptedModel:
    """Stands in for spec_loop.RandomQwen3: prefill/decode return each row's
    greedy token computed from the tokens stored at positions 0..row.  The
    draft (a model with fewer layers than the target) deviates according to
    ``mode``."""

    mode = "exact"  # "exact": draft = target; "some": wrong a third of the time; "never"

    def __init__(self, cfg, seq_blocks, device, seed, native=True):
        self.mc = ModelConfig(cfg)
        self.is_draft = self.mc.num_layers != QWEN3_8B["num_hidden_layers"]
        self.cache = {}
        self.check = None

    def _token(self, seq):
        t = next_token(seq)
        if self.is_draft and (self.mode == "never" or (self.mode == "some" and t % 3 == 0)):
            t = (t + 1) % VOCAB
        return t

    def prefill(self, seq_ids, prompts):
        out = []
        for r, p in zip(seq_ids, prompts):
            assert r not in self.cache, f"request {r} prefilled twice"
            self.cache[r] = list(p)
            out.append(self._token(self.cache[r]))
        return out

    def decode(self, seq_ids, seq_lens, tokens, as_tensor=False, lane=0):
        if isinstance(tokens, torch.Tensor):  # the loop passes device-resident proposals
            tokens = tokens.tolist()
        assert len(seq_ids) == len(seq_lens) == len(tokens)
        out = []
        for r, n, t in zip(seq_ids, seq_lens, tokens):
            c = self.cache[r]
            pos = n - 1
            assert 0 < pos <= len(c), f"request {r}: position {pos} past the {len(c)} stored tokens"
            del c[pos:]  # the row rewrites its position; later positions are stale
            c.append(int(t))
            out.append(self._token(c))
        return torch.tensor(out, dtype=torch.long) if as_tensor else out


def target_continuations(n_requests, new_tokens):
    """Every prompt's greedy continuation under the target, prompts drawn as run() draws them."""
    rng = np.random.default_rng(SEED)
    plens = rng.integers(PROMPT_LO, PROMPT_HI + 1, n_requests).tolist()
    outs = []
    for n in plens:
        seq = rng.integers(0, VOCAB, n).tolist()
        for _ in range(new_tokens):
            seq.append(next_token(seq))
        outs.append(seq[n:])
    return outs


def run_scripted(monkeypatch, mode, n_requests, new_tokens, share=False):
    monkeypatch.setattr(ScriptedModel, "mode", mode)
    monkeypatch.setattr(spec_loop, "RandomQwen3", ScriptedModel)
    res = spec_loop.run(n_requests=n_requests, prompt_lo=PROMPT_LO, prompt_hi=PROMPT_HI,
                        new_tokens=new_tokens, draft_batch=8, target_batch=3, depth=4, seed=SEED,
                        device="cpu", share_weights=share, return_outputs=True)
    assert res["outputs"] == target_continuations(n_requests, new_tokens)
    assert res["generated_tokens"] == n_requests * new_tokens
    return res


@pytest.mark.parametrize("share", [True, False])
def test_exact_draft_accepts_every_proposal(monkeypatch, share):
    # share=True builds the draft from the target's configuration (the GPU
    # run's shared-weight mode); share=False keeps the draft's own, exact here
    res = run_scripted(monkeypatch, "exact", 20, 23, share)
    assert res["partial_accepts"] == 0
    assert res["full_accepts"] > 0 and res["reconcile_groups"] > 0
    if not share:  # the draft model is the one that reconciles
        assert res["reconcile_groups"] <= res["full_accepts"]
    assert res["acceptance_rate"] >= 0.9  # below 1 only where the output limit clips


def test_deviating_draft_accepts_in_part(monkeypatch):
    res = run_scripted(monkeypatch, "some", 20, 23)
    assert res["partial_accepts"] > 0 and res["multi_token_appends"] > 0
    assert 0 < res["acceptance_rate"] < 1


def test_disagreeing_draft_commits_one_token_per_round(monkeypatch):
    res = run_scripted(monkeypatch, "never", 6, 9)
    assert res["accepted"] == 0 and res["reconcile_groups"] == 0
    assert res["multi_token_appends"] == 0
    assert res["rounds"] == 9 - 1  # the prefill makes the first token
