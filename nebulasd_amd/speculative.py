"""Verify-row construction and greedy acceptance (host side of the path).

The verify rows are what the attention kernels consume: a request with
anchor + K draft tokens becomes K+1 decode rows with one seq_id and
seq_lens ``logical+1 .. logical+K+1`` (swiftLLM/swiftllm/speculative.py:75-89;
nebulasd/src/nebulasd/workers/target/backend.py:101-110).
"""

from __future__ import annotations


def build_linear_verification_rows(prompt_len: int, output_token_ids, draft_token_ids):
    """(tokens, seq_lens) of one linear verify request (speculative.py:75-89)."""
    if not output_token_ids:
        raise ValueError("linear speculative verification requires an unstored anchor token")
    tokens = [output_token_ids[-1], *draft_token_ids]
    base = prompt_len + len(output_token_ids)
    return tokens, list(range(base, base + len(tokens)))


def expand_verify_rows(requests):
    """Flatten ``(seq_id, logical, anchor, proposal)`` requests into decode rows.

    Returns (input_ids, seq_ids, seq_lens), rows of a request contiguous
    (target/backend.py:101-110).
    """
    input_ids, seq_ids, seq_lens = [], [], []
    for seq_id, logical, anchor, proposal in requests:
        n = 1 + len(proposal)
        input_ids += [anchor, *proposal]
        seq_ids += [seq_id] * n
        seq_lens += list(range(logical + 1, logical + n + 1))
    return input_ids, seq_ids, seq_lens


def aggregate_max_lens_by_seq_id(seq_ids_list, seq_lens_list) -> dict:
    """Largest seq_len per seq_id (speculative.py:203-213)."""
    if len(seq_ids_list) != len(seq_lens_list):
        raise ValueError("seq_ids_list and seq_lens_list must have the same length")
    out: dict = {}
    for sid, sl in zip(seq_ids_list, seq_lens_list):
        if sl > out.get(sid, 0):
            out[sid] = sl
    return out


def compute_greedy_acceptance(draft_token_ids, posterior_token_ids, remaining_output_len=None,
                              stop_token_ids=()):
    """(tokens_to_append, num_accepted_draft_tokens) of greedy verification (speculative.py:122-156)."""
    if remaining_output_len is not None and remaining_output_len < 0:
        raise ValueError("remaining_output_len must be non-negative")
    k = len(draft_token_ids)
    if len(posterior_token_ids) < k + 1:
        raise ValueError("posterior_token_ids must contain K+1 tokens for K draft tokens")
    n = next((i for i in range(k) if posterior_token_ids[i] != draft_token_ids[i]), k)
    accepted = [*draft_token_ids[:n], posterior_token_ids[n]]
    if remaining_output_len is not None:
        accepted = accepted[:remaining_output_len]
    stops = {int(t) for t in stop_token_ids}
    if any(t < 0 for t in stops):
        raise ValueError("stop_token_ids must be non-negative")
    cut = next((i for i, t in enumerate(accepted) if t in stops), None)
    if cut is not None:
        accepted = accepted[:cut + 1]
    return accepted, min(n, len(accepted))
