"""Pins for the rest-of-layer oracle (CPU only): torch's own functional
routines, closed forms, known answers, and planted mistakes the pins reject."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle


def _h(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def test_fused_add_rmsnorm_matches_torch():
    rng = np.random.default_rng(0)
    x, r, w = _h(rng, 7, 4096), _h(rng, 7, 4096), (rng.random(4096) + 0.5).astype(np.float16)
    out, res = oracle.fused_add_rmsnorm(x, r, w, 1e-6)
    want_res = (torch.from_numpy(x) + torch.from_numpy(r)).numpy()  # torch's fp16 add
    np.testing.assert_array_equal(res, want_res)
    want = F.rms_norm(torch.from_numpy(res).double(), (4096,), torch.from_numpy(w).double(), 1e-6)
    np.testing.assert_allclose(out.astype(np.float64), want.numpy(), rtol=1e-3, atol=1e-3)


def test_fused_add_rmsnorm_constant_row_closed_form():
    x = np.full((2, 64), 1.5, np.float16)
    r = np.full((2, 64), -0.25, np.float16)
    w = np.linspace(0.5, 2, 64).astype(np.float16)
    out, res = oracle.fused_add_rmsnorm(x, r, w, 0.0)
    assert (res == np.float16(1.25)).all()
    np.testing.assert_array_equal(out, np.broadcast_to(w, out.shape))  # c / sqrt(c^2) = 1 -> the weights


def test_fused_add_rmsnorm_rejects_planted_mistake():
    rng = np.random.default_rng(1)
    x, r, w = _h(rng, 3, 256), _h(rng, 3, 256), np.ones(256, np.float16)
    out, res = oracle.fused_add_rmsnorm(x, r, w, 1e-6)
    wrong = oracle.rmsnorm_rows(x, w, 1e-6)  # norm of x alone
    assert np.abs(out.astype(np.float64) - wrong.astype(np.float64)).max() > 0.1


def test_silu_and_mul_matches_torch():
    rng = np.random.default_rng(2)
    x = _h(rng, 9, 2 * 768, scale=3.0)
    got = oracle.silu_and_mul(x)
    t = torch.from_numpy(x).double()
    gate = F.silu(t[:, 768:]).half().double()  # x * sigmoid(x): another float64 rounding path
    want = (t[:, :768] * gate).half().numpy()
    np.testing.assert_allclose(got.astype(np.float64), want.astype(np.float64), rtol=2e-3, atol=1e-6)
    assert (got == want).mean() > 0.995  # differences only where the fp16 rounding of silu is a near tie


def test_silu_and_mul_closed_forms_and_planted_swap():
    x = np.zeros((1, 16), np.float16)
    x[0, :8] = np.float16(3.0)      # up
    x[0, 8:12] = np.float16(0.0)    # gate 0 -> silu 0
    x[0, 12:] = np.float16(20.0)    # gate large -> silu(g) ~ g
    got = oracle.silu_and_mul(x)[0]
    assert (got[:4] == 0).all()
    np.testing.assert_allclose(got[4:].astype(np.float64), 60.0, rtol=1e-3)
    swapped = oracle.silu_and_mul(np.concatenate([x[:, 8:], x[:, :8]], axis=1))[0]
    assert not np.array_equal(swapped, got)


def test_argmax_first_known_answers_and_torch():
    rows = np.array([[1, 3, 3, 2], [-0.0, 0.0, -1, -2], [np.nan, 5, 6, 7], [1, np.nan, np.nan, 9],
                     [-np.inf, -np.inf, -5, -5]], np.float16)
    assert oracle.argmax_first(rows).tolist() == [1, 0, 0, 1, 2]
    assert torch.argmax(torch.from_numpy(rows), dim=1).tolist() == [1, 0, 0, 1, 2]
    rng = np.random.default_rng(3)
    big = _h(rng, 40, 5000)
    big[::3, 4999] = big[::3].max(axis=1) + 1  # maxima at the last column too
    np.testing.assert_array_equal(oracle.argmax_first(big), torch.argmax(torch.from_numpy(big), dim=1).numpy())


def test_last_token_indices_known_answer():
    # prompts of 3 and 5 tokens, then 2 decode rows -> [2, 7, 8, 9]
    assert oracle.last_token_indices([0, 3], [3, 5], 8, 10).tolist() == [2, 7, 8, 9]
    assert oracle.last_token_indices([], [], 0, 4).tolist() == [0, 1, 2, 3]


def test_lm_head_logits_and_post_layer_match_torch():
    rng = np.random.default_rng(4)
    x = _h(rng, 12, 256)
    w = _h(rng, 1000, 256, scale=0.1)
    fn = (rng.random(256) + 0.5).astype(np.float16)
    idx = [2, 5, 11]
    tokens, logits = oracle.post_layer(x, idx, fn, w, 1e-6)
    last = F.rms_norm(torch.from_numpy(x[idx]).double(), (256,), torch.from_numpy(fn).double(), 1e-6).half()
    want = F.linear(last.double(), torch.from_numpy(w).double()).half()
    np.testing.assert_allclose(logits.astype(np.float64), want.double().numpy(), rtol=2e-3, atol=2e-3)
    top2 = np.sort(want.double().numpy(), axis=1)[:, -2:]
    clear = top2[:, 1] - top2[:, 0] > 1e-2
    np.testing.assert_array_equal(tokens[clear], torch.argmax(want, dim=1).numpy()[clear])


def test_capi_argument_checks_without_gpu():
    """The rest-of-layer entry points reject bad shapes and pointers before
    any HIP call, and return success with nothing to do."""
    from nebulasd_amd import _lib

    if not _lib.LIB_PATH.exists():
        from nebulasd_amd.build import build

        build()
    lib = _lib.load()
    p = 0x10000  # 16-byte aligned, never dereferenced: every call below fails or has nothing to do
    cases = [
        (lambda: lib.nsd_fused_add_rmsnorm_inplace(p, p, p, 4, 8200, 1e-6, None), 2, "hidden=8200"),
        (lambda: lib.nsd_fused_add_rmsnorm_inplace(p, p, p, 4, 12, 1e-6, None), 2, "hidden=12"),
        (lambda: lib.nsd_fused_add_rmsnorm_inplace(None, p, p, 4, 64, 1e-6, None), 1, "null"),
        (lambda: lib.nsd_fused_add_rmsnorm_inplace(p + 2, p, p, 4, 64, 1e-6, None), 2, "aligned"),
        (lambda: lib.nsd_silu_and_mul_inplace(p, 4, 12, None), 2, "inter_dim=12"),
        (lambda: lib.nsd_silu_and_mul_inplace(None, 4, 16, None), 1, "null"),
        (lambda: lib.nsd_lm_head_argmax(p, p, 4, 100, 1000, p, p, None), 2, "hidden=100"),
        (lambda: lib.nsd_lm_head_argmax(p, p, 4, 128, 0, p, p, None), 1, "bad shape"),
        (lambda: lib.nsd_lm_head_argmax(p, p, 4, 128, 1000, None, p, None), 1, "null"),
        (lambda: lib.nsd_argmax_rows(p, 4, 0, p, None), 1, "bad shape"),
    ]
    for call, code, msg in cases:
        rc = call()
        assert rc == code and msg in _lib.last_error(), (rc, code, msg, _lib.last_error())
    assert lib.nsd_fused_add_rmsnorm_inplace(None, None, None, 0, 4096, 1e-6, None) == 0
    assert lib.nsd_silu_and_mul_inplace(None, 0, 16, None) == 0
    assert lib.nsd_lm_head_argmax(None, None, 0, 128, 10, None, None, None) == 0
    assert lib.nsd_argmax_rows(None, 0, 10, None, None) == 0



def _tiny_layer(rng, hidden=32, hq=4, hkv=2, d=16, inter=24):
    w = {"n_in": (rng.random(hidden) + 0.5).astype(np.float16),
         "wqkv": _h(rng, (hq + 2 * hkv) * d, hidden, scale=0.2),
         "q_norm": (rng.random(d) + 0.5).astype(np.float16),
         "k_norm": (rng.random(d) + 0.5).astype(np.float16),
         "wo": _h(rng, hidden, hq * d, scale=0.2),
         "n_post": (rng.random(hidden) + 0.5).astype(np.float16),
         "wug": _h(rng, 2 * inter, hidden, scale=0.2),
         "wd": _h(rng, hidden, inter, scale=0.2)}
    return w


def _tiny_state(rng, seq_lens, hkv=2, d=16, n_blocks=12):
    """Three sequences, one row each at the given lengths, their blocks a
    shuffled pool; caches filled with noise (the rows' own slots included)."""
    bt = rng.permutation(n_blocks).astype(np.int32).reshape(3, 4)
    kc = _h(rng, n_blocks, 2, hkv, 16, d)
    vc = _h(rng, n_blocks, 2, hkv, 16, d)
    cos, sin = oracle.rope_cache(d, 10000.0, 64)
    return bt, kc, vc, cos, sin, [0, 1, 2], list(seq_lens)


def test_decoder_layer_zero_projections_pass_the_residual():
    rng = np.random.default_rng(10)
    w = _tiny_layer(rng)
    w["wo"][:] = 0
    w["wd"][:] = 0
    bt, kc, vc, cos, sin, sids, slens = _tiny_state(rng, [5, 17, 40])
    x, res = _h(rng, 3, 32), _h(rng, 3, 32)
    y, r2 = oracle.decoder_layer(x, res, w, 1e-6, cos, sin, kc, vc, bt, sids, slens, 1, 4, 2)
    assert (y == 0).all()
    np.testing.assert_array_equal(r2, (torch.from_numpy(x) + torch.from_numpy(res)).numpy())


def test_decoder_layer_first_tokens_closed_form():
    """Every row is its sequence's first token: attention returns the row's
    own v (one kv head per GQA group of q heads), so the residual out is
    fp16(x + residual) + v repeated over the group times W_o; the V slot
    holds the v rows of the stacked projection (rows q | k | v), and a
    gate half of zeros zeroes the output (the gate is the second half)."""
    rng = np.random.default_rng(11)
    hidden, hq, hkv, d, inter = 32, 4, 2, 16, 24
    w = _tiny_layer(rng)
    bt, kc, vc, cos, sin, sids, slens = _tiny_state(rng, [1, 1, 1])
    x, res = _h(rng, 3, hidden), _h(rng, 3, hidden)
    w0 = {k: v.copy() for k, v in w.items()}
    w0["wug"][inter:] = 0
    kc0, vc0 = kc.copy(), vc.copy()
    y, r2 = oracle.decoder_layer(x, res, w0, 1e-6, cos, sin, kc0, vc0, bt, sids, slens, 0, hq, hkv)
    assert (y == 0).all()
    r1 = (x.astype(np.float32) + res.astype(np.float32)).astype(np.float16)
    xf = r1.astype(np.float64)
    h = (xf / np.sqrt((xf * xf).mean(1, keepdims=True) + 1e-6) * w["n_in"].astype(np.float64)).astype(np.float16)
    v = (h.astype(np.float64) @ w["wqkv"][(hq + hkv) * d:].astype(np.float64).T).astype(np.float16)
    v = v.reshape(3, hkv, d)
    for r in range(3):
        np.testing.assert_array_equal(vc0[bt[r, 0], 0, :, 0], v[r])
    o = np.repeat(v, hq // hkv, axis=1).reshape(3, hq * d)  # q head j reads kv head j // (hq / hkv)
    a = (o.astype(np.float64) @ w["wo"].astype(np.float64).T).astype(np.float16)
    want = (a.astype(np.float32) + r1.astype(np.float32)).astype(np.float16)
    np.testing.assert_array_equal(r2, want)
    # the same layer with the gate kept: a non-zero output, changed by a swap of the halves
    y1, _ = oracle.decoder_layer(x, res, w, 1e-6, cos, sin, kc.copy(), vc.copy(), bt, sids, slens, 0, hq, hkv)
    assert np.abs(y1.astype(np.float64)).max() > 0
    ws = dict(w, wug=np.concatenate([w["wug"][inter:], w["wug"][:inter]]))
    ys, _ = oracle.decoder_layer(x, res, ws, 1e-6, cos, sin, kc.copy(), vc.copy(), bt, sids, slens, 0, hq, hkv)
    assert not np.array_equal(ys, y1)


def test_decoder_layer_linear_matches_torch():
    rng = np.random.default_rng(12)
    x, wt = _h(rng, 5, 64), _h(rng, 48, 64, scale=0.1)
    want = F.linear(torch.from_numpy(x).double(), torch.from_numpy(wt).double()).half().numpy()
    np.testing.assert_array_equal(oracle.linear(x, wt), want)
