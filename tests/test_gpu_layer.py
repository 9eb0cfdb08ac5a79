"""GPU parity of the rest-of-layer kernels (fused add-RMSNorm, SiLU-and-mul,
the fused up/gate projection + SiLU-and-mul, lm_head + argmax, argmax)
against the numpy oracle, and against the reference's own torch
formulation on the same GPU.

Every case prints its name first (pytest -v) so a failing GPU step is named.
Tolerances: residual and argmax over given logits bit-exact; normalised and
activated values within 1e-3 (fp16 output, one rounding apart); the fused
up/gate + SiLU-and-mul within rtol 4e-3 / atol 2e-3 and at least 90% bit-equal
(its up or gate value may sit one fp16 rounding from the float64 sum's, which
the SiLU and the product carry); lm_head
argmax equal to the float64 reference's except where the two candidates'
float64 logits are within 2e-3 of each other (accumulation order decides a
near tie).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from nebulasd_amd import _lib
from nebulasd_amd.kernels import fused_add_rmsnorm_inplace, silu_and_mul_inplace, up_gate_silu_and_mul
from nebulasd_amd.kernels.post_layer import (argmax_rows, last_token_indices, lm_head_argmax,
                                             post_layer_forward)

pytestmark = pytest.mark.gpu


def _randn(gpu, *shape, scale=1.0, seed=0):
    g = torch.Generator(device=gpu).manual_seed(seed)
    return (torch.randn(shape, device=gpu, generator=g) * scale).half()


@pytest.mark.parametrize("rows,hidden", [(1, 4096), (80, 4096), (4097, 1024), (33, 8), (7, 2056), (5, 8192)])
def test_fused_add_rmsnorm_matches_oracle(gpu, rows, hidden):
    x, r = _randn(gpu, rows, hidden, seed=1), _randn(gpu, rows, hidden, seed=2, scale=4.0)
    w = (torch.rand(hidden, device=gpu) + 0.5).half()
    want_x, want_r = oracle.fused_add_rmsnorm(x.cpu().numpy(), r.cpu().numpy(), w.cpu().numpy(), 1e-6)
    fused_add_rmsnorm_inplace(x, r, w, 1e-6)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(r.cpu().numpy(), want_r)
    got = x.cpu().numpy().astype(np.float64)
    np.testing.assert_allclose(got, want_x.astype(np.float64), rtol=1e-3, atol=1e-5)
    print(f"fused_add_rmsnorm {rows}x{hidden}: exact {np.mean(got == want_x.astype(np.float64)):.4f}", flush=True)


def test_fused_add_rmsnorm_rejects_bad_shapes(gpu):
    x = torch.zeros(2, 8200, dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.NativeLibraryError, match="hidden=8200"):
        fused_add_rmsnorm_inplace(x, x.clone(), torch.ones(8200, dtype=torch.float16, device=gpu), 1e-6)
    x = torch.zeros(2, 12, dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.NativeLibraryError, match="hidden=12"):
        fused_add_rmsnorm_inplace(x, x.clone(), torch.ones(12, dtype=torch.float16, device=gpu), 1e-6)


@pytest.mark.parametrize("rows,inter", [(1, 12288), (80, 12288), (3000, 3072), (5, 8)])
def test_silu_and_mul_matches_oracle(gpu, rows, inter):
    x = _randn(gpu, rows, 2 * inter, scale=3.0, seed=3)
    x0 = x.cpu().numpy()
    want = oracle.silu_and_mul(x0)
    silu_and_mul_inplace(x)
    torch.cuda.synchronize()
    got = x.cpu().numpy()
    np.testing.assert_array_equal(got[:, inter:], x0[:, inter:])  # the gate half is left alone
    np.testing.assert_allclose(got[:, :inter].astype(np.float64), want.astype(np.float64), rtol=2e-3, atol=1e-6)
    exact = np.mean(got[:, :inter] == want)
    assert exact > 0.99
    print(f"silu_and_mul {rows}x{inter}: exact {exact:.4f}", flush=True)


@pytest.mark.parametrize("rows,hidden,inter", [(1, 4096, 12288), (80, 4096, 12288), (97, 4096, 12288),
                                               (128, 4096, 12288), (64, 1024, 3072),
                                               (129, 1024, 3072), (33, 256, 4800), (16, 128, 16),
                                               (20, 512, 28672)])
def test_up_gate_silu_and_mul_matches_oracle(gpu, rows, hidden, inter):
    """The FFN's up/gate GEMM + SiLU-and-mul in one pass against the oracle's
    float64 GEMM rounded to fp16 then its SiLU-and-mul (transformer_layer.py:
    199-200), and against the library GEMM then this build's SiLU-and-mul.
    Shapes: the Qwen3-8B verify and Qwen3-0.6B draft batches, one row, two
    passes of rows (129), output tiles not a multiple of the CU count (300),
    one tile, and more tiles per workgroup than one group holds (7 of 6);
    the Qwen3-8B shape (one 48-column unit per CU) takes the split-k GEMM's
    gated unit at 1, 80 and 97 rows (up to 112), the ring kernel at 128.
    Rows past the output are never written."""
    x = _randn(gpu, rows, hidden, seed=11)
    w = _randn(gpu, 2 * inter, hidden, seed=12, scale=0.03)
    big = torch.full((rows + 1, inter), 7.0, dtype=torch.float16, device=gpu)
    out = up_gate_silu_and_mul(x, w, out=big[:rows])
    torch.cuda.synchronize()
    assert out.data_ptr() == big.data_ptr()
    assert bool((big[rows] == 7.0).all()), "a row past the output was written"
    got = out.cpu().numpy().astype(np.float64)
    want = oracle.silu_and_mul(oracle.lm_head_logits(x.cpu().numpy(), w.cpu().numpy())).astype(np.float64)
    # fp32 against float64 sums: an up or gate value one fp16 rounding apart
    np.testing.assert_allclose(got, want, rtol=4e-3, atol=2e-3)
    exact = float(np.mean(got == want))
    assert exact > 0.9
    ug = F.linear(x, w)
    silu_and_mul_inplace(ug)
    lib = ug[:, :inter].float().cpu().numpy()
    np.testing.assert_allclose(got, lib, rtol=4e-3, atol=2e-3)
    print(f"up_gate_silu_and_mul {rows}x{hidden}x{inter}: exact vs oracle {exact:.4f}, "
          f"vs library path {float(np.mean(got == lib)):.4f}", flush=True)


def test_up_gate_silu_and_mul_rejects_bad_shapes(gpu):
    x = torch.zeros(2, 100, dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.NativeLibraryError, match="hidden=100"):
        up_gate_silu_and_mul(x, torch.zeros(32, 100, dtype=torch.float16, device=gpu))
    x = torch.zeros(2, 128, dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.NativeLibraryError, match="inter=24"):
        up_gate_silu_and_mul(x, torch.zeros(48, 128, dtype=torch.float16, device=gpu))
    with pytest.raises(ValueError):
        up_gate_silu_and_mul(x, torch.zeros(33, 128, dtype=torch.float16, device=gpu))
    with pytest.raises(ValueError):
        up_gate_silu_and_mul(x, torch.zeros(32, 128, dtype=torch.float16, device=gpu),
                             out=torch.zeros(2, 15, dtype=torch.float16, device=gpu))
    assert up_gate_silu_and_mul(x[:0], torch.zeros(32, 128, dtype=torch.float16, device=gpu)).shape == (0, 16)


def _check_argmax(tokens, logits64, what):
    """tokens vs the first maximum of fp16(logits64); a differing token must
    be a near tie in float64."""
    l16 = logits64.half()
    want = torch.argmax(l16, dim=1)
    diff = (tokens != want).nonzero().flatten().tolist()
    for r in diff:
        a, b = logits64[r, tokens[r]].item(), logits64[r, want[r]].item()
        assert abs(a - b) <= 2e-3 * max(1.0, abs(b)), f"{what}: row {r} token {tokens[r]} ({a}) vs {want[r]} ({b})"
    print(f"{what}: {len(diff)} near-tie rows of {len(tokens)}", flush=True)
    return len(diff)


@pytest.mark.parametrize("rows,hidden,vocab", [(1, 1024, 1000), (17, 4096, 4099), (129, 1024, 2000),
                                               (300, 256, 777)])
def test_lm_head_argmax_matches_oracle(gpu, rows, hidden, vocab):
    """Row counts around the 16-row tiles and the 128-row pass; vocab sizes
    that are not a multiple of the 256-row workgroup."""
    x = _randn(gpu, rows, hidden, seed=4)
    w = _randn(gpu, vocab, hidden, seed=5, scale=0.05)
    tokens = lm_head_argmax(x, w)
    torch.cuda.synchronize()
    want_logits = oracle.lm_head_logits(x.cpu().numpy(), w.cpu().numpy())
    want = oracle.argmax_first(want_logits)
    l64 = torch.from_numpy(x.cpu().numpy().astype(np.float64) @ w.cpu().numpy().astype(np.float64).T)
    got = tokens.cpu()
    n = _check_argmax(got, l64, f"lm_head_argmax {rows}x{hidden}x{vocab}")
    assert n <= max(1, rows // 50)
    assert (got.numpy() == want).mean() >= 0.98


def test_lm_head_argmax_wide_many_rows(gpu):
    """200 rows (two passes of the fused kernel) at hidden 2048: the fused
    tokens agree with the library GEMM + the argmax kernel and with float64
    logits."""
    rows, hidden, vocab = 200, 2048, 3001
    x = _randn(gpu, rows, hidden, seed=13)
    w = _randn(gpu, vocab, hidden, seed=14, scale=0.03)
    fused = lm_head_argmax(x, w)
    routed = argmax_rows(torch.nn.functional.linear(x, w))
    torch.cuda.synchronize()
    l64 = torch.from_numpy(x.cpu().numpy().astype(np.float64) @ w.cpu().numpy().astype(np.float64).T)
    assert _check_argmax(routed.cpu(), l64, "wide rows, GEMM route") <= 2
    assert _check_argmax(fused.cpu(), l64, "wide rows, fused") <= 2


def test_lm_head_argmax_ties_nan_and_repeat(gpu):
    """Two identical vocab rows that are the maximum: the first wins; a NaN
    logit (inf weights against mixed-sign x) counts as the maximum; the keys
    buffer is left zero, so repeated calls agree."""
    rows, hidden, vocab = 40, 1024, 2048
    x = _randn(gpu, rows, hidden, seed=6)
    w = _randn(gpu, vocab, hidden, seed=7, scale=0.02)
    w[516] = (x[3].float() * 0.05).half()
    w[900] = w[516]  # same tile position (mod 32), same arithmetic
    t1 = lm_head_argmax(x, w)
    t2 = lm_head_argmax(x, w)
    torch.cuda.synchronize()
    assert t1[3].item() == 516
    assert torch.equal(t1, t2)
    w[1500] = float("inf")
    t3 = lm_head_argmax(x, w)
    torch.cuda.synchronize()
    assert (t3 == 1500).all(), t3.tolist()
    print("ties / NaN / repeat: ok", flush=True)


def test_lm_head_argmax_qwen3_8b_vocab_vs_reference_formulation(gpu):
    """Full Qwen3-8B lm_head (151,936 x 4096) at the verify batch (16
    requests x 5 rows): against float64 logits, and against the reference's
    own formulation on the same GPU (F.linear then torch.argmax)."""
    rows, hidden, vocab = 80, 4096, 151936
    x = _randn(gpu, rows, hidden, seed=8)
    w = _randn(gpu, vocab, hidden, seed=9, scale=0.02)
    tokens = lm_head_argmax(x, w)
    ref = torch.argmax(F.linear(x, w), dim=1)
    l64 = x.double() @ w.double().T
    torch.cuda.synchronize()
    n = _check_argmax(tokens.cpu(), l64.cpu(), "qwen3-8b lm_head")
    assert n <= 2
    same = (tokens == ref).float().mean().item()
    print(f"vs F.linear + argmax: {same:.4f} identical", flush=True)
    assert same >= 0.95


def test_argmax_rows_matches_torch(gpu):
    """Over given fp16 logits the argmax is bit-exact: ties, NaN, -0/+0,
    infinities, and a 151,936-wide row."""
    rows = torch.tensor([[1, 3, 3, 2], [-0.0, 0.0, -1, -2], [float("nan"), 5, 6, 7], [1, float("nan"), float("nan"), 9],
                         [-float("inf"), -float("inf"), -5, -5], [float("inf"), 1, float("inf"), 0]],
                        dtype=torch.float16, device=gpu)
    assert argmax_rows(rows).tolist() == [1, 0, 0, 1, 2, 0]
    big = _randn(gpu, 50, 151936, seed=10)
    big[::7, -1] = 100.0
    big[::5, 77] = 100.0
    got = argmax_rows(big)
    assert torch.equal(got, torch.argmax(big, dim=1))
    assert torch.equal(got.cpu(), torch.from_numpy(oracle.argmax_first(big.cpu().numpy())))


def test_post_layer_forward_matches_oracle(gpu):
    """post_layer.py:49-79 on an infer state with two prompts and decode rows."""
    from nebulasd_amd.config import QWEN3_0_6B, ModelConfig
    from nebulasd_amd.infer_state import build_infer_state, rope_cache

    mc = ModelConfig(QWEN3_0_6B)
    cos, sin = rope_cache(128, mc.rope_theta, 512, gpu)
    st = build_infer_state([0, 1, 2, 3, 4], [40, 41, 90], [7, 12], mc, cos, sin, gpu)
    hidden, vocab = 1024, 3000
    x = _randn(gpu, st.num_tokens, hidden, seed=11)
    fn = (torch.rand(hidden, device=gpu) + 0.5).half()
    w = _randn(gpu, vocab, hidden, seed=12, scale=0.05)
    tokens = post_layer_forward(x, st, fn, w, 1e-6)
    idx = last_token_indices(st).cpu().numpy()
    assert idx.tolist() == oracle.last_token_indices([0, 7], [7, 12], 19, 22).tolist()
    want, logits = oracle.post_layer(x.cpu().numpy(), idx, fn.cpu().numpy(), w.cpu().numpy(), 1e-6)
    got = tokens.cpu().numpy()
    assert got.shape == (st.batch_size,)
    assert (got == want).mean() >= 0.8 and all(
        abs(float(logits[i, got[i]]) - float(logits[i, want[i]])) <= 2e-2 for i in range(len(got)))


def test_lm_head_argmax_graph_replay(gpu):
    """Replays of a captured pair of lm_head + argmax calls give the eager
    tokens every time: each call's finalize leaves the key buffer at zero for
    the next call, replayed or eager (Qwen3-0.6B shape, 64 rows)."""
    g = torch.Generator(device=gpu).manual_seed(3)
    w = (torch.randn(151936, 1024, device=gpu, generator=g) * 0.05).half()
    xs = [torch.randn(64, 1024, device=gpu, generator=g).half() for _ in range(2)]
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()  # w and x are written on the default stream
    with torch.cuda.stream(stream):
        want = [lm_head_argmax(x, w) for x in xs]  # eager on the capture stream first
    torch.cuda.synchronize()
    assert not torch.equal(want[0], want[1])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            got = [lm_head_argmax(x, w) for x in xs]
    torch.cuda.synchronize()
    for rep in range(3):
        for t in got:
            t.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b), rep
        with torch.cuda.stream(stream):
            again = [lm_head_argmax(x, w) for x in xs]  # eager calls between replays
        torch.cuda.synchronize()
        for a, b in zip(again, want):
            assert torch.equal(a, b), rep
