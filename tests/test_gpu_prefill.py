"""GPU parity of the prefill (prompt) attention against the numpy oracle.

Every case prints its name first (pytest -v) so a failing GPU step is named.
Tolerances (tests/helpers.py): o within 2e-3 abs + 1e-2 rel, natural-log
LSE within 1e-4 abs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from helpers import ATOL_LSE, ATOL_O, RTOL_O, assert_close
from nebulasd_amd.config import QWEN3_0_6B, QWEN3_8B, ModelConfig
from nebulasd_amd.infer_state import build_infer_state, rope_cache
from nebulasd_amd.kernels import flash_attn_varlen_func, prefill_attention
from nebulasd_amd.workload import make_prefill_workload

pytestmark = pytest.mark.gpu

EDGE_LENS = [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 127, 128, 129, 255, 256, 257]


def run_prefill(w, validate=True):
    lse = torch.empty(w.q.shape[:2], dtype=torch.float32, device=w.q.device)
    o = flash_attn_varlen_func(w.q, w.k, w.v, w.cu_seqlens, w.cu_seqlens, max(w.lens), max(w.lens),
                               softmax_scale=w.spec.head_dim ** -0.5, causal=True, lse=lse,
                               validate=validate)
    torch.cuda.synchronize()
    return o, lse


def check(w, o, lse, what, cu=None):
    cu = w.cu_seqlens.cpu().numpy() if cu is None else cu
    wo, wl = oracle.prefill_attention(w.q.cpu().numpy(), w.k.cpu().numpy(), w.v.cpu().numpy(), cu)
    e_o = assert_close(o.float().cpu().numpy(), wo, ATOL_O, RTOL_O, f"{what} o")
    e_l = assert_close(lse.cpu().numpy(), wl, ATOL_LSE, 0.0, f"{what} lse")
    print(f"{what}: max|do|={e_o:.2e} max|dlse|={e_l:.2e}", flush=True)


@pytest.mark.parametrize("model", [QWEN3_8B, QWEN3_0_6B], ids=["8b", "06b"])
def test_prefill_edge_lengths(gpu, model):
    """Prompt lengths on both sides of the 16/32-token tile and position-block edges."""
    w = make_prefill_workload("prefill_target", 1, device=gpu, lens=EDGE_LENS, model=model)
    o, lse = run_prefill(w)
    check(w, o, lse, f"edges {ModelConfig(model).num_q_heads}q")


@pytest.mark.parametrize("name,seed", [("prefill_target", 0), ("prefill_draft", 0)])
def test_prefill_workload_matches_oracle(gpu, name, seed):
    """The benchmark's prompt batch (16 prompts of U[128, 1024] tokens)."""
    w = make_prefill_workload(name, seed, device=gpu)
    o, lse = run_prefill(w)
    check(w, o, lse, f"{name} seed {seed}")


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (32, 8), (64, 8), (32, 4)])
def test_prefill_gqa_ratios(gpu, hq, hkv):
    model = dict(QWEN3_8B, num_attention_heads=hq, num_key_value_heads=hkv)
    w = make_prefill_workload("prefill_target", 2, device=gpu, lens=[300, 1, 77, 512], model=model)
    o, lse = run_prefill(w)
    check(w, o, lse, f"gqa {hq}/{hkv}")


def test_prefill_matches_torch_sdpa_loop(gpu):
    """The reference's own formulation on the same GPU (transformer_layer.py:7-32):
    per-prompt scaled_dot_product_attention(is_causal=True) after
    repeat_interleave, here in fp32."""
    w = make_prefill_workload("prefill_target", 3, device=gpu, lens=[700, 33, 1024, 5])
    o, _ = run_prefill(w)
    cu = w.cu_seqlens.cpu().tolist()
    outs = []
    for s0, s1 in zip(cu[:-1], cu[1:]):
        qi = w.q[s0:s1].float().transpose(0, 1).unsqueeze(0).contiguous()
        ki = w.k[s0:s1].float().transpose(0, 1).unsqueeze(0).repeat_interleave(4, dim=1).contiguous()
        vi = w.v[s0:s1].float().transpose(0, 1).unsqueeze(0).repeat_interleave(4, dim=1).contiguous()
        outs.append(torch.nn.functional.scaled_dot_product_attention(qi, ki, vi, is_causal=True)
                    .squeeze(0).transpose(0, 1))
    want = torch.cat(outs).cpu().numpy()
    e = assert_close(o.float().cpu().numpy(), want, ATOL_O, RTOL_O, "vs torch sdpa loop")
    print(f"vs torch sdpa loop: max|do|={e:.2e}", flush=True)


def test_prefill_attention_entry_point_and_cut_last_prompt(gpu):
    """The Triton-style entry point on an infer state with prompts and decode
    rows: cu_seqlens ends at the forward's token count (model.py:412-415), so
    the last prompt's range is cut at num_prefill_tokens, as the reference's
    slicing of q[:num_prefill_tokens] cuts it."""
    mc = ModelConfig(QWEN3_8B)
    lens = [90, 17, 200]
    n_dec = 6
    cos, sin = rope_cache(128, mc.rope_theta, 512, gpu)
    st = build_infer_state([0, 1, 2, 3, 3, 3, 4, 5, 6], [50, 51, 52, 80, 9, 10], lens, mc, cos, sin, gpu)
    assert st.prefill_seq_start_locs_with_end[-1].item() == sum(lens) + n_dec
    w = make_prefill_workload("prefill_target", 4, device=gpu, lens=lens + [n_dec])
    o = torch.zeros_like(w.q)
    lse = torch.zeros(w.q.shape[:2], dtype=torch.float32, device=gpu)
    prefill_attention(w.q, w.k, w.v, o, mc, None, st, lse=lse[:sum(lens)], validate=True)
    torch.cuda.synchronize()
    npt = sum(lens)
    cu = np.array([0, 90, 107, 307])
    wo, wl = oracle.prefill_attention(w.q[:npt].cpu().numpy(), w.k[:npt].cpu().numpy(),
                                      w.v[:npt].cpu().numpy(), cu)
    assert_close(o[:npt].float().cpu().numpy(), wo, ATOL_O, RTOL_O, "entry point o")
    assert_close(lse[:npt].cpu().numpy(), wl, ATOL_LSE, 0.0, "entry point lse")
    assert (o[npt:] == 0).all(), "decode rows must be left alone"


def test_prefill_flags_bad_metadata(gpu):
    """A decreasing cu_seqlens pair and a prompt longer than max_seqlen are
    flagged (the kernel skips them; no access leaves the token range)."""
    w = make_prefill_workload("prefill_target", 5, device=gpu, lens=[64, 64, 64])
    bad = torch.tensor([0, 100, 50, 192], dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="invalid metadata"):
        flash_attn_varlen_func(w.q, w.k, w.v, bad, bad, 100, 100, validate=True)
    with pytest.raises(RuntimeError, match="invalid metadata"):
        flash_attn_varlen_func(w.q, w.k, w.v, w.cu_seqlens, w.cu_seqlens, 32, 32, validate=True)
    torch.cuda.synchronize()


def test_prefill_repeatable(gpu):
    """Fixed work split and summation order: repeated calls are bit-identical."""
    w = make_prefill_workload("prefill_target", 6, device=gpu, lens=[333, 1000])
    o1, l1 = run_prefill(w)
    o2, l2 = run_prefill(w)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_prefill_prompt_order_is_only_a_schedule(gpu):
    """The optional longest-first prompt order changes which workgroup runs
    when, not the arithmetic: natural order, longest first and a reversed
    order give bit-identical outputs; an entry outside the prompts is flagged."""
    from nebulasd_amd import _lib

    w = make_prefill_workload("prefill_target", 7, device=gpu, lens=[40, 700, 5, 300, 1000, 64])
    mx = max(w.lens)
    lens_t = w.cu_seqlens[1:] - w.cu_seqlens[:-1]
    orders = [None, torch.argsort(lens_t, descending=True, stable=True).int(),
              torch.arange(len(w.lens) - 1, -1, -1, dtype=torch.int32, device=gpu)]
    outs = []
    for order in orders:
        o = torch.empty_like(w.q)
        _lib.call("nsd_prefill_attention", w.q.data_ptr(), w.k.data_ptr(), w.v.data_ptr(), o.data_ptr(),
                  None, w.cu_seqlens.data_ptr(), None if order is None else order.data_ptr(), len(w.lens),
                  mx, w.tokens, w.q.shape[1], w.k.shape[1], 128, 128 ** -0.5, None,
                  torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        outs.append(o)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    bad = torch.tensor([0, 1, 2, 3, 4, 6], dtype=torch.int32, device=gpu)  # 6 is past the prompts
    o = torch.empty_like(w.q)
    _lib.call("nsd_prefill_attention", w.q.data_ptr(), w.k.data_ptr(), w.v.data_ptr(), o.data_ptr(), None,
              w.cu_seqlens.data_ptr(), bad.data_ptr(), len(w.lens), mx, w.tokens, w.q.shape[1],
              w.k.shape[1], 128, 128 ** -0.5, status.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert status.item() & _lib.STATUS_BAD_SEQ


def test_prefill_graph_replay_bit_identical(gpu):
    """A HIP graph of prefill calls replays to the eager output and LSE bit
    for bit, three times, with eager calls between (the prompts' longest-first
    order is computed by the eager call before capture and reused)."""
    w = make_prefill_workload("prefill_target", 8, device=gpu, lens=[40, 700, 5, 300, 1000, 64])
    mx = max(w.lens)
    lses = [torch.empty(w.q.shape[:2], dtype=torch.float32, device=gpu) for _ in range(2)]
    stream = torch.cuda.Stream()

    def calls():
        return [flash_attn_varlen_func(w.q, w.k, w.v, w.cu_seqlens, w.cu_seqlens, mx, mx,
                                       softmax_scale=w.spec.head_dim ** -0.5, causal=True, lse=lse)
                for lse in lses]

    torch.cuda.synchronize()  # the workload is written on the default stream
    with torch.cuda.stream(stream):
        want = [(o, lse.clone()) for o, lse in zip(calls(), lses)]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            got = calls()  # outputs in the graph's memory, rewritten by every replay
    torch.cuda.synchronize()
    for rep in range(3):
        for o, lse in zip(got, lses):
            o.zero_()
            lse.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o, lse, (wo, wl) in zip(got, lses, want):
            assert torch.equal(o, wo) and torch.equal(lse, wl), rep
        with torch.cuda.stream(stream):
            again = calls()
        torch.cuda.synchronize()
        for o, (wo, _) in zip(again, want):
            assert torch.equal(o, wo), rep
