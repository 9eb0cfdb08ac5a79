"""Host-side pieces around the path (no GPU): forward-phase ranges, the
ignore_kvcache flag of the infer state, the prefill order cache."""

from __future__ import annotations

import importlib

import pytest
import torch

from nebulasd_amd.config import QWEN3_8B, ModelConfig


def test_phase_ranges_follow_the_reference_switch(monkeypatch):
    calls = []
    monkeypatch.setattr(torch.cuda.nvtx, "range_push", lambda name: calls.append(("push", name)))
    monkeypatch.setattr(torch.cuda.nvtx, "range_pop", lambda: calls.append(("pop",)))
    monkeypatch.setenv("STARSD_ENABLE_FORWARD_PHASE_NVTX", "0")
    import nebulasd_amd.phases as phases
    phases = importlib.reload(phases)
    with phases.forward_phase_range("layer_3_paged_attention"):
        pass
    assert calls == []
    monkeypatch.setenv("STARSD_ENABLE_FORWARD_PHASE_NVTX", "on")
    phases = importlib.reload(phases)
    with phases.forward_phase_range("layer_3_paged_attention"):
        calls.append(("body",))
    assert calls == [("push", "layer_3_paged_attention"), ("body",), ("pop",)]


def test_phase_range_failures_do_not_stop_the_forward(monkeypatch):
    def boom(*a):
        raise RuntimeError("no profiler")
    monkeypatch.setattr(torch.cuda.nvtx, "range_push", boom)
    monkeypatch.setattr(torch.cuda.nvtx, "range_pop", boom)
    monkeypatch.setenv("STARSD_ENABLE_FORWARD_PHASE_NVTX", "1")
    import nebulasd_amd.phases as phases
    phases = importlib.reload(phases)
    ran = []
    with phases.forward_phase_range("post_lm_head"):
        ran.append(1)
    assert ran == [1]
    monkeypatch.setenv("STARSD_ENABLE_FORWARD_PHASE_NVTX", "0")
    importlib.reload(phases)


def test_ignore_kvcache_only_without_decode_rows():
    from nebulasd_amd.infer_state import build_infer_state, rope_cache

    mc = ModelConfig(QWEN3_8B)
    cos, sin = rope_cache(128, 1e6, 64, "cpu")
    st = build_infer_state([0, 1], [], [5, 7], mc, cos, sin, "cpu", ignore_kvcache=True)
    assert st.ignore_kvcache and st.num_prefill_seqs == 2
    assert not build_infer_state([0], [9], [], mc, cos, sin, "cpu").ignore_kvcache
    with pytest.raises(ValueError, match="ignore_kvcache"):
        build_infer_state([0, 1], [9], [5], mc, cos, sin, "cpu", ignore_kvcache=True)
