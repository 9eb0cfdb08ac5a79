"""Benchmark of the verify/decode paged-attention layer call on one MI355X.

A step is one pass over the model's layers: one verify-attention layer call
per layer (Qwen3-8B shape: 36 calls; B=16, q_len=5, contexts U[256, 4096],
24,576-block pool, fp16) on inputs already resident in HBM.  Cycling
``cur_layer`` over all 36 layers keeps the ~158 MB per-layer working set from
staying in the 256 MB Infinity Cache.  A HIP graph of one pass is replayed
``--warmup`` times untimed, then ``--steps`` times timed, with HIP events on
the stream the kernels run on: ``value`` is µs per layer call (all timed
calls), ``ms_per_step`` ms per pass, and the per-pass median / p10 / p90 are
reported beside it, with a same-layer "hot" figure (every call on layer 0,
whose blocks stay cached) as a diagnostic.  The fused prologue (QK-RMSNorm +
RoPE + KV store) is timed alone, followed by the attention (two launches per
layer), and inside the attention's own launch (one launch per layer).

Beside the headline: Draft decode (Qwen3-0.6B shape, B=64), ragged
long-context verify (q_len=9, contexts log-U[1024, 32768]) and the small
4-request decode case; the attention at the shapes the single-GPU
speculative loop produces (Qwen3-0.6B draft batch 64 + Qwen3-8B target
batch 16, depth 4, prompts U[128, 1024]); the prefill attention of one
16-prompt chunk (both model shapes) with its MFMA roofline and the
reference's per-prompt SDPA loop; the rest-of-layer kernels, the block-table
writer and the HostKV copies; and two ceiling probes -- a contiguous
streaming read and a gather of exactly the K/V tiles each attention workload
reads, with no arithmetic -- so that the attention's rate can be read
against what the device delivers for the same bytes.  The CPU baseline runs
the PyTorch-CPU fp32 restatement of the reference's row-wise attention on
this host's affinity cores, median per layer call, for every workload.

Prints one JSON line (see ``--help``).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=30,
                   help="timed passes; a pass is one attention call per layer of the model")
    p.add_argument("--warmup", type=int, default=3, help="untimed passes before the timed ones")
    p.add_argument("--workload", default="target_verify")
    p.add_argument("--secondary", default="draft_decode,ragged_verify,cpu_plumbing",
                   help="comma-separated workloads measured beside the headline ('' to skip)")
    p.add_argument("--prefill", default="prefill_target,prefill_draft",
                   help="comma-separated prefill-attention workloads ('' to skip)")
    p.add_argument("--block-table", type=int, default=1, help="1: time the block-table metadata writer")
    p.add_argument("--hostkv", type=int, default=1, help="1: time the HostKV block-range copies")
    p.add_argument("--layer-rest", type=int, default=1, help="1: time the rest-of-layer kernels")
    p.add_argument("--layer-step", type=int, default=1, help="1: time one whole target-verify layer")
    p.add_argument("--spec-loop", type=int, default=1,
                   help="1: time the attention at the speculative loop's shapes (64 requests x 16 tokens)")
    p.add_argument("--probes", type=int, default=1, help="1: run the HBM ceiling probes")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--cpu-baseline-seconds", type=float, default=12.0,
                   help="bound on CPU oracle time (0 disables the CPU baseline)")
    p.add_argument("--other-cpu-seconds", type=float, default=4.0,
                   help="bound on CPU oracle time for each secondary workload")
    return p.parse_args()


def _time_graph(fn, stream, reps: int, wreps: int):
    """Capture fn() in a HIP graph on `stream` and replay it `reps` times
    back to back after `wreps` untimed replays.  HIP events recorded on that
    same stream before the first timed replay and after each one give the
    mean µs per replay (first to last event) and the per-replay durations."""
    import torch

    fn()  # plans, kernel attributes: everything a capture must not do
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            fn()
    torch.cuda.synchronize()
    events = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    with torch.cuda.stream(stream):
        for _ in range(wreps):
            graph.replay()
        events[0].record(stream)
        for i in range(reps):
            graph.replay()
            events[i + 1].record(stream)
    torch.cuda.synchronize()
    del graph
    per = [events[i].elapsed_time(events[i + 1]) * 1e3 for i in range(reps)]
    return events[0].elapsed_time(events[reps]) * 1e3 / reps, per


def _spread(per_replay, calls_per_replay: int) -> dict:
    """Median, p10 and p90 of µs per layer call over the timed replays."""
    import numpy as np

    x = np.asarray(per_replay, dtype=np.float64) / calls_per_replay
    p10, p50, p90 = np.percentile(x, (10, 50, 90))
    return {"median": float(p50), "p10": float(p10), "p90": float(p90), "replays": len(x)}


def measure(name: str, seed: int, steps: int, warmup: int):
    """Time `steps` passes over the layers for workload `name`; returns (result dict, workload).

    Four graphs of one pass over all layers are timed: the attention alone
    (the headline), the fused prologue alone, prologue then attention (two
    launches per layer), and both in the attention's launch
    (paged_attention_fused).  The prologue works on copies of q and fresh
    k/v rows, so the attention inputs of the first graph are never modified.
    """
    import torch

    from nebulasd_amd.config import EngineConfig, ModelConfig
    from nebulasd_amd.infer_state import build_infer_state, rope_cache
    from nebulasd_amd._lib import NativeLibraryError
    from nebulasd_amd.kernels import paged_attention, paged_attention_fused, qk_norm_rope_store
    from nebulasd_amd.workload import make_workload

    dev = torch.device("cuda:0")
    w = make_workload(name, seed, device=dev)
    mc = ModelConfig(w.spec.model)
    ec = EngineConfig(block_size=16, max_blocks_per_seq=w.block_table.shape[1])
    cos, sin = rope_cache(128, mc.rope_theta, max(w.seq_lens) + 1, dev)
    st = build_infer_state(w.seq_ids, w.seq_lens, [], mc, cos, sin, dev)
    L = mc.num_layers
    o = torch.empty_like(w.q)
    g = torch.Generator(device=dev).manual_seed(seed + 1000)
    hkv = mc.num_kv_heads
    qp = w.q.clone()
    kn = torch.randn((w.rows, hkv, 128), device=dev, generator=g).half()
    vn = torch.randn((w.rows, hkv, 128), device=dev, generator=g).half()
    qw = (torch.rand(128, device=dev, generator=g) + 0.5).half()
    kw = (torch.rand(128, device=dev, generator=g) + 0.5).half()

    def attn_pass():
        for layer in range(L):
            paged_attention(w.q, w.k_cache, w.v_cache, w.block_table, mc, ec, st, layer, o)

    def prologue_pass():
        for layer in range(L):
            qk_norm_rope_store(qp, kn, vn, w.k_cache, w.v_cache, w.block_table, qw, kw, mc, ec,
                               st, layer, cos, sin)

    def layer_pass():
        for layer in range(L):
            qk_norm_rope_store(qp, kn, vn, w.k_cache, w.v_cache, w.block_table, qw, kw, mc, ec,
                               st, layer, cos, sin)
            paged_attention(qp, w.k_cache, w.v_cache, w.block_table, mc, ec, st, layer, o)

    def fused_pass():
        for layer in range(L):
            paged_attention_fused(w.q, kn, vn, w.k_cache, w.v_cache, w.block_table, qw, kw, mc, ec, st, layer,
                                  cos, sin, o)

    def hot_pass():
        for _ in range(L):
            paged_attention(w.q, w.k_cache, w.v_cache, w.block_table, mc, ec, st, 0, o)

    stream = torch.cuda.Stream()
    reps, wreps = max(1, steps), max(0, warmup)
    t0 = time.perf_counter()
    us_pass, per = _time_graph(attn_pass, stream, reps, wreps)
    us = us_pass / L
    wall = time.perf_counter() - t0
    us_pro, per_pro = _time_graph(prologue_pass, stream, reps, wreps)
    us_layer, per_layer = _time_graph(layer_pass, stream, reps, wreps)
    try:  # a plan that splits a sequence over verify groups has no fused launch
        us_fused, per_fused = _time_graph(fused_pass, stream, reps, wreps)
    except NativeLibraryError:
        us_fused, per_fused = None, None
    # Diagnostic only: every call reads layer 0, whose blocks then stay in
    # the 256 MB Infinity Cache between calls.
    us_hot, _ = _time_graph(hot_pass, stream, reps, wreps)
    nbytes = w.algorithmic_bytes()
    gbps = nbytes / (us * 1e-6) / 1e9
    plan = st.attn_plan
    res = {
        "workload": name,
        "steps": reps,
        "layer_calls": reps * L,
        "us_per_pass": us_pass,
        "us_per_layer_call": us,
        "wall_ms": wall * 1e3,
        "algorithmic_bytes": nbytes,
        "hbm_gbps": gbps,
        "hbm_frac": gbps / HBM_PEAK_GBPS,
        "tokens_per_s": w.rows / (us * 1e-6 * L),
        "tflops": w.flops() / (us * 1e-6) / 1e12,
        "rows": w.rows,
        "kv_tokens": w.kv_tokens(),
        "plan_workers": int(plan.host[5]),
        "plan_rows_max": plan.rows_max,
        "us_per_layer_call_spread": _spread(per, L),
        "hot_same_layer_us": us_hot / L,
        "prologue_us": us_pro / L,
        "prologue_us_spread": _spread(per_pro, L),
        "prologue_bytes": w.prologue_bytes(),
        "prologue_gbps": w.prologue_bytes() / (us_pro / L * 1e-6) / 1e9,
        "prologue_plus_attention_us": us_layer / L,
        "prologue_plus_attention_us_spread": _spread(per_layer, L),
        "fused_layer_us": us_fused / L if us_fused is not None else None,
        "fused_layer_us_spread": _spread(per_fused, L) if per_fused is not None else None,
    }
    return res, w


MFMA_F16_PEAK_TFLOPS = 2500.0


def measure_prefill(name: str, seed: int, steps: int, warmup: int, cpu_seconds: float):
    """Prefill (prompt) attention of workload `name`: µs per layer call from a
    HIP graph of `calls` back-to-back launches on the same prompts, the
    reference's per-prompt SDPA loop (transformer_layer.py:7-32) timed the
    same way on the GPU, and the numpy oracle on the host (bounded)."""
    import numpy as np
    import torch

    from nebulasd_amd.kernels import flash_attn_varlen_func
    from nebulasd_amd.workload import make_prefill_workload

    dev = torch.device("cuda:0")
    w = make_prefill_workload(name, seed, device=dev)
    mx = max(w.lens)
    calls = w.spec.num_layers

    def kernel_pass():
        for _ in range(calls):
            flash_attn_varlen_func(w.q, w.k, w.v, w.cu_seqlens, w.cu_seqlens, mx, mx)

    cu = w.cu_seqlens.cpu().tolist()
    g = w.q.shape[1] // w.k.shape[1]

    def sdpa_pass():  # the reference's loop, fp16 on the GPU
        outs = []
        for s0, s1 in zip(cu[:-1], cu[1:]):
            qi = w.q[s0:s1].transpose(0, 1).unsqueeze(0)
            ki = w.k[s0:s1].transpose(0, 1).unsqueeze(0).repeat_interleave(g, dim=1)
            vi = w.v[s0:s1].transpose(0, 1).unsqueeze(0).repeat_interleave(g, dim=1)
            outs.append(torch.nn.functional.scaled_dot_product_attention(qi, ki, vi, is_causal=True)
                        .squeeze(0).transpose(0, 1))
        return torch.cat(outs)

    stream = torch.cuda.Stream()
    reps, wreps = max(1, steps), max(0, warmup)
    us, per = _time_graph(kernel_pass, stream, reps, wreps)
    us /= calls
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    sdpa_pass()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(5):
        sdpa_pass()
    e1.record()
    torch.cuda.synchronize()
    us_sdpa = e0.elapsed_time(e1) * 1e3 / 5
    flops = w.flops()
    tflops = flops / (us * 1e-6) / 1e12
    res = {
        "workload": name,
        "kind": "prefill",
        "steps": reps,
        "layer_calls": reps * calls,
        "us_per_layer_call": us,
        "us_per_layer_call_spread": _spread(per, calls),
        "prompts": w.lens,
        "tokens": w.tokens,
        "flops": flops,
        "tflops": tflops,
        "mfma_frac": tflops / MFMA_F16_PEAK_TFLOPS,
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": tflops / MFMA_F16_PEAK_TFLOPS, "traffic": None},
        "algorithmic_bytes": w.algorithmic_bytes(),
        "reference_sdpa_loop_us": us_sdpa,
        "speedup_vs_sdpa_loop": us_sdpa / us,
    }
    if cpu_seconds > 0:
        import oracle
        from threadpoolctl import threadpool_info, threadpool_limits

        q, k, v = (x.cpu().numpy() for x in (w.q, w.k, w.v))
        cores = _cpu_threads()
        times = []
        with threadpool_limits(limits=cores):
            threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
            t_end = time.perf_counter() + cpu_seconds
            while True:
                t0 = time.perf_counter()
                oracle.prefill_attention(q, k, v, cu, dtype=np.float32)
                times.append(time.perf_counter() - t0)
                if time.perf_counter() > t_end or len(times) >= 20:
                    break
        res["cpu_baseline"] = {"value": float(np.median(times)) * 1e6, "unit": "us/layer-call",
                               "cores": int(min(threads, cores)), "kind": "port",
                               "sample": f"{len(times)} calls of {name}, numpy fp32 oracle, median",
                               "cpu_model": _cpu_model()}
    del w
    torch.cuda.empty_cache()
    return res


def measure_block_table(seed: int, reps: int = 50, cpu_seconds: float = 0.0):
    """Bank-switch metadata: 128 block-table rows get contiguous ranges of
    U[0, 256] blocks.  Host-to-completion latency per write (median over
    `reps`, synchronised) of this build's writer and of the reference's
    formulation (dma_process.py:111-121: host index/value arrays in pinned
    memory, two H2D copies, index_copy_, event sync)."""
    import numpy as np
    import torch

    from nebulasd_amd.kernels import write_block_table_ranges

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(seed)
    rows_n, stride = 128, 2560
    rows = rng.permutation(rows_n).tolist()
    counts = rng.integers(0, 257, rows_n).tolist()
    begins = np.cumsum([0] + counts[:-1]).tolist()
    bt = torch.zeros((rows_n, stride), dtype=torch.int32, device=dev)
    na = torch.zeros(rows_n, dtype=torch.int32, device=dev)
    stream = torch.cuda.Stream()
    cap = sum(counts)
    indices = torch.empty(cap, dtype=torch.int64, pin_memory=True)
    values = torch.empty(cap, dtype=torch.int32, pin_memory=True)
    gi, gv = torch.empty_like(indices, device=dev), torch.empty_like(values, device=dev)
    ix, val = indices.numpy(), values.numpy()

    def ours():
        with torch.cuda.stream(stream):
            write_block_table_ranges(bt, rows, begins, counts, na)
        stream.synchronize()

    def reference():
        n = 0
        for row, begin, count in zip(rows, begins, counts):
            ix[n:n + count] = np.arange(row * stride, row * stride + count)
            val[n:n + count] = np.arange(begin, begin + count)
            n += count
        with torch.cuda.stream(stream):
            gi[:n].copy_(indices[:n], non_blocking=True)
            gv[:n].copy_(values[:n], non_blocking=True)
            bt.view(-1).index_copy_(0, gi[:n], gv[:n])
            done = torch.cuda.Event()
            done.record(stream)
        done.synchronize()

    out = {}
    for name, fn in (("ours", ours), ("reference", reference)):
        for _ in range(5):
            fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append((time.perf_counter() - t0) * 1e6)
        out[name] = float(np.median(ts))
    ref_bt = bt.clone()
    ours()
    same = bool(torch.equal(bt, ref_bt))
    cpu = None
    if cpu_seconds > 0:
        import oracle

        btn, nan_ = bt.cpu().numpy(), na.cpu().numpy()
        cpu = _cpu_time(lambda: oracle.write_block_ranges(btn, rows, begins, counts, nan_), cpu_seconds, 200,
                        what="the numpy oracle's range writer over the same 128 rows")
    return {"workload": "block_table_bank_switch", "kind": "metadata", "rows": rows_n, "cpu_baseline": cpu,
            "blocks_written": cap, "us_per_write": out["ours"], "reference_us_per_write": out["reference"],
            "speedup_vs_reference": out["reference"] / out["ours"], "identical_tables": same,
            "note": "host-to-completion latency, median of %d synchronised writes" % reps}


HOST_LINK_PEAK_GBPS = 64.0  # PCIe 5.0 x16, one direction: 32 GT/s x 16 lanes / 8


def _hip_runtime():
    """The HIP runtime the native library is bound to (ctypes handle), for
    the reference's own call pattern: hipMemcpyAsync through ctypes."""
    import ctypes

    from nebulasd_amd import _lib

    _lib.load()
    with open("/proc/self/maps") as f:
        paths = {line.split()[-1] for line in f if "libamdhip64" in line}
    hip = ctypes.CDLL(sorted(paths)[0])
    hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                   ctypes.c_void_p]
    hip.hipMemcpyAsync.restype = ctypes.c_int
    return hip


def measure_hostkv(seed: int, reps: int = 6):
    """HostKV copies of Qwen3-8B blocks (1,179,648 bytes per K or V block) in
    the layout of the reference's copy benchmark
    (nebulasd/tests/support/copy_benchmark.py:11-56): 8 requests of 32
    blocks, a guard block each side, one region per request, D2H then H2D;
    then a swap of 128 scattered single blocks each way.  Copy interval from
    events on the copy stream, median of `reps`.  Legs: the reference's
    formulation (one hipMemcpyAsync per region and plane through ctypes,
    cuda_transfer.py:93-106 with cuda_memcpy.py:52-55), the DMA engine and
    the kernel engine.  Bytes are compared after the timed copies."""
    import numpy as np
    import torch

    from nebulasd_amd.hostkv import HostKVArena, copy_block_ranges, swap_blocks

    dev = torch.device("cuda:0")
    shape = (36, 8, 16, 128)
    batch, blocks = 8, 32
    cap = blocks + 2
    nb = batch * cap
    k = torch.empty((nb, *shape), dtype=torch.float16, device=dev)
    v = torch.empty_like(k)
    bb = k[0].numel() * 2
    arena = HostKVArena.create(total_blocks=nb, block_bytes=bb, kv_block_shape=shape)
    addr, plane = arena.address(), arena.descriptor.plane_bytes
    hip = _hip_runtime()
    stream = torch.cuda.Stream()
    regions = [(i * cap + 1, i * cap + 1, blocks) for i in range(batch)]
    g_, h_, c_ = zip(*regions)
    plan_bytes = 2 * batch * blocks * bb

    scratch = torch.empty_like(k)

    def randomize():
        """Fresh random bytes on both sides (the host planes through a pinned
        copy of a random device buffer, so every block differs)."""
        for host in (arena.k, arena.v):
            scratch.view(torch.int16).random_(-30000, 30000)
            host.view(-1).copy_(scratch.view(torch.uint8).view(-1))
        k.view(torch.int16).random_(-30000, 30000)
        v.view(torch.int16).random_(-30000, 30000)
        torch.cuda.synchronize()

    def reference(direction):
        kind = 2 if direction == "D2H" else 1
        for g, h, c in regions:
            n = c * bb
            for cache, host in ((k, addr), (v, addr + plane)):
                gpu_p, host_p = cache.data_ptr() + g * bb, host + h * bb
                dst, src = (host_p, gpu_p) if direction == "D2H" else (gpu_p, host_p)
                rc = hip.hipMemcpyAsync(dst, src, n, kind, stream.cuda_stream)
                if rc:
                    raise RuntimeError(f"hipMemcpyAsync failed with status {rc}")

    def engine(name):
        return lambda direction: copy_block_ranges(k, v, addr, addr + plane, nb, g_, h_, c_, direction, name,
                                                   stream.cuda_stream)

    def timed_once(fn, *a):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        fn(*a)
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1), (time.perf_counter() - t0) * 1e6

    def same_bytes():
        ok = True
        for g, h, c in regions:
            for cache, host in ((k, arena.k), (v, arena.v)):
                ok &= bool(torch.equal(cache[g:g + c].view(torch.uint8).reshape(c, -1).cpu(), host[h:h + c]))
        return ok

    legs = (("reference", reference), ("dma", engine("dma")), ("kernel", engine("kernel")))
    out, identical = {}, True
    for direction in ("D2H", "H2D"):
        # untimed pass per leg: fresh bytes on both sides, copy, compare
        for _, fn in legs:
            randomize()
            fn(direction)
            stream.synchronize()
            identical &= same_bytes()
        # timed rounds, leg order alternating (as copy_benchmark.py:31 alternates its paths)
        for _, fn in legs:
            fn(direction)
        stream.synchronize()
        samples = {leg: ([], []) for leg, _ in legs}
        for rnd in range(reps):
            for leg, fn in (legs if rnd % 2 == 0 else legs[::-1]):
                ms, us = timed_once(fn, direction)
                samples[leg][0].append(plan_bytes / ms / 1e6)
                samples[leg][1].append(us)
        row = {}
        for leg, (gbps, us) in samples.items():
            row[f"{leg}_gbps"] = float(np.median(gbps))
            row[f"{leg}_gbps_min_max"] = [float(min(gbps)), float(max(gbps))]
            row[f"{leg}_host_to_completion_us"] = float(np.median(us))
        out[direction] = row

    def timed(fn, *a):
        fn(*a)
        stream.synchronize()
        return float(np.median([timed_once(fn, *a)[0] for _ in range(reps)])), None

    # swap_blocks: 128 scattered single blocks (runs of consecutive ids are rare)
    rng = np.random.default_rng(seed)
    gpu_ids = rng.permutation(nb)[:128].tolist()
    host_ids = rng.permutation(nb)[:128].tolist()
    ks, vs = arena.k.view(nb, *shape[:-1], 2 * shape[-1]), arena.v.view(nb, *shape[:-1], 2 * shape[-1])
    ks, vs = ks.view(torch.float16), vs.view(torch.float16)
    swap = {}
    for is_in in (False, True):
        src, dst = (host_ids, gpu_ids) if is_in else (gpu_ids, host_ids)
        row = {}
        for name in ("dma", "kernel"):
            def fn(name=name):
                with torch.cuda.stream(stream):
                    swap_blocks(src, dst, is_in, k, v, ks, vs, engine=name)
            randomize()
            ms, _ = timed(fn)
            for gi, hi in zip(gpu_ids, host_ids):
                identical &= bool(torch.equal(k[gi].view(torch.uint8).reshape(-1).cpu(), arena.k[hi]))
            row[f"{name}_gbps"] = 2 * 128 * bb / ms / 1e6
        swap["in" if is_in else "out"] = row
    # the link's ceiling as torch's own pinned copy of one whole plane sees it
    flat_dev, flat_host = k.view(torch.uint8).view(-1), arena.k.view(-1)
    ceil = {}
    for d, fn in (("H2D", lambda: flat_dev.copy_(flat_host, non_blocking=True)),
                  ("D2H", lambda: flat_host.copy_(flat_dev, non_blocking=True))):
        with torch.cuda.stream(stream):
            ms, _ = timed(fn)
        ceil[d] = plane / ms / 1e6
    best = min(max(out[d]["dma_gbps"], out[d]["kernel_gbps"]) for d in out)
    return {"workload": "hostkv_copy", "kind": "host_link", "block_bytes": bb, "requests": batch,
            "blocks_per_request": blocks, "bytes_per_plan": plan_bytes, **out,
            "swap_128_scattered_blocks": swap, "torch_pinned_copy_gbps": ceil,
            "roofline": {"bound": "host_link", "achieved": best, "peak": HOST_LINK_PEAK_GBPS, "unit": "GB/s",
                         "frac": best / HOST_LINK_PEAK_GBPS},
            "identical_bytes": identical,
            "note": ("copy interval from events on the copy stream; median (and min, max) of %d plans per leg, "
                     "legs in alternating order; bytes compared in a separate untimed pass per leg" % reps)}


def measure_layer_step(seed: int, reps: int = 20):
    """One whole Qwen3-8B target-verify decoder layer (16 requests x 5 rows,
    contexts U[256, 4096]) in the reference's order
    (transformer_layer.py:83-201) on this build's kernels, the q/k/v, O and
    down GEMMs through torch.mm (hipBLASLt): fused add-RMSNorm, one fused
    q/k/v GEMM (the reference runs three; both are timed), the fused prologue
    reading its rows, paged attention, O GEMM, fused add-RMSNorm, the up/gate
    projection with SiLU-and-mul in one pass (also timed as the library GEMM
    then SiLU-and-mul), down GEMM.  Passes of four layers (weights of four distinct layers,
    1.7 GB, so each layer reads its weights from HBM): the whole layer, the
    GEMMs alone and the rest alone.  Floor: weight bytes + the attention's
    K/V bytes at the device-copy rate.  Timed eagerly (see below)."""
    import numpy as np
    import torch
    import torch.nn.functional as F

    from nebulasd_amd.config import EngineConfig, ModelConfig
    from nebulasd_amd.infer_state import build_infer_state, rope_cache
    from nebulasd_amd.kernels import (fused_add_rmsnorm_inplace, paged_attention, qk_norm_rope_store,
                                      silu_and_mul_inplace, up_gate_silu_and_mul)
    from nebulasd_amd.workload import make_workload

    dev = torch.device("cuda:0")
    w = make_workload("target_verify", seed, device=dev)
    mc = ModelConfig(w.spec.model)
    ec = EngineConfig(block_size=16, max_blocks_per_seq=w.block_table.shape[1])
    cos, sin = rope_cache(128, mc.rope_theta, max(w.seq_lens) + 1, dev)
    st = build_infer_state(w.seq_ids, w.seq_lens, [], mc, cos, sin, dev)
    H, I, hq, hkv, d = mc.hidden_size, mc.ffn_inter_dim, mc.num_q_heads, mc.num_kv_heads, mc.head_dim
    T = w.rows
    g = torch.Generator(device=dev).manual_seed(seed + 7)

    def rnd(*shape, scale=0.02):
        return (torch.randn(shape, device=dev, generator=g) * scale).half()
    n_layers = 4
    layers = [dict(wqkv=rnd((hq + 2 * hkv) * d, H), wo=rnd(H, hq * d),
                   wug=rnd(2 * I, H), wd=rnd(H, I), n_in=(torch.rand(H, device=dev, generator=g) + 0.5).half(),
                   n_post=(torch.rand(H, device=dev, generator=g) + 0.5).half(),
                   qn=(torch.rand(d, device=dev, generator=g) + 0.5).half(),
                   kn=(torch.rand(d, device=dev, generator=g) + 0.5).half()) for _ in range(n_layers)]
    for lw in layers:  # the reference's three projections are row blocks of the fused weight
        lw["wq"], lw["wk"], lw["wv"] = lw["wqkv"].split([hq * d, hkv * d, hkv * d])
    weight_bytes = sum(t.numel() * 2 for n, t in layers[0].items() if n not in ("wq", "wk", "wv"))
    x0 = rnd(T, H, scale=1.0)
    x, res = x0.clone(), torch.zeros_like(x0)
    o = torch.empty((T, hq, d), dtype=torch.float16, device=dev)
    q = torch.empty_like(o)
    k = torch.empty((T, hkv, d), dtype=torch.float16, device=dev)
    v = torch.empty_like(k)
    oo = torch.empty((T, H), dtype=torch.float16, device=dev)
    qkv = torch.empty((T, (hq + 2 * hkv) * d), dtype=torch.float16, device=dev)
    qs = qkv[:, :hq * d].view(T, hq, d)
    ks = qkv[:, hq * d:(hq + hkv) * d].view(T, hkv, d)
    vs = qkv[:, (hq + hkv) * d:].view(T, hkv, d)
    ug = torch.empty((T, 2 * I), dtype=torch.float16, device=dev)
    hh = torch.empty((T, I), dtype=torch.float16, device=dev)
    kv_layer = [mc.num_layers // 2 + i for i in range(n_layers)]

    def layer(i, gemms=True, rest=True, fused_qkv=True, fused_ffn=True):
        lw = layers[i]
        if rest:
            fused_add_rmsnorm_inplace(x, res, lw["n_in"], mc.rms_norm_eps)
        if gemms and fused_qkv:
            torch.mm(x, lw["wqkv"].t(), out=qkv)
        elif gemms:
            torch.mm(x, lw["wq"].t(), out=q.view(T, -1))
            torch.mm(x, lw["wk"].t(), out=k.view(T, -1))
            torch.mm(x, lw["wv"].t(), out=v.view(T, -1))
        if rest:
            if fused_qkv:
                qk_norm_rope_store(qs, ks, vs, w.k_cache, w.v_cache, w.block_table, lw["qn"], lw["kn"], mc, ec,
                                   st, kv_layer[i], cos, sin, q_out=q)
            else:
                qk_norm_rope_store(q, k, v, w.k_cache, w.v_cache, w.block_table, lw["qn"], lw["kn"], mc, ec, st,
                                   kv_layer[i], cos, sin)
            paged_attention(q, w.k_cache, w.v_cache, w.block_table, mc, ec, st, kv_layer[i], o)
        if gemms:
            torch.mm(o.view(T, -1), lw["wo"].t(), out=oo)
        if rest:
            fused_add_rmsnorm_inplace(oo, res, lw["n_post"], mc.rms_norm_eps)
        if gemms and fused_ffn:  # the up/gate projection and SiLU-and-mul in one kernel
            up_gate_silu_and_mul(oo, lw["wug"], out=hh)
        elif gemms:
            torch.mm(oo, lw["wug"].t(), out=ug)
        if rest and not fused_ffn:
            silu_and_mul_inplace(ug)
        if gemms:
            torch.mm(hh if fused_ffn else ug[:, :I], lw["wd"].t(), out=x)

    # Eager, not a graph: captured with the library GEMMs these passes did not
    # replay to the eager result, so they stay out of graphs.  `reps` passes
    # of four layers are enqueued back to back with an event between passes;
    # the figure is the median pass (a pass the host fell behind in, e.g. when
    # the process was descheduled, shows as a device gap and is an outlier).
    # The host's enqueue time is kept too, so a host-bound figure shows as
    # host_us >= device us.
    stream = torch.cuda.current_stream()
    out, host, spread = {}, {}, {}
    for name, kw in (("layer", {}), ("gemms_only", {"rest": False}), ("rest_only", {"gemms": False}),
                     ("layer_three_qkv_gemms", {"fused_qkv": False}), ("layer_unfused_ffn", {"fused_ffn": False})):
        for i in range(n_layers):
            layer(i, **kw)
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        t0 = time.perf_counter()
        ev[0].record(stream)
        for r in range(reps):
            for i in range(n_layers):
                layer(i, **kw)
            ev[r + 1].record(stream)
        host[name] = (time.perf_counter() - t0) * 1e6 / (reps * n_layers)
        ev[-1].synchronize()
        per = np.array([ev[r].elapsed_time(ev[r + 1]) * 1e3 / n_layers for r in range(reps)])
        out[name] = float(np.median(per))
        spread[name] = [float(np.percentile(per, q)) for q in (10, 50, 90)]
    kv_bytes = w.algorithmic_bytes()
    copy = getattr(measure_layer_step, "copy_gbps", None)
    floor = (weight_bytes + (kv_bytes or 0)) / (copy * 1e3) if copy and kv_bytes else None
    del w, layers
    torch.cuda.empty_cache()
    return {"workload": "layer_step_target_verify", "kind": "whole_layer", "rows": T,
            "us_per_layer": out["layer"], "gemms_only_us": out["gemms_only"], "rest_only_us": out["rest_only"],
            "us_per_layer_three_qkv_gemms": out["layer_three_qkv_gemms"],
            "us_per_layer_unfused_ffn": out["layer_unfused_ffn"],
            "us_per_layer_p10_p50_p90": spread,
            "host_enqueue_us_per_layer": host,
            "weight_bytes_per_layer": weight_bytes, "kv_bytes_per_layer": kv_bytes,
            "floor_us_at_copy_rate": floor,
            "note": "q/k/v, O and down GEMMs through torch.mm (hipBLASLt): one fused q/k/v projection read by the "
                    "strided prologue (us_per_layer_three_qkv_gemms: the reference's three); the up/gate projection "
                    "and SiLU-and-mul in one kernel of this build, counted with the GEMMs (us_per_layer_unfused_ffn: "
                    "the library up/gate GEMM then this build's SiLU-and-mul); the rest is this build's kernels; "
                    "eager passes of four layers with distinct weights"}


def measure_native_layers(seed: int, reps: int = 20) -> dict:
    """The native decoder stack (nsd_decoder_forward: every layer enqueued
    from C++ on this build's kernels, split-k projections included) over
    four layers with distinct weights, graph-replayed: µs per layer at the
    target-verify batch (Qwen3-8B, 16 requests x 5 rows, contexts
    U[256, 4096]) and the draft batch (Qwen3-0.6B, 64 rows, contexts
    U[512, 2048]); the weights of four layers (1.5 GB for Qwen3-8B) exceed
    the 256 MB MALL, so each layer reads its weights from HBM."""
    import numpy as np
    import torch

    from nebulasd_amd.config import EngineConfig, ModelConfig
    from nebulasd_amd.decoder import DecoderStack
    from nebulasd_amd.infer_state import build_infer_state, rope_cache
    from nebulasd_amd.workload import make_workload

    dev = torch.device("cuda:0")
    out = {}
    n_layers = 4
    for name, workload in (("target_verify", "target_verify"), ("draft_decode", "draft_decode")):
        w = make_workload(workload, seed, device=dev, num_layers=n_layers)
        cfg = dict(w.spec.model, num_hidden_layers=n_layers)
        mc = ModelConfig(cfg)
        ec = EngineConfig(block_size=16, max_blocks_per_seq=w.block_table.shape[1])
        cos, sin = rope_cache(128, mc.rope_theta, max(w.seq_lens) + 1, dev)
        st = build_infer_state(w.seq_ids, w.seq_lens, [], mc, cos, sin, dev)
        H, I, hq, hkv, d = mc.hidden_size, mc.ffn_inter_dim, mc.num_q_heads, mc.num_kv_heads, mc.head_dim
        g = torch.Generator(device=dev).manual_seed(seed + 11)

        def rnd(*shape, scale=0.02):
            return (torch.randn(shape, device=dev, generator=g) * scale).half()
        layers = [dict(wqkv=rnd((hq + 2 * hkv) * d, H), wo=rnd(H, hq * d), wug=rnd(2 * I, H), wd=rnd(H, I),
                       n_in=(torch.rand(H, device=dev, generator=g) + 0.5).half(),
                       n_post=(torch.rand(H, device=dev, generator=g) + 0.5).half(),
                       q_norm=(torch.rand(d, device=dev, generator=g) + 0.5).half(),
                       k_norm=(torch.rand(d, device=dev, generator=g) + 0.5).half()) for _ in range(n_layers)]
        weight_bytes = sum(t.numel() * 2 for t in layers[0].values())
        stack = DecoderStack(mc, layers)
        x = rnd(w.rows, H, scale=1.0)
        res = torch.zeros_like(x)

        def fwd():
            stack.forward(x, res, w.k_cache, w.v_cache, w.block_table, ec, st, cos, sin)
        us, per = _time_graph(fwd, torch.cuda.Stream(), reps, 2)
        per = np.array(per) / n_layers
        kv = w.algorithmic_bytes()
        out[name] = {"rows": w.rows, "us_per_layer": us / n_layers,
                     "us_per_layer_p10_p50_p90": [float(np.percentile(per, q)) for q in (10, 50, 90)],
                     "weight_bytes_per_layer": weight_bytes, "kv_bytes_per_layer": kv,
                     "gbps": (weight_bytes + (kv or 0)) / (us / n_layers) / 1e3}
        stack.close()
        del w, layers, stack, x, res
        torch.cuda.empty_cache()
    return out


def measure_layer_rest(seed: int, reps: int = 50, cpu_seconds: float = 0.0):
    """The rest of the layer around the attention path, each kernel beside the
    reference's formulation on the same GPU (median of `reps` event-timed
    calls after warmup):

    * lm_head + argmax (post_layer.py:68-69: F.linear then torch.argmax) at
      the target-verify batch (16 requests x 5 rows, Qwen3-8B lm_head
      151,936 x 4096) and the draft batch (64 rows, Qwen3-0.6B 151,936 x 1024);
      algorithmic bytes = the lm_head weight, read once;
    * the FFN's up/gate projection + SiLU-and-mul in one pass
      (transformer_layer.py:199-200) at the verify batch (80 rows, Qwen3-8B
      12,288 x 2 x 4096) and the draft batch (64 rows, Qwen3-0.6B
      3072 x 2 x 1024), beside the library GEMM then this build's
      SiLU-and-mul and the reference's torch formulation; algorithmic bytes =
      the stacked weight, read once;
    * the q/k/v, O and down projections (the layer's F.linear calls) through
      this build's split-k GEMM (fp32 split partials, which the next kernel
      of the layer sums) beside torch.mm (hipBLASLt), at both batches;
      algorithmic bytes = the weight, read once;
    * fused add-RMSNorm (rmsnorm.py:39-89) and SiLU-and-mul
      (silu_and_mul.py:5-34) at the verify batch (80 tokens) and a prefill
      chunk (8,192 tokens), Qwen3-8B widths; algorithmic bytes = every element
      read and written once.

    Eager figures (`us_per_call`) are `inner` calls back to back between two
    events for both legs; `us_per_call_graph` replays this build's calls from
    a HIP graph (device time without launch gaps), which `hbm_gbps` uses for
    the element-wise kernels."""
    import itertools

    import numpy as np
    import torch
    import torch.nn.functional as F

    from nebulasd_amd.kernels import (fused_add_rmsnorm_inplace, lm_head_argmax, silu_and_mul_inplace,
                                      up_gate_silu_and_mul)

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    stream = torch.cuda.current_stream()

    def timed(fn, inner=10):
        """µs per call, eager: `inner` calls back to back between two events
        (median over `reps` groups).  Small kernels are launch-bound here, as
        the reference's eager layer is."""
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(max(3, reps // inner)):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(inner):
                fn()
            e1.record(stream)
            e1.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3 / inner)
        return float(np.median(ts))

    gstream = torch.cuda.Stream()

    def graph_us(fn, calls=20):
        """µs per call of this build's kernels replayed from a HIP graph on a
        side stream (no launch gaps; these kernels record no memset).  The
        warm-up runs on that stream, so per-stream buffers exist before the
        capture."""
        with torch.cuda.stream(gstream):
            mean, per = _time_graph(lambda: [fn() for _ in range(calls)], gstream, 20, 3)
        return float(np.median(per)) / calls

    out = {}
    for name, rows, hidden in (("lm_head_argmax_target_verify", 80, 4096), ("lm_head_argmax_draft_decode", 64, 1024)):
        vocab = 151936
        x = (torch.randn(rows, hidden, device=dev, generator=g)).half()
        w = (torch.randn(vocab, hidden, device=dev, generator=g) * 0.02).half()
        ours = timed(lambda: lm_head_argmax(x, w))
        ref = timed(lambda: torch.argmax(F.linear(x, w), dim=1))
        ours_graph = graph_us(lambda: lm_head_argmax(x, w), calls=4)
        same = float((lm_head_argmax(x, w) == torch.argmax(F.linear(x, w), dim=1)).float().mean().item())
        nbytes = vocab * hidden * 2
        cpu = None
        if cpu_seconds > 0:
            import oracle

            xn, wn32 = x.cpu().numpy(), w.cpu().numpy().astype(np.float32)
            cpu = _cpu_time(lambda: oracle.argmax_first(oracle.lm_head_logits(xn, wn32, np.float32)),
                            cpu_seconds, what=f"the numpy oracle's lm_head logits (fp32 sums) + argmax, "
                                              f"{rows} x {hidden} x {vocab}")
            del wn32
        out[name] = {"rows": rows, "hidden": hidden, "vocab": vocab, "us_per_call": ours, "cpu_baseline": cpu,
                     "us_per_call_graph": ours_graph,
                     "reference_us_per_call": ref, "speedup_vs_reference": ref / ours,
                     "hbm_gbps": nbytes / ours / 1e3, "identical_tokens_vs_reference": same,
                     "roofline": {"bound": "hbm", "achieved": nbytes / ours / 1e3, "peak": HBM_PEAK_GBPS,
                                  "unit": "GB/s", "frac": nbytes / ours / 1e3 / HBM_PEAK_GBPS}}
        del x, w
    torch.cuda.empty_cache()
    for name, rows, hidden, inter in (("up_gate_silu_and_mul_target_verify", 80, 4096, 12288),
                                      ("up_gate_silu_and_mul_draft_decode", 64, 1024, 3072)):
        # weight sets used in turn, together past the 256 MB MALL, so every
        # call reads its weight from HBM
        nbytes = 2 * inter * hidden * 2
        n_sets = max(2, -(-600_000_000 // nbytes))
        ws = [(torch.randn(2 * inter, hidden, device=dev, generator=g) * 0.03).half() for _ in range(n_sets)]
        x = torch.randn(rows, hidden, device=dev, generator=g).half()
        h = torch.empty(rows, inter, device=dev, dtype=torch.float16)
        wturn = itertools.cycle(range(n_sets))

        def ours_ug():
            up_gate_silu_and_mul(x, ws[next(wturn)], out=h)

        def lib_ug():  # the library GEMM, then this build's SiLU-and-mul
            ug = F.linear(x, ws[next(wturn)])
            silu_and_mul_inplace(ug)

        def ref_ug():  # the reference's formulation in torch
            ug = F.linear(x, ws[next(wturn)])
            ug[:, :inter] = ug[:, :inter] * F.silu(ug[:, inter:].float()).half()
        ours = timed(ours_ug)
        lib = timed(lib_ug)
        ref = timed(ref_ug)
        ours_graph = graph_us(ours_ug, calls=n_sets)
        ug = F.linear(x, ws[0])
        silu_and_mul_inplace(ug)
        diff = float((up_gate_silu_and_mul(x, ws[0]).float() - ug[:, :inter].float()).abs().max().item())
        out[name] = {"rows": rows, "hidden": hidden, "inter": inter, "us_per_call": ours,
                     "us_per_call_graph": ours_graph, "library_gemm_then_silu_us_per_call": lib,
                     "reference_us_per_call": ref, "speedup_vs_reference": ref / ours,
                     "speedup_vs_library_gemm_then_silu": lib / ours, "hbm_gbps": nbytes / ours_graph / 1e3,
                     "max_abs_diff_vs_library_gemm_then_silu": diff,
                     "roofline": {"bound": "hbm", "achieved": nbytes / ours_graph / 1e3, "peak": HBM_PEAK_GBPS,
                                  "unit": "GB/s", "frac": nbytes / ours_graph / 1e3 / HBM_PEAK_GBPS}}
        del ws, x, h, ug
    torch.cuda.empty_cache()
    from nebulasd_amd.kernels import linear_partials, linear_splits, sum_partials

    for name, rows, n_out, n_in in (("proj_qkv_target_verify", 80, 6144, 4096),
                                    ("proj_o_target_verify", 80, 4096, 4096),
                                    ("proj_down_target_verify", 80, 4096, 12288),
                                    ("proj_qkv_draft_decode", 64, 4096, 1024),
                                    ("proj_o_draft_decode", 64, 1024, 2048),
                                    ("proj_down_draft_decode", 64, 1024, 3072)):
        # weight sets used in turn, together past the 256 MB MALL
        nbytes = n_out * n_in * 2
        n_sets = max(2, -(-600_000_000 // nbytes))
        ws = [(torch.randn(n_out, n_in, device=dev, generator=g) * 0.03).half() for _ in range(n_sets)]
        x = torch.randn(rows, n_in, device=dev, generator=g).half()
        splits = linear_splits(rows, n_out, n_in)
        part = torch.empty((splits, rows, n_out), device=dev, dtype=torch.float32)
        y = torch.empty((rows, n_out), device=dev, dtype=torch.float16)
        wturn = itertools.cycle(range(n_sets))

        def ours_proj():
            linear_partials(x, ws[next(wturn)], part)

        def lib_proj():  # F.linear (hipBLASLt), as the reference's linear()
            torch.mm(x, ws[next(wturn)].t(), out=y)
        ours = timed(ours_proj)
        lib = timed(lib_proj)
        ours_graph = graph_us(ours_proj, calls=n_sets)
        lib_graph = graph_us(lib_proj, calls=n_sets)
        diff = float((sum_partials(linear_partials(x, ws[0])).float() - F.linear(x, ws[0]).float()).abs().max())
        out[name] = {"rows": rows, "n_out": n_out, "n_in": n_in, "splits": splits, "us_per_call": ours,
                     "us_per_call_graph": ours_graph, "library_us_per_call": lib,
                     "library_us_per_call_graph": lib_graph, "speedup_vs_library_graph": lib_graph / ours_graph,
                     "partial_bytes": splits * rows * n_out * 4, "hbm_gbps": nbytes / ours_graph / 1e3,
                     "max_abs_diff_vs_library": diff,
                     "roofline": {"bound": "hbm", "achieved": nbytes / ours_graph / 1e3, "peak": HBM_PEAK_GBPS,
                                  "unit": "GB/s", "frac": nbytes / ours_graph / 1e3 / HBM_PEAK_GBPS}}
        del ws, x, part, y
    torch.cuda.empty_cache()
    hidden, inter = 4096, 12288
    for tokens in (80, 8192):
        # three (x, residual) sets used in turn: 402 MB at 8,192 tokens, more
        # than the 256 MB MALL, so each call reads HBM
        sets = [(torch.randn(tokens, hidden, device=dev, generator=g).half(),
                 torch.randn(tokens, hidden, device=dev, generator=g).half()) for _ in range(3)]
        wn = (torch.rand(hidden, device=dev, generator=g) + 0.5).half()
        turn = itertools.cycle(range(3))

        def ours_norm():
            x, r = sets[next(turn)]
            fused_add_rmsnorm_inplace(x, r, wn, 1e-6)

        def ref_norm():
            x, r = sets[next(turn)]
            r.add_(x)
            x.copy_(F.rms_norm(r.float(), (hidden,), wn.float(), 1e-6).half())
        ours = timed(ours_norm)
        ours_graph = graph_us(ours_norm, calls=21)
        ref = timed(ref_norm)
        cpu = None
        if cpu_seconds > 0:
            import oracle

            xn, rn, wnn = sets[0][0].cpu().numpy(), sets[0][1].cpu().numpy(), wn.cpu().numpy()
            cpu = _cpu_time(lambda: oracle.fused_add_rmsnorm(xn, rn, wnn, 1e-6), cpu_seconds,
                            what=f"the numpy oracle's fused add-RMSNorm, {tokens} x {hidden}")
        nbytes = 4 * tokens * hidden * 2
        out[f"fused_add_rmsnorm_{tokens}_tokens"] = {
            "us_per_call": ours, "us_per_call_graph": ours_graph, "reference_us_per_call": ref,
            "speedup_vs_reference": ref / ours, "hbm_gbps": nbytes / ours_graph / 1e3, "cpu_baseline": cpu}
        # two buffers used in turn (804 MB at 8,192 tokens); the gate half is
        # centred near 1.3 so repeated in-place calls keep the up half finite
        ugs = [torch.randn(tokens, 2 * inter, device=dev, generator=g).half() for _ in range(2)]
        for ug in ugs:
            ug[:, inter:] = 1.28
        sturn = itertools.cycle(range(2))

        def ours_silu():
            silu_and_mul_inplace(ugs[next(sturn)])

        def ref_silu():
            ug = ugs[next(sturn)]
            ug[:, :inter] = ug[:, :inter] * F.silu(ug[:, inter:].float()).half()
        ours_s = timed(ours_silu)
        ref_s = timed(ref_silu)
        ours_g = graph_us(ours_silu)
        cpu = None
        if cpu_seconds > 0:
            import oracle

            un = ugs[0].cpu().numpy()
            cpu = _cpu_time(lambda: oracle.silu_and_mul(un), cpu_seconds,
                            what=f"the numpy oracle's SiLU-and-mul, {tokens} x {inter}")
        nbytes = tokens * inter * 2 * 3
        out[f"silu_and_mul_{tokens}_tokens"] = {
            "us_per_call": ours_s, "us_per_call_graph": ours_g, "reference_us_per_call": ref_s,
            "speedup_vs_reference": ref_s / ours_s, "hbm_gbps": nbytes / ours_g / 1e3, "cpu_baseline": cpu}
        del sets, ugs
    torch.cuda.empty_cache()
    return {"workload": "layer_rest", "kind": "rest_of_layer", **out}


def traffic_from_profiles(workload: str):
    """HBM bytes per attention launch for `workload`, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (already scaled by the copy
    calibration), or None when no row matches."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 5 and parts[0] == workload and not line.startswith("#"):
                try:
                    return float(parts[4])
                except ValueError:
                    return None
    return None


def copy_probe(nbytes: int = 1 << 30, reps: int = 10) -> float:
    """Achievable HBM rate of a plain device copy (read + write bytes / time), GB/s."""
    import torch

    src = torch.empty(nbytes // 2, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1.0)
    dst.copy_(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    sec = start.elapsed_time(end) / 1e3 / reps
    del src, dst
    torch.cuda.empty_cache()
    return 2 * nbytes / sec / 1e9


STREAM_PROBE_BYTES = 4 << 30


def stream_read_probe(steps: int) -> dict:
    """Contiguous read of a 4 GiB buffer (nsd_probe_stream_read_unroll): the
    device's sequential-read rate, swept over the grid (1-16 workgroups per
    CU) and the 16-byte loads in flight per thread (1, 4, 8); each point is
    the mean over `steps` graph replays.  `gbps` is the best point."""
    import torch

    from nebulasd_amd import _lib

    buf = torch.empty(STREAM_PROBE_BYTES // 2, dtype=torch.float16, device="cuda")
    buf.normal_()
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sweep = []
    for unroll in (1, 4, 8):
        for per_cu in (1, 2, 4, 8, 16):
            grid = per_cu * cus

            def one(grid=grid, unroll=unroll):
                _lib.call("nsd_probe_stream_read_unroll", buf.data_ptr(), STREAM_PROBE_BYTES, sink.data_ptr(),
                          grid, unroll, torch.cuda.current_stream().cuda_stream)
            us, _ = _time_graph(one, torch.cuda.Stream(), max(3, steps), 2)
            sweep.append({"grid": grid, "unroll": unroll, "us": us, "gbps": STREAM_PROBE_BYTES / us / 1e3})
    del buf
    torch.cuda.empty_cache()
    best = max(sweep, key=lambda r: r["gbps"])
    return {"bytes": STREAM_PROBE_BYTES, "us": best["us"], "gbps": best["gbps"],
            "frac_of_peak": best["gbps"] / HBM_PEAK_GBPS, "best": dict(best), "sweep": sweep}


def empty_launch_probe(steps: int) -> dict:
    """A kernel that does nothing (nsd_probe_empty), 36 launches per graph
    replay: the cost of one more launch inside a captured forward, for one
    workgroup and for a grid of two per CU."""
    import torch

    from nebulasd_amd import _lib

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    out = {}
    for name, grid in (("one_workgroup", 1), ("two_per_cu", 2 * cus)):
        def one(grid=grid):
            st = torch.cuda.current_stream().cuda_stream
            for _ in range(36):
                _lib.call("nsd_probe_empty", grid, st)
        us, _ = _time_graph(one, torch.cuda.Stream(), max(5, steps), 2)
        out[name] = us / 36
    out["us_per_launch"] = out["two_per_cu"]
    return out


def attention_tiles(w, layer: int):
    """Element offsets of the K (= V) tiles one attention call of workload
    `w` reads at `layer`: every (sequence, kv head, block) its rows reach,
    ordered by sequence, head, block."""
    import numpy as np

    n_layers, hkv, bs = w.k_cache.shape[1], w.k_cache.shape[2], w.k_cache.shape[3]
    tile = bs * w.k_cache.shape[4]
    bt = w.block_table.cpu().numpy().astype(np.int64)
    need = {}
    for sid, n in zip(w.seq_ids, w.seq_lens):
        need[sid] = max(need.get(sid, 0), (int(n) + bs - 1) // bs)
    return np.concatenate([((bt[sid, :nb] * n_layers + layer) * hkv + h) * tile
                           for sid, nb in need.items() for h in range(hkv)])


def attention_segments(w) -> list:
    """(first tile, tiles) of every (sequence, kv head) segment, in the order
    of attention_tiles."""
    bs, hkv = w.k_cache.shape[3], w.k_cache.shape[2]
    need = {}
    for sid, n in zip(w.seq_ids, w.seq_lens):
        need[sid] = max(need.get(sid, 0), (int(n) + bs - 1) // bs)
    segs, pos = [], 0
    for nb in need.values():
        for _ in range(hkv):
            segs.append((pos, nb))
            pos += nb
    return segs


def chunk_pieces(segs, chunk: int) -> list:
    """Every segment cut into near-equal pieces of at most `chunk` tiles,
    longest first (as the hardware then dispatches them)."""
    import numpy as np

    pieces = []
    for s, n in segs:
        k = -(-n // chunk)
        cuts = np.rint(np.linspace(0, n, k + 1)).astype(int)
        pieces += [(s + int(a), s + int(b)) for a, b in zip(cuts[:-1], cuts[1:])]
    pieces.sort(key=lambda p: -(p[1] - p[0]))
    return pieces


# LDS pad that leaves `per_cu` workgroups of the given LDS use on one CU.
def _lds_pad(base: int, per_cu: int) -> int:
    return max(0, {2: 80, 3: 53, 4: 40}[per_cu] * 1024 - base)


# The gather mechanisms of gather_probes: name -> (probe, pieces, arguments).
# "split" cuts the tile stream evenly over two workgroups per CU; "chunkN"
# cuts every segment into pieces of at most N tiles.
GATHER_PROBES = {
    "lds_ring_2_per_cu": ("tile_gather", "split", ()),
    "lds_ring_3_per_cu": ("gather_pieces", "chunk8", ("ring", 6, 3)),
    "lds_ring_4_per_cu": ("gather_pieces", "chunk4", ("ring", 4, 4)),
    "registers": ("gather_vgpr", "chunk8", (1,)),
    "wave_private_registers": ("gather_wave", "chunk16", (1, 0, 0, 0)),
    "wave_private_lds_dma_2_per_cu": ("gather_wave", "chunk16", (1, 0, 1, 2)),
}


def gather_probes(w, steps: int, warmup: int) -> dict:
    """The K/V tiles that workload `w`'s attention reads, one launch per
    layer over all layers, gathered with no arithmetic by each mechanism of
    GATHER_PROBES: an LDS ring filled by DMA at 2, 3 and 4 workgroups per CU,
    16-byte loads straight into registers, and waves streaming on their own
    (no barriers) into registers or into a double buffer of their own in LDS
    (the attention kernel's mechanism).  The fastest is the attention's K/V
    read floor on this device (`us_per_layer_call`, `gbps`)."""
    import numpy as np
    import torch

    from nebulasd_amd import _lib

    n_layers = w.k_cache.shape[1]
    base = np.stack([attention_tiles(w, layer) for layer in range(n_layers)])  # [L, n_tiles]
    n_tiles = base.shape[1]
    segs = attention_segments(w)
    assert sum(n for _, n in segs) == n_tiles
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    dev = w.k_cache.device
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    ce = w.k_cache.numel()
    assert int(base.max()) + 2048 <= ce and int(base.min()) >= 0
    kv_bytes = n_tiles * 2 * 2048 * w.k_cache.element_size()
    out = {}
    for name, (probe, split, extra) in GATHER_PROBES.items():
        if split == "split":
            workers = 2 * cus
            while -(-n_tiles // workers) > 1536:
                workers *= 2
            starts = np.rint(np.linspace(0, n_tiles, workers + 1)).astype(np.int64)
            order = np.arange(n_tiles)
        else:
            pieces = chunk_pieces(segs, int(split[5:]))
            assert max(b - a for a, b in pieces) <= 256
            order = np.concatenate([np.arange(a, b) for a, b in pieces])
            starts = np.concatenate([[0], np.cumsum([b - a for a, b in pieces])]).astype(np.int64)
        n_p = len(starts) - 1
        tiles = torch.from_numpy(np.ascontiguousarray(base[:, order]).reshape(-1)).to(dev)
        pst = torch.from_numpy(starts).to(dev)

        def one_pass(probe=probe, extra=extra, tiles=tiles, pst=pst, n_p=n_p):
            st = torch.cuda.current_stream().cuda_stream
            for layer in range(n_layers):
                tp = tiles.data_ptr() + layer * n_tiles * 8
                common = (w.k_cache.data_ptr(), w.v_cache.data_ptr(), ce, tp, n_tiles, pst.data_ptr(), n_p)
                if probe == "tile_gather":
                    _lib.call("nsd_probe_tile_gather", *common, sink.data_ptr(), st)
                elif probe == "gather_pieces":
                    ring, per_cu = extra[1], extra[2]
                    _lib.call("nsd_probe_gather_pieces", *common, ring,
                              _lds_pad(ring * 8192 + 2048, per_cu), sink.data_ptr(), st)
                elif probe == "gather_vgpr":
                    _lib.call("nsd_probe_gather_vgpr", *common, extra[0], sink.data_ptr(), st)
                else:
                    rnd, kmode, vmode, per_cu = extra
                    pad = _lds_pad(2048 + 4 * 2 * rnd * 4096, per_cu) if vmode else 0
                    _lib.call("nsd_probe_gather_wave", *common, rnd, kmode, vmode, pad, sink.data_ptr(), st)
        us_pass, per = _time_graph(one_pass, torch.cuda.Stream(), max(1, steps), max(0, warmup))
        us = us_pass / n_layers
        out[name] = {"workgroups": n_p, "us_per_layer_call": us, "gbps": kv_bytes / us / 1e3}
        del tiles, pst
    best = min(out, key=lambda k: out[k]["us_per_layer_call"])
    return {"tiles_per_layer_call": n_tiles, "kv_bytes": kv_bytes, "mechanisms": out,
            "best": dict(out[best], mechanism=best), "us_per_layer_call": out[best]["us_per_layer_call"],
            "gbps": out[best]["gbps"], "frac_of_peak": out[best]["gbps"] / HBM_PEAK_GBPS,
            "same_mechanism_us": out["wave_private_lds_dma_2_per_cu"]["us_per_layer_call"]}


def with_gather_floor(res: dict, w, steps: int, warmup: int) -> None:
    """Adds the gather probes of workload `w` to its leg `res`: the floor,
    the attention's fraction of it, and of the floor of its own mechanism."""
    fl = gather_probes(w, steps, warmup)
    res["kv_gather_floor"] = fl
    res["frac_of_gather_floor"] = fl["us_per_layer_call"] / res["us_per_layer_call"]
    res["frac_of_same_mechanism_floor"] = fl["same_mechanism_us"] / res["us_per_layer_call"]


def measure_spec_loop(seed: int, steps: int, cpu_seconds: float) -> dict:
    """The attention at the shapes the single-GPU speculative loop produces.

    Runs the loop (random-init Qwen3-0.6B draft + Qwen3-8B target, draft
    batch 64, target batch 16, depth 4, prompts U[128, 1024]) over 64
    requests x 16 generated tokens; every 5th forward hands its mid-depth
    attention call to a timer that replays a HIP graph of that forward's
    attention over all of the model's layers (`steps` timed passes, the
    forward's own rows, lengths and caches).  Reports µs per layer call at
    the observed draft and target shapes, the CPU baseline at one sampled
    shape of each, and the loop's own counters.  Then runs the same loop
    twice more with no sampling, its decode/verify layers once through the
    native decoder stack and once from Python, and reports the decode
    tokens per second of each (`throughput`).
    """
    import numpy as np
    import torch

    from nebulasd_amd.infer_state import build_infer_state
    from nebulasd_amd.kernels import paged_attention
    from nebulasd_amd.spec_loop import run

    dev = torch.device("cuda:0")
    samples = {"draft": [], "target": []}
    cpu = {}
    stream = torch.cuda.Stream()

    def make_timer():
        def timer(model, layer, q, o, lse, seq_ids, seq_lens):
            mc = model.mc
            role = "draft" if mc.num_layers == 28 else "target"
            st = build_infer_state(seq_ids, seq_lens, [], mc, model.cos, model.sin, dev)
            out = torch.empty_like(q)

            def attn_pass():
                for li in range(mc.num_layers):
                    paged_attention(q, model.k_cache, model.v_cache, model.block_table, mc, model.ec,
                                    st, li, out)
            us_pass, _ = _time_graph(attn_pass, stream, max(1, steps // 4), 1)
            us = us_pass / mc.num_layers
            per_seq = {}
            for sid, n in zip(seq_ids, seq_lens):
                per_seq[sid] = max(per_seq.get(sid, 0), n)
            hkv, hq = mc.num_kv_heads, mc.num_q_heads
            kv_tokens = sum(per_seq.values())
            nbytes = (kv_tokens * hkv * 128 * 2 * 2 + len(seq_ids) * hq * 128 * 2 * 2
                      + sum((n + 15) // 16 for n in per_seq.values()) * 4)
            _, counts = np.unique(np.asarray(seq_ids), return_counts=True)
            samples[role].append({"rows": len(seq_ids), "max_q_len": int(counts.max()),
                                  "kv_tokens": kv_tokens, "us_per_layer_call": us,
                                  "gbps": nbytes / us / 1e3})
            if cpu_seconds > 0 and role not in cpu and len(seq_ids) == (64 if role == "draft" else 80):
                cpu[role] = cpu_attention_baseline(q, model.k_cache, model.v_cache, model.block_table,
                                                   seq_ids, seq_lens, layer, cpu_seconds,
                                                   f"the loop's {role} forward ({len(seq_ids)} rows)")
        return timer

    t0 = time.perf_counter()
    res = run(n_requests=64, prompt_lo=128, prompt_hi=1024, new_tokens=16, draft_batch=64,
              target_batch=16, depth=4, seed=seed, check_every=5, make_check=make_timer, device=dev)
    wall = time.perf_counter() - t0
    out = {"workload": "spec_loop_shapes", "loop": {k: v for k, v in res.items()},
           "bench_wall_s": wall}
    thr = {}
    for name, native, overlap in (("native_decoder_stack", True, True), ("native_one_stream", True, False),
                                  ("python_layers", False, True)):
        r = run(n_requests=128, prompt_lo=128, prompt_hi=1024, new_tokens=32, draft_batch=64, target_batch=16,
                depth=4, seed=seed, device=dev, native=native, overlap=overlap)
        thr[name] = {
            "decode_tokens_per_s": r["decode_tokens_per_s"], "wall_s": r["wall_s"], "prefill_s": r["prefill_s"],
            "rounds": r["rounds"], "generated_tokens": r["generated_tokens"]}
        torch.cuda.empty_cache()
    out["throughput"] = dict(thr, config="128 requests x 32 generated tokens, prompts U[128, 1024], draft batch 64 "
                                         "(two draft groups per round), target batch 16, depth 4, no sampled "
                                         "checks; draft and target forwards on two streams except "
                                         "native_one_stream")
    for role, xs in samples.items():
        if not xs:
            continue
        us = np.array([x["us_per_layer_call"] for x in xs])
        out[role] = {"samples": len(xs), "us_per_layer_call_median": float(np.median(us)),
                     "us_per_layer_call_min": float(us.min()), "us_per_layer_call_max": float(us.max()),
                     "gbps_median": float(np.median([x["gbps"] for x in xs])),
                     "rows": sorted({x["rows"] for x in xs}),
                     "kv_tokens_median": float(np.median([x["kv_tokens"] for x in xs])),
                     "cpu_baseline": cpu.get(role)}
    torch.cuda.empty_cache()
    return out


def _cpu_threads() -> int:
    """The host cores this process may run on (its CPU affinity)."""
    return len(os.sched_getaffinity(0))


def cpu_attention_baseline(q, k_cache, v_cache, block_table, seq_ids, seq_lens, layer: int,
                           budget_s: float, what: str) -> dict:
    """Time the PyTorch-CPU fp32 restatement of the reference's row-wise
    attention (oracle/attention_torch.py) on the referenced blocks of one
    layer, on every affinity core; median of calls within ~budget_s seconds."""
    import numpy as np
    import torch

    from oracle.attention_torch import paged_attention_rowwise

    bs = k_cache.shape[3]
    bt = block_table.cpu().numpy()
    ids = sorted({int(bt[s, i]) for s, n in zip(seq_ids, seq_lens) for i in range((n + bs - 1) // bs)})
    remap = np.zeros(k_cache.shape[0], dtype=np.int64)
    remap[ids] = np.arange(len(ids))
    idx = torch.tensor(ids, device=k_cache.device)
    kc = k_cache[idx, layer].unsqueeze(1).cpu()
    vc = v_cache[idx, layer].unsqueeze(1).cpu()
    bt_s = torch.from_numpy(remap[bt])
    qc = q.cpu()
    threads_before = torch.get_num_threads()
    cores = _cpu_threads()
    torch.set_num_threads(cores)
    times = []
    try:
        t_end = time.perf_counter() + budget_s
        while True:
            t0 = time.perf_counter()
            paged_attention_rowwise(qc, kc, vc, bt_s, seq_ids, seq_lens, 0)
            times.append(time.perf_counter() - t0)
            if time.perf_counter() > t_end or len(times) >= 20:
                break
        used = torch.get_num_threads()
    finally:
        torch.set_num_threads(threads_before)
    return {
        "value": float(np.median(times)) * 1e6,
        "unit": "us/layer-call",
        "cores": int(used),
        "affinity_cores": cores,
        "kind": "port",
        "sample": f"{len(times)} layer calls of {what} (one layer, the same inputs as the GPU run), "
                  "PyTorch-CPU fp32 row-wise attention, median",
        "cpu_model": _cpu_model(),
    }


def cpu_baseline(w, budget_s: float):
    """CPU baseline of workload `w` at its middle layer."""
    return cpu_attention_baseline(w.q, w.k_cache, w.v_cache, w.block_table, w.seq_ids, w.seq_lens,
                                  w.spec.num_layers // 2, budget_s, w.spec.name)


def _cpu_time(fn, budget_s: float, max_reps: int = 20, what: str = "") -> dict:
    """Median wall time of fn() on the affinity cores, at least one call and
    about `budget_s` seconds."""
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits

    cores = _cpu_threads()
    times = []
    with threadpool_limits(limits=cores):
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
        t_end = time.perf_counter() + budget_s
        while True:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
            if time.perf_counter() > t_end or len(times) >= max_reps:
                break
    return {"value": float(np.median(times)) * 1e6, "unit": "us/call", "cores": int(min(threads, cores)),
            "kind": "port", "sample": f"{len(times)} calls of {what}, median", "cpu_model": _cpu_model()}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# The stdout line is read back from a bounded tail of the run's output: it
# keeps the headline, the roofline, the CPU baseline, the probes and a few
# scalar figures per secondary leg, and stays under this many bytes.  The
# full per-leg results go to stderr as one "# detail " JSON line.
LINE_MAX_BYTES = 7500
# Scalar figures a secondary leg keeps on the stdout line, when it has them.
LEG_KEYS = ("us_per_layer_call", "hbm_gbps", "hbm_frac", "frac_of_gather_floor", "frac_of_same_mechanism_floor",
            "tflops", "mfma_frac",
            "us_per_write", "reference_us_per_write", "us_per_layer", "floor_us_at_copy_rate",
            "reference_sdpa_loop_us", "us_per_call", "reference_us_per_call", "us_per_call_graph",
            "prologue_plus_attention_us", "fused_layer_us")
# Second-level dicts of a leg whose scalar figures are kept as well.
LEG_SUBKEYS = ("kv_gather_floor", "native_decoder_stack", "throughput", "draft", "target", "D2H", "H2D")


def _sig(x):
    """x rounded to 5 significant digits (ints and non-numbers unchanged)."""
    if isinstance(x, bool) or not isinstance(x, float):
        return x
    return float(f"{x:.5g}")


def _compact_cpu(c):
    if not isinstance(c, dict):
        return None
    return {k: _sig(c[k]) for k in ("value", "unit", "cores", "kind") if k in c}


def _layer_note(r: dict) -> str:
    """Prologue + attention per layer: two launches, and one fused launch."""
    fused = r.get("fused_layer_us")
    return (f"; with the prologue {r['prologue_plus_attention_us']:.2f} us (two launches), "
            + (f"{fused:.2f} us (one fused launch)" if fused is not None else "no fused launch for this plan"))


def _scalars(d: dict, keys) -> dict:
    return {k: _sig(d[k]) for k in keys if isinstance(d.get(k), (int, float)) and not isinstance(d.get(k), bool)}


def compact_leg(r: dict) -> dict:
    """The figures of one secondary leg that the stdout line keeps."""
    out = _scalars(r, LEG_KEYS)
    for sub in LEG_SUBKEYS:
        v = r.get(sub)
        if not isinstance(v, dict):
            continue
        s = _scalars(v, LEG_KEYS + ("decode_tokens_per_s", "us_per_layer_call_median", "gbps", "kernel_gbps",
                                    "dma_gbps", "reference_gbps"))
        for k2, v2 in v.items():  # one more level (e.g. throughput variants, per-shape layers)
            if isinstance(v2, dict):
                s2 = _scalars(v2, ("decode_tokens_per_s", "us_per_layer", "us_per_call"))
                if s2:
                    s[k2] = s2
        if sub == "kv_gather_floor":  # the floor's mechanism and every mechanism's time
            if isinstance(v.get("best"), dict):
                s["best"] = v["best"].get("mechanism")
            if isinstance(v.get("mechanisms"), dict):
                s["mechanisms_us"] = {k2: _sig(m.get("us_per_layer_call")) for k2, m in v["mechanisms"].items()
                                      if isinstance(m, dict)}
        if s:
            out[sub] = s
    for k, v in r.items():  # rest-of-layer legs: one dict per kernel and shape
        if k not in LEG_SUBKEYS and isinstance(v, dict) and "us_per_call" in v:
            out[k] = _scalars(v, ("us_per_call", "reference_us_per_call", "us_per_call_graph",
                                  "library_us_per_call_graph", "gbps"))
    cpu = _compact_cpu(r.get("cpu_baseline"))
    if cpu:
        out["cpu_baseline"] = cpu
    return out


PROBE_KEYS = ("gbps", "frac_of_peak", "us", "us_per_launch", "us_per_layer_call", "best_gbps", "workgroups",
              "grid", "unroll", "ring", "per_cu")


def _compact_probes(probes: dict) -> dict:
    """Probe figures for the stdout line: the scalars of each probe and of
    its best sweep point (sweeps themselves stay in the detail line)."""
    out = {}
    for name, p in probes.items():
        if not isinstance(p, dict):
            out[name] = _sig(p)
            continue
        s = _scalars(p, PROBE_KEYS)
        for k, v in p.items():
            if isinstance(v, dict) and k.startswith("best"):
                s[k] = _scalars(v, PROBE_KEYS)
        out[name] = s
    return out


def stdout_line(line: dict, secondary: dict) -> str:
    """The JSON line for stdout: `line` plus the compact secondary legs,
    dropping leg detail (then whole legs, last first) until it fits in
    LINE_MAX_BYTES."""
    legs = {name: compact_leg(r) for name, r in secondary.items()}
    out = dict(line, secondary=legs)
    text = json.dumps(out)
    if len(text.encode()) <= LINE_MAX_BYTES:
        return text
    for name in legs:  # keep only the top-level scalars and the CPU baseline
        legs[name] = {k: v for k, v in legs[name].items() if not isinstance(v, dict) or k == "cpu_baseline"}
    text = json.dumps(out)
    for name in reversed(list(legs)):
        if len(text.encode()) <= LINE_MAX_BYTES:
            break
        del legs[name]
        text = json.dumps(out)
    return text


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(every box has a single MI355X)", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    from nebulasd_amd import _lib

    if not _lib.LIB_PATH.exists():
        from nebulasd_amd.build import build

        build()
    copy_gbps = copy_probe()
    probes = {"copy_gbps": copy_gbps}
    if args.probes:
        probes["stream_read"] = stream_read_probe(args.steps)
        probes["empty_launch_in_graph"] = empty_launch_probe(args.steps)
        print(f"# probes: contiguous read {probes['stream_read']['gbps']:.0f} GB/s "
              f"(grid {probes['stream_read']['best']['grid']}, {probes['stream_read']['best']['unroll']} loads "
              f"in flight), copy {copy_gbps:.0f} GB/s, empty launch in a graph "
              f"{probes['empty_launch_in_graph']['us_per_launch']:.2f} us", file=sys.stderr, flush=True)
    res, w = measure(args.workload, args.seed, args.steps, args.warmup)
    if args.probes:
        with_gather_floor(res, w, args.steps, args.warmup)
    print(f"# {args.workload}: {res['us_per_layer_call']:.2f} us/layer-call, "
          f"{res['hbm_gbps']:.0f} GB/s" + (f" (K/V gather floor {res['kv_gather_floor']['us_per_layer_call']:.2f} us)"
                                          if args.probes else "") + _layer_note(res), file=sys.stderr, flush=True)
    cpu = None
    if args.cpu_baseline_seconds > 0:
        cpu = cpu_baseline(w, args.cpu_baseline_seconds)
    spec = w.spec
    del w
    torch.cuda.empty_cache()
    secondary = {}
    # the other attention workloads first, right after the headline: the
    # path's own legs, measured before the longer widening legs load the GPU
    for name in filter(None, args.secondary.split(",")):
        r2, w2 = measure(name, args.seed, args.steps, args.warmup)
        if args.probes:
            with_gather_floor(r2, w2, args.steps, args.warmup)
        print(f"# {name}: {r2['us_per_layer_call']:.2f} us/layer-call, "
              f"{r2['hbm_gbps']:.0f} GB/s" + _layer_note(r2), file=sys.stderr, flush=True)
        if args.cpu_baseline_seconds > 0:
            r2["cpu_baseline"] = cpu_baseline(w2, args.other_cpu_seconds)
        secondary[name] = r2
        del w2
        torch.cuda.empty_cache()
    for name in filter(None, args.prefill.split(",")):
        r2 = measure_prefill(name, args.seed, args.steps, args.warmup, args.other_cpu_seconds
                             if args.cpu_baseline_seconds > 0 else 0)
        print(f"# {name}: {r2['us_per_layer_call']:.2f} us/layer-call, {r2['tflops']:.0f} TFLOP/s "
              f"(reference SDPA loop {r2['reference_sdpa_loop_us']:.0f} us)", file=sys.stderr, flush=True)
        secondary[name] = r2
    if args.block_table:
        r2 = measure_block_table(args.seed, cpu_seconds=min(1.0, args.other_cpu_seconds) if args.cpu_baseline_seconds > 0 else 0)
        print(f"# block table bank switch: {r2['us_per_write']:.1f} us per write "
              f"(reference formulation {r2['reference_us_per_write']:.1f} us)", file=sys.stderr, flush=True)
        secondary[r2["workload"]] = r2
    if args.layer_step:
        measure_layer_step.copy_gbps = copy_gbps
        r2 = measure_layer_step(args.seed)
        r2["native_decoder_stack"] = nat = measure_native_layers(args.seed)
        print("# native decoder stack: target verify %.1f us/layer (%d rows), draft decode %.1f us/layer (%d rows)"
              % (nat["target_verify"]["us_per_layer"], nat["target_verify"]["rows"],
                 nat["draft_decode"]["us_per_layer"], nat["draft_decode"]["rows"]), file=sys.stderr, flush=True)
        print("# target verify layer: %.1f us (three q/k/v GEMMs %.1f; library up/gate GEMM + SiLU-mul %.1f; "
              "GEMMs alone %.1f, rest alone %.1f; floor %s us)"
              % (r2["us_per_layer"], r2["us_per_layer_three_qkv_gemms"], r2["us_per_layer_unfused_ffn"],
                 r2["gemms_only_us"], r2["rest_only_us"],
                 "%.1f" % r2["floor_us_at_copy_rate"] if r2["floor_us_at_copy_rate"] else "n/a"),
              file=sys.stderr, flush=True)
        secondary[r2["workload"]] = r2
    if args.layer_rest:
        r2 = measure_layer_rest(args.seed, cpu_seconds=args.other_cpu_seconds if args.cpu_baseline_seconds > 0 else 0)
        print("# rest of layer: lm_head+argmax verify %.1f us (reference %.1f), draft %.1f us (reference %.1f); "
              "up/gate+silu-mul verify %.1f us (library GEMM + silu-mul %.1f), draft %.1f us (%.1f); "
              "add-rmsnorm 8192 tok %.1f us (reference %.1f); silu-mul 8192 tok %.1f us (reference %.1f)" % (
                  r2["lm_head_argmax_target_verify"]["us_per_call"],
                  r2["lm_head_argmax_target_verify"]["reference_us_per_call"],
                  r2["lm_head_argmax_draft_decode"]["us_per_call"],
                  r2["lm_head_argmax_draft_decode"]["reference_us_per_call"],
                  r2["up_gate_silu_and_mul_target_verify"]["us_per_call"],
                  r2["up_gate_silu_and_mul_target_verify"]["library_gemm_then_silu_us_per_call"],
                  r2["up_gate_silu_and_mul_draft_decode"]["us_per_call"],
                  r2["up_gate_silu_and_mul_draft_decode"]["library_gemm_then_silu_us_per_call"],
                  r2["fused_add_rmsnorm_8192_tokens"]["us_per_call"],
                  r2["fused_add_rmsnorm_8192_tokens"]["reference_us_per_call"],
                  r2["silu_and_mul_8192_tokens"]["us_per_call"],
                  r2["silu_and_mul_8192_tokens"]["reference_us_per_call"]), file=sys.stderr, flush=True)
        print("# projections (split-k / torch.mm, graph us): " + "; ".join(
            f"{n[5:]} {r2[n]['us_per_call_graph']:.1f} / {r2[n]['library_us_per_call_graph']:.1f}"
            for n in r2 if n.startswith("proj_")), file=sys.stderr, flush=True)
        secondary[r2["workload"]] = r2
    if args.hostkv:
        r2 = measure_hostkv(args.seed)
        print("# hostkv copy (GB/s, reference / dma / kernel): " + "; ".join(
            f"{d} {r2[d]['reference_gbps']:.1f} / {r2[d]['dma_gbps']:.1f} / {r2[d]['kernel_gbps']:.1f}"
            for d in ("D2H", "H2D")) + "; scattered swap-in dma / kernel: "
            f"{r2['swap_128_scattered_blocks']['in']['dma_gbps']:.1f} / "
            f"{r2['swap_128_scattered_blocks']['in']['kernel_gbps']:.1f}", file=sys.stderr, flush=True)
        secondary[r2["workload"]] = r2
    if args.spec_loop:
        r2 = measure_spec_loop(args.seed, args.steps, args.other_cpu_seconds if args.cpu_baseline_seconds > 0 else 0)
        print("# speculative loop shapes: " + "; ".join(
            f"{role} {r2[role]['us_per_layer_call_median']:.1f} us/layer-call over {r2[role]['samples']} forwards"
            for role in ("draft", "target") if role in r2) + "; decode %.0f tokens/s (native decoder stack, "
              "draft and target streams), %.0f (one stream), %.0f (layers from Python)"
              % tuple(r2["throughput"][k]["decode_tokens_per_s"]
                      for k in ("native_decoder_stack", "native_one_stream", "python_layers")),
              file=sys.stderr, flush=True)
        secondary[r2["workload"]] = r2
    line = {
        "metric": "verify/decode attn µs per layer + HBM GB/s (% peak), Qwen3-8B B=16 q_len=5",
        "value": res["us_per_layer_call"],
        "unit": "us/layer-call",
        "n_gpus": 1,
        "steps": res["steps"],
        "warmup": args.warmup,
        "ms_per_step": res["us_per_pass"] / 1e3,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": f"{args.workload}: Qwen3-8B attention shape (32q/8kv heads, d=128), B={spec.batch}, "
                        f"q_len={spec.q_len}, contexts {spec.ctx[0]} [{spec.ctx[1]},{spec.ctx[2]}], "
                        f"block 16, pool {spec.pool_blocks} blocks, layers cycled 0..{spec.num_layers - 1}; "
                        f"a step is one pass of {spec.num_layers} layer calls",
            "batch": spec.batch,
            "q_len": spec.q_len,
            "seed": args.seed,
        },
        "hbm_gbps": res["hbm_gbps"],
        "hbm_frac": res["hbm_frac"],
        "tokens_per_s": res["tokens_per_s"],
        "roofline": {
            "bound": "hbm",
            "achieved": res["hbm_gbps"],
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": res["hbm_frac"],
            "traffic": traffic_from_profiles(args.workload),
            "kernels": "paged_attn_kernel (+ combine_table_kernel, the merge of split segments), one layer call",
        },
        "copy_probe_gbps": copy_gbps,
        "probes": _compact_probes(probes),
        "cpu_baseline": cpu,
        "detail": compact_leg(res),
    }
    print("# detail " + json.dumps({"detail": res, "probes": probes, "secondary": secondary}),
          file=sys.stderr, flush=True)
    print(stdout_line(line, secondary), flush=True)


if __name__ == "__main__":
    main()
