"""Host-side tests of the C-ABI library (no GPU calls): symbol exports,
argument validation, and the attention planner's invariants."""

from __future__ import annotations

import ctypes
import json
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))
GOLDEN = json.loads((Path(__file__).parent / "golden" / "speculative_cases.json").read_text())


@pytest.fixture(scope="module")
def lib():
    from nebulasd_amd import _lib

    if not _lib.LIB_PATH.exists():
        from nebulasd_amd.build import build

        build()
    return _lib.load()


def header_functions() -> list[str]:
    text = "".join(h.read_text() for h in HEADERS)
    return sorted(set(re.findall(r"^(?:int|int64_t|const char\*)\s+(nsd_\w+)\(", text, re.M)))


def test_library_exports_every_header_symbol(lib):
    from nebulasd_amd import _lib

    names = header_functions()
    assert len(names) >= 11
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/ but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert lib.nsd_version() >= 100


def test_error_paths_without_gpu(lib):
    from nebulasd_amd import _lib

    # unsupported head_dim is rejected before any HIP call
    rc = lib.nsd_store_kvcache(None, None, None, None, None, 1, 1, None, None, 1, 1, 1, 0, 8, 64,
                               16, None, None)
    assert rc == 2 and "head_dim=64" in _lib.last_error()
    rc = lib.nsd_store_kvcache(None, None, None, None, None, 1, 1, None, None, 1, 1, 2, 5, 8, 128,
                               16, None, None)
    assert rc == 1 and "layer=5" in _lib.last_error()
    rc = lib.nsd_rmsnorm_inplace(None, None, 4, 128, 1e-6, None)
    assert rc == 1 and "null" in _lib.last_error()
    # zero rows: nothing to launch
    assert lib.nsd_rmsnorm_inplace(None, None, 0, 128, 1e-6, None) == 0
    plan = np.zeros(16, np.int32)
    rc = lib.nsd_paged_attention(None, None, None, None, None, 1, 1, 0, 32, 8, 128, 16, None, 1,
                                 1, plan.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), None,
                                 None, 0, 0.1, None, None)
    assert rc == 1 and "null plan" in _lib.last_error()
    rc = lib.nsd_paged_attention(None, None, None, None, None, 1, 1, 0, 32, 8, 128, 16, None, 1,
                                 1, plan.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                 plan.ctypes.data, None, 0, 0.1, None, None)
    assert rc == 1 and "not a plan" in _lib.last_error()


# planner constants (nebulasd_amd/csrc/nsd_common.h, nsd_host.cpp)
MAX_WORKER_PIECES, MAX_WORKER_BLOCKS, MIN_PIECE_BLOCKS, PIECE_COST = 4, 1024, 4, 3


def _plan(seq_ids, seq_lens, hq=32, hkv=8, workers=64, max_group_rows=0, bt_rows=None, stride=4096):
    from nebulasd_amd.plan import decode_plan, plan_words

    words, ws = plan_words(seq_ids, seq_lens, hq, hkv, 128, 16, bt_rows or (max(seq_ids) + 1),
                           stride, workers, max_group_rows)
    p = decode_plan(words)
    p["requested_workers"] = workers
    return p, ws


def check_plan_invariants(p, seq_ids, seq_lens, hkv, gqa):
    groups, pieces, ws = p["groups"], p["pieces"], p["worker_start"]
    # groups tile the rows in order with seq_len rising by one inside a group
    r = 0
    for row_start, q_len, sid, ctx in groups:
        assert row_start == r and q_len >= 1 and q_len * gqa <= 64
        for i in range(q_len):
            assert seq_ids[r + i] == sid and seq_lens[r + i] == ctx + 1 + i
        r += q_len
    assert r == len(seq_lens)
    # segment = (group, kv head), in stream order; blocks of 16 tokens
    seg_of = {(int(g[0]), h): i * hkv + h for i, g in enumerate(groups) for h in range(hkv)}
    nblk = [(-(-(int(g[3]) + int(g[1])) // 16)) for g in groups for _ in range(hkv)]
    covered = [np.zeros(n, int) for n in nblk]
    last = (-1, -1)
    for w in range(p["workers"]):
        for pc in range(ws[w], ws[w + 1]):
            h, bb, be, slot, row_start, q_len, sid, ctx, comb, cfirst, cslots, gend = (
                int(x) for x in pieces[pc])
            seg = seg_of[(row_start, h)]
            g = groups[seg // hkv]
            assert (q_len, sid, ctx) == (int(g[1]), int(g[2]), int(g[3]))
            assert 0 <= bb < be <= nblk[seg]
            assert (seg, bb) > last
            last = (seg, be - 1)
            covered[seg][bb:be] += 1
    assert all((c == 1).all() for c in covered)
    # slots exactly for segments cut into several pieces
    per_seg = {}
    for pcs in pieces:
        per_seg.setdefault((int(pcs[4]), int(pcs[0])), []).append(int(pcs[3]))
    combined = {(int(c[3]), int(c[0])): (int(c[1]), int(c[2])) for c in p["combines"]}
    for key, slots in per_seg.items():
        assert len(slots) <= 128
        if len(slots) == 1:
            assert slots == [-1] and key not in combined
        else:
            first, n = combined[key]
            assert slots == list(range(first, first + n))
    # each piece of a split segment names its combine record and slot range
    for pcs in pieces:
        comb, cfirst, cslots = int(pcs[8]), int(pcs[9]), int(pcs[10])
        if int(pcs[3]) < 0:
            assert (comb, cfirst, cslots) == (-1, 0, 0)
        else:
            c = p["combines"][comb]
            assert (int(c[3]), int(c[0])) == (int(pcs[4]), int(pcs[0]))
            assert (cfirst, cslots) == (int(c[1]), int(c[2]))
            assert cfirst <= int(pcs[3]) < cfirst + cslots
    # records sit at a fixed stride per worker (zero records in the gaps);
    # the worker table holds each worker's record range and first record
    stride, recs = p["piece_stride"], p["records"]
    assert len(recs) == p["workers"] * stride
    for w in range(p["workers"]):
        row = p["workers_table"][w]
        n = ws[w + 1] - ws[w]
        assert (row[0], row[1]) == (w * stride, w * stride + n) and n <= stride
        assert (recs[w * stride:w * stride + n] == pieces[ws[w]:ws[w + 1]]).all()
        assert (recs[w * stride + n:(w + 1) * stride] == 0).all()
        if n:
            assert list(row[2:14]) == list(pieces[ws[w]])
    # each record counts the blocks of its worker's earlier pieces (the offset
    # of its block ids in the worker's id list)
    blocks = []
    for w in range(p["workers"]):
        run = 0
        for pc in range(ws[w], ws[w + 1]):
            assert int(pieces[pc][11]) == run
            run += int(pieces[pc][2] - pieces[pc][1])
        blocks.append(run)
    assert p["max_blocks"] == max(blocks)
    # planner limits: pieces and blocks per worker
    for w in range(p["workers"]):
        assert ws[w + 1] - ws[w] <= MAX_WORKER_PIECES and blocks[w] <= MAX_WORKER_BLOCKS
    # near-equal cost per active worker within each dispatch half (blocks
    # plus 3 per piece; the first half's cap 1.5% above the second's); only
    # the last active worker, or one stopped by the piece or block limit,
    # may fall short
    cost = [sum(int(pieces[pc][2] - pieces[pc][1]) + PIECE_COST for pc in range(ws[w], ws[w + 1]))
            for w in range(p["workers"])]
    active = [w for w in range(p["workers"]) if cost[w] > 0]
    half = p.get("requested_workers", p["workers"]) // 2
    for part in ([w for w in active if w < half], [w for w in active if w >= half]):
        if not part:
            continue
        top = max(cost[w] for w in part)
        for w in part:
            if w == active[-1]:
                continue
            assert cost[w] >= top - (PIECE_COST + MIN_PIECE_BLOCKS) or \
                ws[w + 1] - ws[w] == MAX_WORKER_PIECES or blocks[w] == MAX_WORKER_BLOCKS, \
                (w, cost[w], top)
    assert p["workers"] % 8 == 0


def test_plan_caps_pieces_per_segment(lib):
    # one 32k request over many workers: at most 128 pieces per (group, kv head)
    p, _ = _plan([0], [32768], workers=100000, stride=4096)
    check_plan_invariants(p, [0], [32768], 8, 4)
    assert max(int(c[2]) for c in p["combines"]) <= 128


def test_plan_groups_reference_literal_rows(lib):
    case = GOLDEN["linear_rows"][0]
    p, _ = _plan([3, 3, 3, 3], case["expect_seq_lens"])
    assert p["groups"].tolist() == [[0, 4, 3, 102]]
    check_plan_invariants(p, [3] * 4, case["expect_seq_lens"], 8, 4)


def test_plan_rowwise_mode(lib):
    lens = [103, 104, 105, 106]
    p, _ = _plan([3] * 4, lens, max_group_rows=1)
    assert p["groups"].tolist() == [[i, 1, 3, lens[i] - 1] for i in range(4)]
    check_plan_invariants(p, [3] * 4, lens, 8, 4)


@pytest.mark.parametrize("seed", range(6))
def test_plan_invariants_random(lib, seed):
    rng = np.random.default_rng(seed)
    seq_ids, seq_lens = [], []
    for sid in range(rng.integers(1, 40)):
        ctx = int(rng.integers(0, 5000))
        q = int(rng.integers(1, 20))
        seq_ids += [sid] * q
        seq_lens += list(range(ctx + 1, ctx + q + 1))
    # a broken run (not rising by one) must split into groups
    seq_ids += [99, 99]
    seq_lens += [50, 50]
    workers = int(rng.choice([8, 64, 256, 1000]))
    for hq, hkv in ((32, 8), (16, 8), (8, 8)):
        p, ws = _plan(seq_ids, seq_lens, hq, hkv, workers, bt_rows=100)
        check_plan_invariants(p, seq_ids, seq_lens, hkv, hq // hkv)
        # partials: fp16 O (128 x 2 bytes) + fp32 lse per slot row
        part = -(-p["slots"] * p["rows_max"] * (128 * 2 + 4) // 256) * 256
        assert ws == (part if len(p["combines"]) else 0)


def test_plan_splits_long_groups(lib):
    # q_len 20 with GQA 4 -> 80 rows > 64: split into 16 + 4
    lens = list(range(501, 521))
    p, _ = _plan([0] * 20, lens)
    assert p["groups"].tolist() == [[0, 16, 0, 500], [16, 4, 0, 516]]
    assert p["rows_max"] == 64


@pytest.mark.parametrize("bad", [
    dict(seq_lens=[0]), dict(seq_lens=[4097]), dict(seq_ids=[5]), dict(seq_ids=[-1]),
])
def test_plan_rejects_bad_rows(lib, bad):
    from nebulasd_amd import _lib
    from nebulasd_amd.plan import plan_words

    args = dict(seq_ids=[0], seq_lens=[10])
    args.update(bad)
    with pytest.raises(_lib.NativeLibraryError):
        plan_words(args["seq_ids"], args["seq_lens"], 32, 8, 128, 16, 2, 256, 64)


def test_plan_rejects_unsupported_shapes(lib):
    from nebulasd_amd import _lib
    from nebulasd_amd.plan import plan_words

    with pytest.raises(_lib.NativeLibraryError, match="head_dim"):
        plan_words([0], [10], 32, 8, 64, 16, 1, 256, 64)
    with pytest.raises(_lib.NativeLibraryError, match="block_size"):
        plan_words([0], [10], 32, 8, 128, 32, 1, 256, 64)
    with pytest.raises(_lib.NativeLibraryError, match="multiple"):
        plan_words([0], [10], 30, 8, 128, 16, 1, 256, 64)


def test_plan_empty(lib):
    from nebulasd_amd.plan import decode_plan, plan_words

    words, ws = plan_words([], [], 32, 8, 128, 16, 1, 16, 64)
    p = decode_plan(words)
    assert p["workers"] == 0 and len(p["pieces"]) == 0 and ws == 0


def test_package_speculative_matches_golden():
    from nebulasd_amd import speculative as sp

    for case in GOLDEN["linear_rows"]:
        assert sp.build_linear_verification_rows(case["prompt_len"], case["output_token_ids"],
                                                 case["draft_token_ids"]) == \
            (case["expect_tokens"], case["expect_seq_lens"])
    for case in GOLDEN["greedy_acceptance"]:
        assert sp.compute_greedy_acceptance(case["draft"], case["posterior"], case["remaining"],
                                            case["stops"]) == (case["expect"], case["count"])
    c = GOLDEN["aggregate_max_lens"]
    assert sp.aggregate_max_lens_by_seq_id(c["seq_ids"], c["seq_lens"]) == \
        {int(k): v for k, v in c["expect"].items()}
    with pytest.raises(ValueError, match="non-negative"):
        sp.compute_greedy_acceptance([1], [1, 2], -1)


def test_qwen3_shape_constants():
    from nebulasd_amd.config import QWEN3_8B, ModelConfig

    g = GOLDEN["qwen3_8b_shape"]
    cfg = ModelConfig(QWEN3_8B)
    assert (cfg.num_q_heads, cfg.num_kv_heads, cfg.hidden_size, cfg.head_dim, cfg.vocab_size) == \
        (g["num_q_heads"], g["num_kv_heads"], g["hidden_size"], g["head_dim"], g["vocab_size"])
    assert cfg.rope_theta == g["rope_theta"] and cfg.rms_norm_eps == g["rms_norm_eps"]
    assert cfg.has_qk_norm


def test_plan_respects_kernel_limits(lib):
    # thousands of one-block segments: at most 32 pieces per worker, so the
    # plan grows past the requested 8 workers
    n = 2000
    p, _ = _plan(list(range(n)), [1] * n, hq=16, hkv=8, workers=8, bt_rows=n, stride=16)
    check_plan_invariants(p, list(range(n)), [1] * n, 8, 2)
    assert p["workers"] > 8
    # one long request asked onto one worker: no worker streams more than
    # 1024 blocks (its LDS id list), so the 8 x 4000 blocks take 32 workers
    p, _ = _plan([0], [16 * 4000], workers=1, stride=4096)
    check_plan_invariants(p, [0], [16 * 4000], 8, 4)
    assert p["max_blocks"] == MAX_WORKER_BLOCKS
    assert sum(1 for w in range(p["workers"]) if p["worker_start"][w + 1] > p["worker_start"][w]) \
        == 32


def _attention_with_plan(lib, words, hq=32, hkv=8, bt_rows=2, bt_stride=4096):
    """Call nsd_paged_attention with host buffers standing in for device ones.

    Only the host-side plan checks run: every call here must be rejected
    before any HIP call (a plan that passes would fail at the launch)."""
    i32p = ctypes.POINTER(ctypes.c_int32)
    buf = np.zeros(1 << 16, np.uint8)  # 16-byte aligned stand-in pointer
    p = buf.ctypes.data + (-buf.ctypes.data) % 16
    ws = np.zeros(1 << 22, np.uint8)
    wp = ws.ctypes.data + (-ws.ctypes.data) % 16
    return lib.nsd_paged_attention(p, p, None, p, p, 1000, 2, 0, hq, hkv, 128, 16, p, bt_rows,
                                   bt_stride, words.ctypes.data_as(i32p), p, wp, ws.size - 16,
                                   128 ** -0.5, None, None)


@pytest.mark.skipif(Path("/dev/kfd").exists(),
                    reason="passes host buffers as device pointers: only where no GPU can run it")
def test_attention_rejects_corrupt_plans(lib):
    """The kernel claims blocks from the records it is given: the launch
    checks stride, block counts, block-table shape, slots and row counts first."""
    from nebulasd_amd import _lib
    from nebulasd_amd.plan import PIECE_WORDS, plan_words

    sid, sl = [0] * 5 + [1] * 5, [3000 + i for i in range(1, 6)] + [900 + i for i in range(1, 6)]
    words, _ = plan_words(sid, sl, 32, 8, 128, 16, 2, 4096, 16)
    h = words[:_lib.PLAN_HEADER_WORDS]
    op = int(h[_lib.PLAN_OFF_PIECES])
    split = next(i for i in range(int(h[_lib.PLAN_PIECES]))
                 if words[op + PIECE_WORDS * i + 3] >= 0)  # a piece with a partial slot

    def corrupt(idx, value):
        w = words.copy()
        w[idx] = value
        return w

    cases = [
        (corrupt(_lib.PLAN_MAX_BLOCKS, 0), "header"),
        (corrupt(_lib.PLAN_PIECE_STRIDE, 0), "header"),
        (corrupt(_lib.PLAN_PIECES, int(h[_lib.PLAN_PIECES]) + 1), "header"),
        (corrupt(op + 11, words[op + 11] + 1), "piece 0"),                      # block offset
        (corrupt(op + 6, 2), "piece 0"),                                        # seq_id past the table
        (corrupt(op + 2, 4096 * 2), "piece 0"),                                 # past the block table row
        (corrupt(op + 5, 64), "piece 0"),                                       # q_len * gqa > rows_max
        (corrupt(op + PIECE_WORDS * split + 3, int(h[_lib.PLAN_SLOTS])), f"piece {split}"),
        (corrupt(op, 8), "piece 0"),                                            # kv head
    ]
    for w, where in cases:
        rc = _attention_with_plan(lib, w)
        assert rc == 1, (where, rc, _lib.last_error())
        assert "corrupt plan" in _lib.last_error() and where in _lib.last_error()


def test_noalloc_rejects_plans_larger_than_its_scratch(lib):
    """A plan whose partials exceed the allocation-free entry point's static
    scratch is refused before any HIP call, with the sizes in the message."""
    from nebulasd_amd import _lib
    from nebulasd_amd.plan import plan_words

    # 32 requests x 16 verify rows (64 query rows per kv head) over 32k contexts
    # cut across 2048 workers: thousands of 64-row partial slots (> 16 MiB)
    sids = [r for r in range(32) for _ in range(16)]
    slens = [32000 + i + 1 for _ in range(32) for i in range(16)]
    words, _ = plan_words(sids, slens, 32, 8, 128, 16, 32, 2100, 2048)
    slots, rows_max = int(words[_lib.PLAN_SLOTS]), int(words[_lib.PLAN_ROWS_MAX])
    assert slots * rows_max * (128 * 2 + 4) > (16 << 20), "the plan should not fit the scratch"
    rc = lib.nsd_paged_attention_noalloc(
        None, None, None, None, None, 24576, 36, 0, 32, 8, 128, 16, None, 32, 2100,
        words.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), None, 0.088, None, None)
    assert rc == _lib.NSD_ERR_WORKSPACE and "static scratch" in _lib.last_error()
    # not a plan: rejected as such
    bad = np.zeros(_lib.PLAN_HEADER_WORDS, np.int32)
    rc = lib.nsd_paged_attention_noalloc(
        None, None, None, None, None, 1, 1, 0, 32, 8, 128, 16, None, 1, 1,
        bad.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), None, 0.088, None, None)
    assert rc == 1 and "not a plan" in _lib.last_error()


@pytest.mark.skipif(Path("/dev/kfd").exists(),
                    reason="passes host buffers as device pointers: only where no GPU can run it")
def test_attention_rejects_plan_for_another_block_table(lib):
    """A plan checked against one block-table shape is refused for a table
    with another row stride or fewer rows (its seq_ids could fall outside)."""
    from nebulasd_amd import _lib
    from nebulasd_amd.plan import plan_words

    words, _ = plan_words([0, 1], [300, 900], 32, 8, 128, 16, 2, 4096, 16)
    for rows, stride in ((1, 4096), (2, 2048)):
        assert _attention_with_plan(lib, words, bt_rows=rows, bt_stride=stride) == 1
        assert "block table" in _lib.last_error()
