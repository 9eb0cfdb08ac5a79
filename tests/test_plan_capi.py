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


# planner constants (nebulasd_amd/csrc/nsd_common.h)
MAX_PIECE_BLOCKS, MIN_PIECE_BLOCKS, MAX_SLOTS, XCDS, MAX_GROUP_ROWS = 256, 8, 128, 8, 48


def _plan(seq_ids, seq_lens, hq=32, hkv=8, workers=64, max_group_rows=0, bt_rows=None, stride=4096,
          static_slots=0):
    from nebulasd_amd.plan import decode_plan, plan_words

    words, ws = plan_words(seq_ids, seq_lens, hq, hkv, 128, 16, bt_rows or (max(seq_ids) + 1),
                           stride, workers, max_group_rows, static_slots)
    p = decode_plan(words)
    p["requested_workers"] = workers
    p["static_slots"] = static_slots
    return p, ws


def check_plan_invariants(p, seq_ids, seq_lens, hkv, gqa):
    groups, recs = p["groups"], p["records"]
    # groups tile the rows in order with seq_len rising by one inside a group
    r = 0
    for row_start, q_len, sid, ctx in groups:
        assert row_start == r and q_len >= 1 and q_len * gqa <= MAX_GROUP_ROWS
        for i in range(q_len):
            assert seq_ids[r + i] == sid and seq_lens[r + i] == ctx + 1 + i
        r += q_len
    assert r == len(seq_lens)
    # segment = (group, kv head); blocks of 16 tokens
    nblk = [(-(-(int(g[3]) + int(g[1])) // 16)) for g in groups for _ in range(hkv)]
    total = sum(nblk)
    # static records: one workgroup each, a multiple of the XCD count; each
    # XCD's records (i, i + 8, ...) are its pieces, empty ones last, and the
    # XCDs' lists differ in length by at most one.  A list is longest first,
    # unless it puts a second workgroup on some of the XCD's C CUs (C =
    # static slots / 16; positions j and j + C share a CU): then the CUs
    # with one workgroup run the longest pieces, and each CU with two pairs
    # one of the next-longest with one of the rest, longest with shortest
    # (positions 0 .. m-1 longest first, C .. C+m-1 shortest first).  Claimed
    # records follow, longest first, none longer than a static one, with
    # half again as many workgroups (rounded up to 8) to claim them.
    n_static, n_claimed = p["static"], p["claimed"]
    assert len(recs) == n_static + n_claimed and n_static % XCDS == 0
    assert p["workers"] == n_static + -(-((3 * n_claimed + 1) // 2) // XCDS) * XCDS
    claimed = recs[n_static:]
    assert (claimed[:, 5] > 0).all()
    csizes = (claimed[:, 2] - claimed[:, 1]).tolist()
    assert csizes == sorted(csizes, reverse=True)
    if n_claimed:
        assert n_static == p["static_slots"] // XCDS * XCDS
        assert min(int(r[2] - r[1]) for r in recs[:n_static] if r[5] > 0) >= csizes[0]
    load, n_live_of = [0] * XCDS, []
    covered = [np.zeros(n, int) for n in nblk]
    pieces_of = {}
    for rec in claimed:
        h, bb, be, slot, row_start, q_len, sid, ctx, comb, cfirst, cslots, seg = (int(v) for v in rec)
        assert h == seg % hkv and (row_start, q_len, sid, ctx) == tuple(int(v) for v in groups[seg // hkv])
        assert 0 <= bb < be <= nblk[seg] and be - bb <= MAX_PIECE_BLOCKS
        covered[seg][bb:be] += 1
        pieces_of.setdefault(seg, []).append((bb, be, slot, comb, cfirst, cslots))
    for x in range(XCDS):
        mine = recs[:n_static][x::XCDS]
        live = mine[:, 5] > 0
        n_live = int(live.sum())
        n_live_of.append(n_live)
        assert live[:n_live].all(), "empty records only at the end of an XCD list"
        sizes = (mine[:n_live, 2] - mine[:n_live, 1]).tolist()
        C = p["static_slots"] // (2 * XCDS)
        if C and C < n_live <= 2 * C:
            m = n_live - C
            shared, lone, second = sizes[:m], sizes[m:C], sizes[C:]
            assert lone == sorted(lone, reverse=True) and shared == sorted(shared, reverse=True)
            assert second == sorted(second)
            assert min(lone, default=max(shared)) >= max(shared) and min(shared) >= max(second)
        else:
            assert sizes == sorted(sizes, reverse=True)
        for rec in mine[:n_live]:
            h, bb, be, slot, row_start, q_len, sid, ctx, comb, cfirst, cslots, seg = (int(v) for v in rec)
            g = groups[seg // hkv]
            assert h == seg % hkv and (row_start, q_len, sid, ctx) == tuple(int(v) for v in g)
            assert 0 <= bb < be <= nblk[seg] and be - bb <= MAX_PIECE_BLOCKS
            covered[seg][bb:be] += 1
            load[x] += be - bb
            pieces_of.setdefault(seg, []).append((bb, be, slot, comb, cfirst, cslots))
        for rec in mine[n_live:]:
            assert int(rec[5]) == 0 and int(rec[3]) == -1
    assert all((c == 1).all() for c in covered)
    if nblk:
        assert max(n_live_of) - min(n_live_of) <= 1 and max(n_live_of) == n_static // XCDS
        assert max(load) - min(load) <= 2 * p["max_blocks"]
    assert p["max_blocks"] == max((int(r[2] - r[1]) for r in p["pieces"]), default=0)
    # pieces per segment: at least ceil(blocks / 256); in all, as many as the
    # planner was asked for, within the fewest the segments need and the most
    # they allow (pieces of >= 4 blocks, <= 128 per segment); extra pieces
    # went to the segments with the longest pieces (no segment still open to
    # a cut has longer pieces than a segment that got an extra one had
    # before its last)
    n_of = [len(pieces_of[s]) for s in range(len(nblk))]
    lo = [max(1, -(-n // MAX_PIECE_BLOCKS)) for n in nblk]
    hi = [max(l, min(MAX_SLOTS, n // MIN_PIECE_BLOCKS)) for l, n in zip(lo, nblk)]
    assert sum(n_of) == max(sum(lo), min(p["sized_for"], sum(hi)))
    assert p["piece_blocks"] == (-(-total // sum(n_of)) if total else 0)
    for s, (n, nb) in enumerate(zip(n_of, nblk)):
        assert lo[s] <= n <= hi[s]
        if n > lo[s]:
            for t, (m, nt) in enumerate(zip(n_of, nblk)):
                if m < hi[t]:
                    assert nt * (n - 1) <= nb * m, (s, t)
    # pieces per segment near nb / k, every piece start on a multiple of the
    # workgroup's four waves and within two blocks of j * nb / k (so only the
    # segment's last piece leaves its waves unequal block counts), unless the
    # pieces are too long for that (then within one block of each other);
    # partial slots in segment order exactly for segments cut into several
    # pieces
    combined = {(int(c[3]), int(c[0])): (int(c[1]), int(c[2])) for c in p["combines"]}
    next_slot = 0
    for seg in sorted(pieces_of):
        ps = sorted(pieces_of[seg])
        k = len(ps)
        assert k <= MAX_SLOTS
        sizes = [be - bb for bb, be, *_ in ps]
        nb = nblk[seg]
        if nb <= (MAX_PIECE_BLOCKS - 4) * k:
            starts = [bb for bb, *_ in ps]
            assert all(s0 % 4 == 0 for s0 in starts)
            assert all(abs(s0 - j * nb / k) <= 2 for j, s0 in enumerate(starts))
            assert min(sizes) >= 1 and max(sizes) <= MAX_PIECE_BLOCKS
        else:
            assert max(sizes) - min(sizes) <= 1
        key = (int(groups[seg // hkv][0]), seg % hkv)
        if k == 1:
            assert ps[0][2:] == (-1, -1, 0, 0) and key not in combined
        else:
            first, n = combined[key]
            assert (first, n) == (next_slot, k)
            assert [x[2] for x in ps] == list(range(first, first + k))
            assert all(x[4:] == (first, k) for x in ps)
            assert all(p["combines"][x[3]][0] == seg % hkv for x in ps)
            next_slot += k
    assert p["slots"] == next_slot


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
        # 256 bytes for the claim counter, then the partials: fp16 O (128 x 2
        # bytes) + fp32 lse per slot row, rounded up to 256 bytes
        part = 256 + -(-p["slots"] * p["rows_max"] * (128 * 2 + 4) // 256) * 256
        assert ws == (part if len(p["combines"]) else 0)


def test_plan_splits_long_groups(lib):
    # q_len 20 with GQA 4 -> 80 rows > 48: split into 12 + 8
    lens = list(range(501, 521))
    p, _ = _plan([0] * 20, lens)
    assert p["groups"].tolist() == [[0, 12, 0, 500], [12, 8, 0, 512]]
    assert p["rows_max"] == 48
    check_plan_invariants(p, [0] * 20, lens, 8, 4)


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
    # thousands of one-block segments: one piece each, no partials
    n = 2000
    p, ws = _plan(list(range(n)), [1] * n, hq=16, hkv=8, workers=8, bt_rows=n, stride=16)
    check_plan_invariants(p, list(range(n)), [1] * n, 8, 2)
    assert len(p["pieces"]) == n * 8 and ws == 0 and len(p["combines"]) == 0
    # one long request asked onto one slot: pieces stop at 256 blocks (four
    # waves, one block id per lane), so 4000 blocks take 16 pieces per kv head
    p, _ = _plan([0], [16 * 4000], workers=1, stride=4096)
    check_plan_invariants(p, [0], [16 * 4000], 8, 4)
    assert p["piece_blocks"] == 250 and 250 <= p["max_blocks"] <= MAX_PIECE_BLOCKS
    assert len(p["pieces"]) == 8 * 16
    # 255 blocks per piece: starts rounded to multiples of four could make a
    # piece longer than 256, so the cut stays the plain near-equal one
    p, _ = _plan([0], [16 * 4080], workers=1, stride=4096)
    check_plan_invariants(p, [0], [16 * 4080], 8, 4)
    sizes = sorted({int(r[2] - r[1]) for r in p["pieces"]})
    assert sizes == [255] and len(p["pieces"]) == 8 * 16


@pytest.mark.parametrize("slots", [64, 100, 512])
def test_plan_claimed_records(lib, slots):
    """More pieces than workgroup slots: the slots' worth of longest pieces
    are bound to workgroups, the rest claimed at run time, longest first."""
    rng = np.random.default_rng(slots)
    ctx = rng.integers(256, 4097, 16)
    sid = [i for i in range(16) for _ in range(9)]
    sl = [int(c) + 1 + k for c in ctx for k in range(9)]
    p, ws = _plan(sid, sl, workers=3 * slots // 2, bt_rows=16, static_slots=slots)
    check_plan_invariants(p, sid, sl, 8, 4)
    n_pieces = max(3 * slots // 2, 16 * 8)  # at least one piece per (request, kv head)
    assert len(p["pieces"]) == n_pieces and p["claimed"] == n_pieces - slots // 8 * 8 and ws > 0
    # nothing to claim when every piece has a slot
    p, _ = _plan(sid, sl, workers=slots, bt_rows=16, static_slots=slots)
    check_plan_invariants(p, sid, sl, 8, 4)
    if slots >= 16 * 8:
        assert p["claimed"] == 0 and p["workers"] == p["static"]


def test_plan_xcd_lists_balance(lib):
    # the verify shape: 16 requests x 8 kv heads over 8 XCDs, equal blocks per XCD
    rng = np.random.default_rng(3)
    ctx = rng.integers(256, 4097, 16)
    sid = [i for i in range(16) for _ in range(5)]
    sl = [int(c) + 1 + k for c in ctx for k in range(5)]
    p, _ = _plan(sid, sl, workers=1000, bt_rows=16)
    check_plan_invariants(p, sid, sl, 8, 4)
    recs = p["records"]
    loads = [int((recs[x::8, 2] - recs[x::8, 1])[recs[x::8, 5] > 0].sum()) for x in range(8)]
    assert max(loads) - min(loads) <= max(-(-(int(c) + 5) // 16) for c in ctx)


@pytest.mark.parametrize("seed", range(4))
def test_plan_pairs_pieces_per_cu(lib, seed):
    """The verify shape on 512 slots (32 CUs per XCD, two workgroups each):
    positions j and j + 32 of an XCD's list share a CU, and the largest CU
    total is the smallest any pairing of that XCD's pieces allows (sorted
    longest to shortest, the i-th longest paired with the i-th shortest
    minimises the largest pair sum), below that of the plain longest-first
    layout."""
    rng = np.random.default_rng(seed)
    ctx = rng.integers(256, 4097, 16)
    sid = [i for i in range(16) for _ in range(5)]
    sl = [int(c) + 1 + k for c in ctx for k in range(5)]
    p, _ = _plan(sid, sl, workers=512, bt_rows=16, static_slots=512)
    check_plan_invariants(p, sid, sl, 8, 4)
    recs = p["records"]
    for x in range(XCDS):
        sz = (recs[x::XCDS, 2] - recs[x::XCDS, 1]).astype(int)
        assert len(sz) == 64 and (sz > 0).all()
        cu = sz[:32] + sz[32:]
        srt = np.sort(sz)[::-1]
        best = max(int(srt[i] + srt[63 - i]) for i in range(32))
        plain = max(int(srt[i] + srt[32 + i]) for i in range(32))
        assert int(cu.max()) == best <= plain
        # brute force over every pairing on a small sample of the pieces
        small = [int(v) for v in srt[::8]]  # 8 pieces, 105 pairings
        def pairings(items):
            if not items:
                yield []
                return
            a = items[0]
            for k in range(1, len(items)):
                for rest in pairings(items[1:k] + items[k + 1:]):
                    yield [(a, items[k])] + rest
        opt = min(max(u + v for u, v in pr) for pr in pairings(small))
        assert opt == max(small[i] + small[7 - i] for i in range(4))


@pytest.mark.parametrize("workers", [300, 400])
def test_plan_pairs_with_single_piece_cus(lib, workers):
    """Fewer pieces than slots: each XCD list of L pieces puts a second
    workgroup on L - 32 of its 32 CUs; those CUs get the shortest first
    pieces and each pairs its long piece with a short one, and the CUs with
    one piece run the longest pieces."""
    rng = np.random.default_rng(workers)
    ctx = rng.integers(256, 4097, 16)
    sid = [i for i in range(16) for _ in range(5)]
    sl = [int(c) + 1 + k for c in ctx for k in range(5)]
    p, _ = _plan(sid, sl, workers=workers, bt_rows=16, static_slots=512)
    check_plan_invariants(p, sid, sl, 8, 4)
    recs = p["records"]
    for x in range(XCDS):
        mine = recs[x::XCDS]
        sz = (mine[:, 2] - mine[:, 1])[mine[:, 5] > 0].astype(int)
        m = len(sz) - 32
        assert 0 < m < 32
        single, first, second = sz[m:32], sz[:m], sz[32:]
        assert min(single) >= max(first) >= min(first) >= max(second)
        # the doubled CUs' largest total is the least any pairing of those pieces allows
        pool = np.sort(np.concatenate([first, second]))[::-1]
        assert int((first + second).max()) == max(int(pool[i] + pool[2 * m - 1 - i]) for i in range(m))


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
    words, _ = plan_words(sid, sl, 32, 8, 128, 16, 2, 4096, 32)
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
        (corrupt(_lib.PLAN_MAX_BLOCKS, 257), "header"),
        (corrupt(_lib.PLAN_PIECES, int(h[_lib.PLAN_PIECES]) + 1), "header"),
        (corrupt(_lib.PLAN_WORKERS, int(h[_lib.PLAN_WORKERS]) + 8), "header"),
        (corrupt(_lib.PLAN_STATIC, int(h[_lib.PLAN_STATIC]) - 3), "header"),    # not whole XCD rows
        (corrupt(_lib.PLAN_CLAIMED, 5), "header"),                              # records != static + claimed
        (corrupt(op + 2, words[op + 1] + 257), "piece 0"),                      # > 256 blocks
        (corrupt(op + 6, 2), "piece 0"),                                        # seq_id past the table
        (corrupt(op + 2, 4096 * 2), "piece 0"),                                 # past the block table row
        (corrupt(op + 5, 64), "piece 0"),                                       # q_len * gqa > rows_max
        (corrupt(op + 7, -1), "piece 0"),                                       # negative context
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


@pytest.mark.skipif(Path("/dev/kfd").exists(),
                    reason="passes host buffers as device pointers: only where no GPU can run it")
def test_fused_attention_rejects_bad_rows_before_launch(lib):
    """The fused prologue + attention entry point refuses, before any HIP
    call: misaligned or badly strided q/k/v rows, one norm weight without the
    other, bad split counts, positions past the RoPE tables, and a plan that
    splits one sequence's rows over several verify groups."""
    from nebulasd_amd import _lib
    from nebulasd_amd.plan import plan_words

    i32p = ctypes.POINTER(ctypes.c_int32)
    buf = np.zeros(1 << 16, np.uint8)
    p = buf.ctypes.data + (-buf.ctypes.data) % 16  # 16-byte aligned stand-in pointer
    ws = np.zeros(1 << 22, np.uint8)
    wp = ws.ctypes.data + (-ws.ctypes.data) % 16
    hq, hkv, qs, kvs = 32, 8, 48 * 128, 48 * 128
    sid = [0] * 5 + [1] * 5
    sl = [3000 + i for i in range(1, 6)] + [900 + i for i in range(1, 6)]
    words, _ = plan_words(sid, sl, hq, hkv, 128, 16, 2, 4096, 32)

    def call(q=p, k=p + 4096, v=p + 8192, ks=kvs, vs=kvs, part=None, splits=0, qn=p, kn=p, n_pos=4096,
             plan=words):
        return lib.nsd_paged_attention_fused(
            q, qs, k, ks, v, vs, part, splits, qn, kn, 1e-6, p, p, n_pos, p, None, p, p, 1000, 2, 0, hq, hkv,
            128, 16, p, 2, 4096, plan.ctypes.data_as(i32p), p, wp, ws.size - 16, 128 ** -0.5, None, None)

    for kwargs, msg in (({"k": p + 4098}, "16-byte aligned"), ({"v": p + 8200 + 2}, "16-byte aligned"),
                        ({"vs": kvs + 4}, "multiples of 8"), ({"ks": 1000}, "multiples of 8"),
                        ({"kn": None}, "both norm weights"), ({"part": p, "splits": 17}, "splits=17"),
                        ({"n_pos": 3004}, "outside the 3004-row RoPE tables")):
        assert call(**kwargs) == 1, (kwargs, _lib.last_error())
        assert msg in _lib.last_error(), (kwargs, _lib.last_error())
    # 17 rows of one request at GQA 4 exceed one 48-row group: the plan splits it
    split, _ = plan_words([0] * 17, [500 + i for i in range(1, 18)], hq, hkv, 128, 16, 1, 4096, 32,
                          max_group_rows=48)
    assert int(split[_lib.PLAN_GROUPS]) > 1
    assert call(plan=split) == 2, _lib.last_error()  # NSD_ERR_UNSUPPORTED
    assert "several verify groups" in _lib.last_error()


def test_plan_reports_whole_sequences(lib):
    """AttnPlan.keeps_sequences_whole: true when every sequence's rows sit in
    one verify group (what the fused prologue + attention launch needs),
    false for a request whose 17 rows at GQA 4 (68 rows) the planner splits
    over 48-row groups; it agrees with the native entry point's own check."""
    from nebulasd_amd.plan import AttnPlan, plan_words

    def plan(sids, slens, max_group_rows=0):
        words, ws = plan_words(sids, slens, 32, 8, 128, 16, 4, 4096, 32, max_group_rows=max_group_rows)
        return AttnPlan(host=words, dev=None, workspace=None, workspace_bytes=ws, num_q_heads=32, num_kv_heads=8)

    whole = plan([0] * 5 + [1] * 5 + [3], [300 + i for i in range(1, 6)] + [900 + i for i in range(1, 6)] + [50])
    assert whole.keeps_sequences_whole
    split = plan([2] * 17, [500 + i for i in range(1, 18)], max_group_rows=48)
    from nebulasd_amd import _lib

    assert int(split.host[_lib.PLAN_GROUPS]) > 1 and not split.keeps_sequences_whole
