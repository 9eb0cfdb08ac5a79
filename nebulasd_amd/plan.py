"""Per-forward attention work plan (host side).

The reference re-derives its launch grid on every layer call from a split
size chosen once per forward (swiftLLM/swiftllm/worker/model.py:365-384,
kernels/paged_attn.py:182-211).  Here the whole work decomposition -- verify
groups, per-workgroup chunk ranges and partial slots -- is computed once per
forward by the native planner ``nsd_attn_plan_build`` from the host copies of
the decode rows' seq_ids / seq_lens, uploaded once, and reused by every layer.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib

PIECE_WORDS = 12
MAX_GROUP_ROWS = 48   # query rows of one (group, kv head): three 16-row tiles in one wave
XCDS = 8              # workgroup i of a launch runs on XCD i % 8
_workers_cache: dict[tuple[int, int], int] = {}


def num_workers(max_rows: int, device_index: int | None = None) -> int:
    """Wave slots of the current GPU (CUs x attention workgroups per CU) for
    plans with ``max_rows`` rows per group: the planner cuts the block
    stream into about this many pieces."""
    import torch

    dev = torch.cuda.current_device() if device_index is None else device_index
    nt = (max_rows + 15) // 16
    key = (dev, nt)
    if key not in _workers_cache:
        out = ctypes.c_int(0)
        with torch.cuda.device(dev):
            _lib.call("nsd_attn_num_workers", 16 * nt, ctypes.byref(out))
        _workers_cache[key] = int(out.value)
    return _workers_cache[key]


# Pieces the planner cuts per workgroup slot.  One per slot binds every
# piece to a workgroup and starts them all at once, the planner pairing a
# long piece with a short one on every CU; more make the slots' worth of
# longest pieces bound and the rest claimed at run time by the workgroups
# that start as slots free up (a faster XCD takes more of them), at the
# price of more pieces to start, merge and combine.  Measured (graph-timed
# layer calls, settings interleaved on one box): decode 54.3 / 57.5 us at
# 1 / 2 per slot, ragged verify (three 16-row tiles) 104.4-109.4 /
# 108.0-111.7 us at 1 / 1.5, verify 34.0 / 36.1 us at 1 / 1.25.  A batch
# with more segments than slots still has its pieces beyond the slots
# claimed (a segment is never shared by two pieces' worth of rows).
PIECES_PER_SLOT = {1: 1.0, 2: 1.0, 3: 1.0}


def pieces_for(slots: int, max_rows: int) -> int:
    """The n_workers the planner is given for a device with `slots`
    workgroup slots, for groups of at most `max_rows` query rows."""
    per = PIECES_PER_SLOT
    f = per if isinstance(per, (int, float)) else per[min(3, (max_rows + 15) // 16)]
    return max(1, int(round(slots * f)))


def plan_words(seq_ids, seq_lens, num_q_heads: int, num_kv_heads: int, head_dim: int,
               block_size: int, bt_rows: int, bt_stride: int, n_workers: int,
               max_group_rows: int = 0, static_slots: int = 0) -> tuple[np.ndarray, int]:
    """Run the native planner on host lists; returns (plan words int32, workspace bytes).
    ``static_slots`` > 0: pieces beyond that many are claimed at run time."""
    sid = np.ascontiguousarray(np.asarray(seq_ids, dtype=np.int32))
    sl = np.ascontiguousarray(np.asarray(seq_lens, dtype=np.int32))
    if sid.shape != sl.shape or sid.ndim != 1:
        raise ValueError("seq_ids and seq_lens must be 1-D of equal length")
    lib = _lib.load()
    cap = lib.nsd_attn_plan_bound(len(sid), num_kv_heads, n_workers)
    if cap < 0:
        raise ValueError(f"bad plan bound arguments (rows={len(sid)}, hkv={num_kv_heads}, "
                         f"workers={n_workers})")
    i32p = ctypes.POINTER(ctypes.c_int32)
    for _ in range(2):  # the bound assumes n_workers; a plan that needs more reports its size
        buf = np.zeros(cap, dtype=np.int32)
        words = ctypes.c_int64(0)
        ws = ctypes.c_int64(0)
        rc = lib.nsd_attn_plan_build_claimed(
            sid.ctypes.data_as(i32p), sl.ctypes.data_as(i32p), len(sid), num_q_heads,
            num_kv_heads, head_dim, block_size, bt_rows, bt_stride, n_workers, static_slots,
            max_group_rows, buf.ctypes.data_as(i32p), cap, ctypes.byref(words), ctypes.byref(ws))
        if rc == _lib.NSD_ERR_WORKSPACE and words.value > cap:
            cap = words.value
            continue
        _lib.check(rc, "nsd_attn_plan_build")
        return buf[: words.value].copy(), int(ws.value)
    raise _lib.NativeLibraryError("nsd_attn_plan_build: plan size did not converge")


def decode_plan(words: np.ndarray) -> dict:
    """Split plan words into named numpy views (for inspection and tests).

    ``records`` holds the pieces: the first ``static`` in dispatch order
    (record i runs on workgroup i, XCD i % 8; records with q_len 0 are
    empty), then ``claimed`` more in the order the later workgroups claim
    them; ``pieces`` lists the non-empty ones in that order.
    """
    h = words[:_lib.PLAN_HEADER_WORDS]
    n_groups, n_records = int(h[_lib.PLAN_GROUPS]), int(h[_lib.PLAN_PIECES])
    n_comb = int(h[_lib.PLAN_COMBINES])
    og, op, oc = int(h[_lib.PLAN_OFF_GROUPS]), int(h[_lib.PLAN_OFF_PIECES]), int(h[_lib.PLAN_OFF_COMBINES])
    # {kv head, blk_begin, blk_end, slot, row_start, q_len, seq_id, ctx,
    #  combine, combine first slot, combine slots, segment}
    records = words[op:op + PIECE_WORDS * n_records].reshape(n_records, PIECE_WORDS)
    used = records[:, 5] > 0
    return {
        "rows": int(h[_lib.PLAN_ROWS]),
        "workers": int(h[_lib.PLAN_WORKERS]),
        "slots": int(h[_lib.PLAN_SLOTS]),
        "rows_max": int(h[_lib.PLAN_ROWS_MAX]),
        "sized_for": int(h[_lib.PLAN_SIZED_FOR]),
        "piece_blocks": int(h[_lib.PLAN_PIECE_BLOCKS]),
        "bt_rows": int(h[_lib.PLAN_BT_ROWS]),
        "bt_stride": int(h[_lib.PLAN_BT_STRIDE]),
        "max_blocks": int(h[_lib.PLAN_MAX_BLOCKS]),
        "static": int(h[_lib.PLAN_STATIC]),
        "claimed": int(h[_lib.PLAN_CLAIMED]),
        "groups": words[og:og + 4 * n_groups].reshape(n_groups, 4),
        "records": records,
        "pieces": records[used],
        "record_index": np.nonzero(used)[0],
        # {kv head, first_slot, n_slots, row_start, q_len, 0 ...}
        "combines": words[oc:oc + PIECE_WORDS * n_comb].reshape(n_comb, PIECE_WORDS),
    }


@dataclass
class AttnPlan:
    """A plan resident on the host and on one GPU, plus its partial workspace."""

    host: np.ndarray          # int32 plan words
    dev: "object"             # torch.int32 tensor on the GPU (same words)
    workspace: "object"       # torch.uint8 tensor (>= workspace_bytes), or None
    workspace_bytes: int
    num_q_heads: int
    num_kv_heads: int

    @property
    def rows_max(self) -> int:
        return int(self.host[_lib.PLAN_ROWS_MAX])

    @property
    def n_rows(self) -> int:
        return int(self.host[_lib.PLAN_ROWS])

    @property
    def keeps_sequences_whole(self) -> bool:
        """Whether every sequence's rows sit in one verify group, as the
        prologue inside the attention launch (``paged_attention_fused``) needs."""
        h = self.host
        n, og = int(h[_lib.PLAN_GROUPS]), int(h[_lib.PLAN_OFF_GROUPS])
        sids = h[og:og + 4 * n].reshape(n, 4)[:, 2]
        return len(np.unique(sids)) == n

    def fits(self, num_q_heads: int, num_kv_heads: int, block_table) -> bool:
        """Whether this plan serves calls with these head counts and block table
        (the table has the row stride the plan was built for and at least its rows)."""
        return (self.num_q_heads == num_q_heads and self.num_kv_heads == num_kv_heads
                and int(self.host[_lib.PLAN_BT_STRIDE]) == block_table.shape[1]
                and int(self.host[_lib.PLAN_BT_ROWS]) <= block_table.shape[0])

    def host_ptr(self):
        return self.host.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def build_attn_plan(seq_ids, seq_lens, num_q_heads: int, num_kv_heads: int, head_dim: int,
                    block_size: int, bt_rows: int, bt_stride: int, device,
                    n_workers: int | None = None, max_group_rows: int = 0) -> AttnPlan:
    """Plan + upload for the decode rows of one forward.

    ``seq_ids`` / ``seq_lens``: host sequences (the decode rows' block-table
    rows and lengths, model.py:329-341).  ``max_group_rows = 1`` disables
    verify grouping (pure row-wise decode, as the reference launches it).
    """
    import torch

    device = torch.device(device)
    gqa = num_q_heads // num_kv_heads
    sized = n_workers is None
    slots = 0
    if sized:
        # size the pieces for the row-tile count the grouping will produce
        guess = min(MAX_GROUP_ROWS, gqa * max(1, (max_group_rows or MAX_GROUP_ROWS) // gqa))
        slots = num_workers(guess, device.index)
        n_workers = pieces_for(slots, guess)
    words, ws = plan_words(seq_ids, seq_lens, num_q_heads, num_kv_heads, head_dim, block_size,
                           bt_rows, bt_stride, n_workers, max_group_rows, slots)
    rows_max = int(words[_lib.PLAN_ROWS_MAX])
    if sized and rows_max > 0 and n_workers != pieces_for(num_workers(rows_max, device.index), rows_max):
        slots = num_workers(rows_max, device.index)
        words, ws = plan_words(seq_ids, seq_lens, num_q_heads, num_kv_heads, head_dim,
                               block_size, bt_rows, bt_stride, pieces_for(slots, rows_max), max_group_rows,
                               slots)
    # pinned and non-blocking: the upload does not wait for the stream
    # (the caching host allocator keeps the pinned block until the copy ran)
    src = torch.from_numpy(words)
    dev = (src.pin_memory().to(device, non_blocking=True) if device.type == "cuda"
           else src.to(device))
    # the claim counter (zero before the first call; every call leaves it
    # zero) and the split segments' partials
    workspace = torch.zeros(max(ws, 256), dtype=torch.uint8, device=device)
    return AttnPlan(words, dev, workspace, ws, num_q_heads, num_kv_heads)


def plan_for(infer_state, model_config, engine_config, block_table) -> AttnPlan:
    """The attention plan of one forward, for this package's ``LlamaInferState``
    or for swiftLLM's own (swiftLLM/swiftllm/worker/infer_state.py:4-29).

    A foreign infer state gets the plan attached as an attribute on first use
    (every layer of the forward then reuses it).  Its decode rows are read
    from ``seq_ids_list`` / ``decoding_seq_lens_list`` when the caller set
    them (the host lists model.py:304-341 already holds), otherwise copied
    from the device tensors once per forward.
    """
    getter = getattr(infer_state, "get_attn_plan", None)
    if getter is not None:
        return getter(model_config, engine_config, block_table)
    plan = getattr(infer_state, "nsd_attn_plan", None)
    if plan is not None and plan.fits(model_config.num_q_heads, model_config.num_kv_heads,
                                      block_table):
        return plan
    npf = int(infer_state.num_prefill_seqs)
    sids = getattr(infer_state, "seq_ids_list", None)
    slens = getattr(infer_state, "decoding_seq_lens_list", None)
    if sids is None:
        sids = infer_state.seq_ids[npf:].cpu().tolist()
    if slens is None:
        slens = infer_state.decoding_seq_lens.cpu().tolist()
    plan = build_attn_plan(sids, slens, model_config.num_q_heads, model_config.num_kv_heads,
                           model_config.head_dim, engine_config.block_size, block_table.shape[0],
                           block_table.shape[1], block_table.device,
                           max_group_rows=int(getattr(infer_state, "max_group_rows", 0)))
    infer_state.nsd_attn_plan = plan
    return plan
