"""ctypes binding of the gfx950 C-ABI library ``_lib/libnsd_attn.so``.

The library is built in-tree by ``nebulasd_amd.build``.  There is no CPU
fallback: if the library is missing every entry point raises
:class:`NativeLibraryError`.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libnsd_attn.so"

NSD_OK = 0
NSD_ERR_WORKSPACE = 4
STATUS_BAD_BLOCK = 1
STATUS_BAD_SEQ = 2
STATUS_BAD_POSITION = 4
PLAN_HEADER_WORDS = 24
COPY_D2H = 0
COPY_H2D = 1
COPY_ENGINE_DMA = 0
COPY_ENGINE_KERNEL = 1

# Plan header word indices (nsd_common.h, enum PlanHeader).
PLAN_MAGIC, PLAN_VERSION, PLAN_ROWS, PLAN_GROUPS, PLAN_PIECES, PLAN_WORKERS, PLAN_COMBINES, \
    PLAN_SLOTS, PLAN_ROWS_MAX, PLAN_HQ, PLAN_HKV, PLAN_OFF_GROUPS, PLAN_SIZED_FOR, \
    PLAN_OFF_PIECES, PLAN_OFF_COMBINES, PLAN_WORDS, PLAN_PIECE_BLOCKS, PLAN_BT_ROWS, \
    PLAN_BT_STRIDE, PLAN_MAX_BLOCKS, PLAN_STATIC, PLAN_CLAIMED = range(22)

_I32P = POINTER(c_int32)

# name -> (restype, argtypes)
SIGNATURES = {
    "nsd_version": (c_int, []),
    "nsd_last_error": (c_char_p, []),
    "nsd_rmsnorm_inplace": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_float, c_void_p]),
    "nsd_rotary_embedding_inplace": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_void_p]),
    "nsd_store_kvcache": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p,
                c_void_p, c_int64, c_int64, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
    "nsd_store_kvcache_prefill": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p,
                c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int, c_int, c_int, c_int, c_int,
                c_void_p, c_void_p]),
    "nsd_qk_norm_rope_store": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_void_p, c_void_p,
                c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p,
                c_int64, c_int64, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
    "nsd_qk_norm_rope_store_strided": (
        c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_float,
                c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p,
                c_int64, c_int64, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
    "nsd_attn_plan_bound": (c_int64, [c_int64, c_int, c_int]),
    "nsd_attn_plan_build": (
        c_int, [_I32P, _I32P, c_int64, c_int, c_int, c_int, c_int, c_int64, c_int64, c_int, c_int,
                _I32P, c_int64, POINTER(c_int64), POINTER(c_int64)]),
    "nsd_attn_plan_build_claimed": (
        c_int, [_I32P, _I32P, c_int64, c_int, c_int, c_int, c_int, c_int64, c_int64, c_int, c_int, c_int,
                _I32P, c_int64, POINTER(c_int64), POINTER(c_int64)]),
    "nsd_attn_num_workers": (c_int, [c_int, POINTER(c_int)]),
    "nsd_paged_attention": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_int,
                c_int, c_int, c_int, c_void_p, c_int64, c_int64, _I32P, c_void_p, c_void_p,
                c_int64, c_float, c_void_p, c_void_p]),
    "nsd_paged_attention_fused": (
        c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int,
                c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_int64, c_void_p, c_void_p,
                c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_int, c_int, c_int,
                c_void_p, c_int64, c_int64, _I32P, c_void_p, c_void_p, c_int64, c_float,
                c_void_p, c_void_p]),
    "nsd_paged_attention_noalloc": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_int,
                c_int, c_int, c_int, c_void_p, c_int64, c_int64, _I32P, c_void_p, c_float,
                c_void_p, c_void_p]),
    "nsd_write_block_ranges": (
        c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p,
                c_void_p]),
    "nsd_set_block_table": (
        c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64,
                c_void_p, c_void_p]),
    "nsd_unset_block_table": (
        c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                c_void_p]),
    "nsd_gather_allocated_blocks_and_unset": (
        c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                c_int64, c_void_p, c_void_p]),
    "nsd_copy_block_ranges": (
        c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p,
                c_void_p, c_int64, c_int, c_int, c_void_p]),
    "nsd_swap_blocks": (
        c_int, [c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_int64, c_void_p, c_void_p,
                c_int64, c_int64, c_int, c_void_p]),
    "nsd_fused_add_rmsnorm_inplace": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_float, c_void_p]),
    "nsd_silu_and_mul_inplace": (c_int, [c_void_p, c_int64, c_int64, c_void_p]),
    "nsd_up_gate_silu_and_mul": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p]),
    "nsd_linear_splits": (c_int, [c_int64, c_int64, c_int64, POINTER(c_int)]),
    "nsd_linear_partials": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p]),
    "nsd_sum_partials": (c_int, [c_void_p, c_int, c_void_p, c_int64, c_int64, c_void_p]),
    "nsd_fused_add_rmsnorm_partials": (
        c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_float, c_void_p]),
    "nsd_qk_norm_rope_store_partials": (
        c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_int64, c_void_p,
                c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_int, c_int, c_int,
                c_int, c_int, c_int, c_void_p, c_void_p]),
    "nsd_decoder_create": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_void_p, c_int,
                                   POINTER(c_void_p)]),
    "nsd_decoder_destroy": (c_int, [c_void_p]),
    "nsd_decoder_forward": (
        c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_int64,
                c_void_p, c_void_p, c_void_p, c_void_p, c_int64, _I32P, c_void_p, c_void_p, c_int64, c_float,
                c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "nsd_lm_head_argmax": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p]),
    "nsd_argmax_rows": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "nsd_probe_stream_read": (c_int, [c_void_p, c_int64, c_void_p, c_int, c_void_p]),
    "nsd_probe_tile_gather": (
        c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int, c_void_p, c_void_p]),
    "nsd_probe_stream_read_unroll": (c_int, [c_void_p, c_int64, c_void_p, c_int, c_int, c_void_p]),
    "nsd_probe_gather_pieces": (
        c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int, c_int, c_int, c_void_p,
                c_void_p]),
    "nsd_probe_gather_vgpr": (
        c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "nsd_probe_empty": (c_int, [c_int, c_void_p]),
    "nsd_probe_atomics": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]),
    "nsd_probe_gather_wave": (
        c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int, c_int, c_int, c_int, c_int,
                c_void_p, c_void_p]),
    "nsd_prefill_attention": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                c_int64, c_int, c_int, c_int, c_float, c_void_p, c_void_p]),
}


class NativeLibraryError(RuntimeError):
    """The gfx950 library is missing, failed to load, or returned an error."""


_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NativeLibraryError(
                    f"{LIB_PATH} is missing: build it with `python -m nebulasd_amd.build` "
                    "(there is no CPU fallback)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def last_error() -> str:
    msg = load().nsd_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != NSD_OK:
        raise NativeLibraryError(f"{what} failed (status {rc}): {last_error()}")


def call(name: str, *args) -> None:
    """Call entry point ``name`` and raise on a nonzero status."""
    check(getattr(load(), name)(*args), name)
