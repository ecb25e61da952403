"""ctypes binding of libhc.so, the C ABI declared in include/hc.h.

The library is loaded from this package directory.  There is no fallback:
if libhc.so is missing or fails to load, every op raises.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhc.so")

HC_OK = 0
HC_ERR_INVALID = -1
HC_ERR_CAPACITY = -2
HC_ERR_HIP = -3

HC_SCORE_CAUSAL_WINDOW = 1
HC_SCORE_SUM_WINDOW = 2
HC_SCORE_ROUND_BF16 = 4
HC_SCORE_ROUND_F16 = 8
HC_SCORE_ACCUMULATE = 16

HC_DTYPE_F32 = 0
HC_DTYPE_F16 = 1
HC_DTYPE_BF16 = 2

c_int, c_int32, c_int64, c_size_t, c_float, c_void_p, c_char_p = (
    ctypes.c_int, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float, ctypes.c_void_p,
    ctypes.c_char_p)

# name -> (restype, argtypes); the single Python mirror of include/hc.h.
SIGNATURES = {
    "hc_last_error": (c_char_p, []),
    "hc_version": (c_int, []),
    "hc_tile_tokens": (c_int, []),
    "hc_head_dim": (c_int, []),
    "hc_read_status": (c_int, [c_void_p, c_int, c_void_p, c_void_p]),
    "hc_stream_read": (c_int, [c_void_p, c_size_t, c_void_p, c_int, c_void_p]),
    "hc_decode_attn": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                               c_int, c_float, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_int64, c_int,
                               c_void_p, c_void_p]),
    "hc_decode_attn_stats": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                     c_int, c_int, c_float, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_int64,
                                     c_int, c_void_p, c_int, c_void_p, c_int64, c_int64, c_int, c_void_p]),
    "hc_decode_attn_noalloc": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_int, c_int, c_float, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_void_p,
                                       c_void_p]),
    "hc_decode_num_parts": (c_int64, [c_void_p, c_int, c_int]),
    "hc_decode_chunk_tiles": (c_int, [c_int, c_void_p, c_int, c_int]),
    "hc_decode_workspace_size": (c_size_t, [c_int, c_int, c_int64]),
    "hc_gather_store": (c_int, [c_int, c_void_p, c_void_p, c_int, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_void_p,
                                c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_int,
                                c_void_p, c_void_p]),
    "hc_gather_store_groups": (c_int, [c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p,
                                       c_void_p]),
    "hc_copy_rows": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_int, c_void_p,
                             c_int64, c_void_p, c_int, c_int, c_int, c_void_p]),
    "hc_prefill_attn": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                c_void_p, c_int, c_int, c_int, c_int, c_int, c_float, c_void_p, c_size_t,
                                c_void_p]),
    "hc_prefill_attn_stats": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_int, c_int, c_int, c_int, c_int, c_float, c_void_p, c_size_t,
                                      c_int, c_void_p, c_void_p]),
    "hc_prefill_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int]),
    "hc_prefill_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "hc_gather_rows": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_void_p, c_int64, c_void_p,
                               c_void_p, c_void_p, c_int64, c_void_p, c_int, c_int, c_void_p]),
    "hc_head_pool": (c_int, [c_int, c_void_p, c_int64, c_int64, c_int, c_int, c_int, c_int, c_int, c_void_p,
                             c_void_p]),
    "hc_append": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                          c_int, c_void_p, c_void_p]),
    "hc_score": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_void_p,
                         c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_void_p,
                         c_void_p, c_size_t, c_void_p, c_void_p]),
    "hc_score_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "hc_score_given_stats": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p,
                                     c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_void_p, c_void_p,
                                     c_void_p, c_void_p]),
    "hc_score_with_stats": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                                    c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_float,
                                    c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_size_t, c_void_p]),
    "hc_cake_score": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int, c_int,
                              c_int, c_int, c_int, c_int, c_float, c_float, c_void_p, c_void_p, c_void_p, c_size_t,
                              c_void_p]),
    "hc_cake_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "hc_select_topk": (c_int, [c_void_p, c_int64, c_int, c_int, c_void_p, c_int, c_void_p, c_int64, c_void_p,
                               c_void_p, c_size_t, c_void_p, c_size_t, c_int, c_void_p]),
    "hc_select_hist_size": (c_size_t, [c_int]),
    "hc_select_scratch_size": (c_size_t, [c_int, c_int]),
    "hc_set_bits": (c_int, [c_void_p, c_int64, c_void_p, c_int, c_int, c_void_p, c_int64, c_int, c_void_p, c_void_p,
                            c_void_p, c_void_p]),
    "hc_overlap_count": (c_int, [c_void_p, c_int64, c_int, c_int, c_void_p, c_int64, c_int, c_void_p, c_void_p,
                                 c_void_p]),
    "hc_drift_select": (c_int, [c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p, c_int, c_void_p, c_int64,
                                c_void_p, c_int, ctypes.c_double, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                c_void_p]),
    "hc_drift_scratch_size": (c_size_t, [c_int, c_int]),
    "hc_drift_decide": (c_int, [c_void_p, c_int, c_int, c_int, c_int, ctypes.c_double, c_void_p, c_void_p, c_void_p,
                                c_void_p]),
    "hc_store_read": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p,
                              c_void_p]),
}

_lib = None


class HCError(RuntimeError):
    """A libhc call returned a non-zero hc_status."""

    def __init__(self, code, msg):
        super().__init__(f"libhc error {code}: {msg}")
        self.code = code


def load():
    """Load libhc.so once and bind every declared symbol."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -m heterocache_amd.build` (or __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc):
    if rc != HC_OK:
        msg = load().hc_last_error()
        raise HCError(rc, msg.decode() if msg else "")
    return rc
