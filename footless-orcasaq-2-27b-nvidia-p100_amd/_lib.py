"""ctypes binding of libfl355.so (include/fl355.h).

The library is loaded once, from this package directory. There is no
fallback: if it is missing or does not load, importing the op layer raises,
so nothing can silently run another implementation.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libfl355.so"

FL_OK, FL_EINVAL, FL_ELAUNCH, FL_ESCRATCH = 0, 1, 2, 3
FL_MAX_SEQS = 16

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_LL = ctypes.c_longlong
_SZ = ctypes.c_size_t
_PP = ctypes.POINTER(ctypes.c_void_p)
_IP = ctypes.POINTER(ctypes.c_int)

# name -> (restype, argtypes); the order is the header's
SIGNATURES = {
    "fl_abi_version": (_I, []),
    "fl_strerror": (ctypes.c_char_p, [_I]),
    "fl_last_error": (ctypes.c_char_p, []),
    "fl_kv_store": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "fl_rmsnorm1p": (_I, [_P, _P, _P, _I, _I, _I, _I, _F, _P]),
    "fl_rope_partial": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _P]),
    "fl_attn_prep": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _F,
                          _P]),
    "fl_attention_split_gqa": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I,
                                    _I, _I, _P]),
    "fl_attention_merge": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _I, _I, _P]),
    "fl_attn_gate": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "fl_attn_decode_work_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "fl_attn_decode": (_I, [_P, _I, _PP, _PP, _IP, _IP, _I, _I, _I, _I, _I, _F, _I, _I, _P, _I,
                            _I, _P, _I, _P, _SZ, _P]),
    "fl_attention_prefill": (_I, [_P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _P, _I,
                                  _P]),
    "fl_attn_decode_noalloc": (_I, [_P, _I, _PP, _PP, _IP, _IP, _I, _I, _I, _I, _I, _F, _I, _I,
                                    _P, _I, _I, _P, _I, _P]),
    "fl_attn_decode_noalloc_max_bytes": (_SZ, []),
    "fl_attention_prefill_plan": (_I, [_I, _I, _I, _I, _I, _P, _I]),
    "fl_attention_prefill_split_count": (_I, [_I, _I, _I, _I]),
    "fl_attention_prefill_split_count_q8": (_I, [_I, _I, _I, _I]),
    "fl_attention_prefill_work_bytes": (_SZ, [_I, _I, _I, _I]),
    "fl_attention_prefill_q8_stage_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "fl_attention_prefill_kv": (_I, [_P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _I,
                                     _P, _I, _P, _SZ, _P]),
    "fl_attention_prefill_kv_q8": (_I, [_P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I,
                                        _I, _P, _I, _P, _SZ, _P]),
    "fl_attention_prefill_gated": (_I, [_P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F,
                                        _I, _I, _P, _I, _P, _SZ, _P]),
    "fl_kv_store_q8": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "fl_attn_prep_q8": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F,
                             _F, _P]),
    "fl_attn_prep_rows": (_I, [_P, _I, _P, _P, _P, _P, _PP, _PP, _IP, _IP, _I, _I, _I, _I, _I,
                               _I, _F, _F, _P]),
    "fl_attention_split_gqa_q8": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F,
                                       _I, _I, _I, _P]),
    "fl_attention_dec_q8": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _I, _P]),
    "fl_attention_dec_merge": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _I, _I, _P]),
    "fl_attn_decode_q8": (_I, [_P, _I, _PP, _PP, _IP, _IP, _I, _I, _I, _I, _I, _F, _I, _I, _P,
                               _I, _I, _P, _I, _P, _SZ, _P]),
    "fl_attention_prefill_q8": (_I, [_P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _P,
                                     _I, _P]),
    "fl_conv1d_causal": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "fl_conv1d_causal_rows": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "fl_l2norm_scaled": (_I, [_P, _P, _I, _I, _I, _F, _F, _I, _P]),
    "fl_l2norm_scaled_strided": (_I, [_P, _P, _I, _I, _LL, _F, _F, _I, _P]),
    "fl_rmsnorm_gated": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _F, _P]),
    "fl_gdn_scalars": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "fl_gdn_scan": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P,
                         _LL, _P]),
    "fl_gdn_decode": (_I, [_P, _I, _I, _P, _PP, _PP, _IP, _P, _P, _I, _P, _P, _PP, _P, _I, _PP,
                           _LL, _I, _I, _I, _I, _I, _I, _F, _F, _P]),
    "fl_gdn_decode_normed": (_I, [_P, _I, _I, _P, _PP, _PP, _IP, _P, _P, _I, _P, _P, _PP, _PP,
                                  _LL, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _F, _F,
                                  _P]),
    "fl_gdn_chunked_work_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "fl_gdn_prefill_chunked": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I,
                                    _F, _I, _I, _P, _SZ, _P]),
    "fl_gdn_prefill_chunked_logits": (_I, [_P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _I, _I, _I,
                                           _I, _I, _I, _I, _I, _F, _I, _I, _P, _SZ, _P]),
}


class FlError(RuntimeError):
    """A libfl355 entry point refused its arguments or a launch failed."""

    def __init__(self, fn: str, status: int, detail: str):
        super().__init__(f"{fn}: {detail or 'status %d' % status}")
        self.status = status


_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(hipcc, gfx950); there is no fallback implementation")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def call(name: str, *args) -> None:
    """Call an int-returning entry point; raise FlError on a non-zero status."""
    rc = getattr(lib(), name)(*args)
    if rc != FL_OK:
        detail = lib().fl_last_error().decode(errors="replace")
        if rc == FL_EINVAL:
            raise ValueError(f"{name}: {detail}")
        raise FlError(name, rc, detail)


def ptr_array(ptrs) -> ctypes.Array:
    arr = (ctypes.c_void_p * max(1, len(ptrs)))()
    for i, p in enumerate(ptrs):
        arr[i] = p
    return arr


def int_array(vals) -> ctypes.Array:
    arr = (ctypes.c_int * max(1, len(vals)))()
    for i, v in enumerate(vals):
        arr[i] = int(v)
    return arr
