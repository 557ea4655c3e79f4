"""ctypes binding of libhba_amd.so (declarations in include/hba_amd.h).

The library is the only compute path: if it is missing or the device is not a
gfx950 GPU, every op raises -- there is no CPU or PyTorch fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhba_amd.so")

F32, BF16 = 0, 1

_c_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_f = ctypes.c_float
_i = ctypes.c_int

# name -> argtypes (restype int unless noted); mirrors include/hba_amd.h
SIGNATURES = {
    "hba_abi_version": [],
    "hba_status_string": [_i],
    "hba_device_check": [],
    "hba_prep_keys": [_i, _vp, _c_i64p, _vp, _c_i64p, _vp, _f, _vp, _vp, _i64, _i64, _i64, _i64,
                      _vp, _vp, _vp, _vp],
    "hba_prep_keys_summarize": [_i, _vp, _c_i64p, _vp, _c_i64p, _vp, _f, _vp, _vp, _i64, _i64, _i64, _i64,
                                _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp],
    "hba_summarize": [_i, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp],
    "hba_build_super": [_i, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp],
    "hba_score_select": [_i, _vp, _c_i64p, _vp, _f, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                         _i64, _i64, _f, _vp, _vp, _vp, _vp, _vp],
    "hba_hier_select": [_i, _vp, _c_i64p, _vp, _f, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                        _i64, _i64, _i64, _i64, _i64, _f, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp],
    "hba_hier_select_workspace_bytes": [_i, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                        ctypes.POINTER(ctypes.c_size_t)],
    "hba_route_queries": [_i, _vp, _c_i64p, _vp, _f, _i64, _i64, _i64, _i64, _i64, _vp, _vp],
    "hba_hier_select_rows": [_i, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f,
                             _vp, _vp, _vp],
    "hba_attn_fwd": [_i, _vp, _c_i64p, _vp, _vp, _f, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                     _i64, _i64, _i64, _i64, _i64, _i64, _f, _vp, ctypes.c_size_t, _vp, _c_i64p, _vp],
    "hba_attn_workspace_size": [_i, _i64, _i64, _i64, ctypes.POINTER(ctypes.c_size_t)],
    "hba_attn_fwd_workspace_bytes": [_i, _i64, _i64, _i64, _i64, ctypes.POINTER(ctypes.c_size_t)],
    "hba_attn_window_fwd": [_vp, _c_i64p, _vp, _vp, _f, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                            _i64, _i64, _f, _vp, ctypes.c_size_t, _vp, _c_i64p, _vp],
    "hba_attn_routed_fwd": [_vp, _c_i64p, _vp, _vp, _f, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                            _i64, _i64, _f, _vp, ctypes.c_size_t, _vp, _c_i64p, _vp],
    "hba_attn_bwd": [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                     _i64, _i64, _i64, _i64, _i64, _i64, _f, _vp, ctypes.c_size_t, _vp, _vp, _vp, _vp, _vp, _vp],
    "hba_attn_bwd_workspace_size": [_i64, _i64, _i64, _i64, ctypes.POINTER(ctypes.c_size_t)],
    "hba_attn_bwd_workspace_bytes": [_i, _i64, _i64, _i64, _i64, _i64, ctypes.POINTER(ctypes.c_size_t)],
    "hba_kv_append": [_i, _vp, _vp, _vp, _f, _vp, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64,
                      _vp, _vp, _vp, _vp],
    "hba_summarize_pages": [_i, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp],
    "hba_kv_append_advance": [_i, _vp, _vp, _vp, _f, _vp, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64,
                              _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp],
    "hba_aux_kl_workspace_size": [_i, _i64, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.POINTER(ctypes.c_size_t)],
    "hba_aux_kl": [_i, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                   _f, _f, _vp, ctypes.c_size_t, _vp, _vp, _vp, _vp],
    "hba_summarize_filled": [_i, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp],
    "hba_decode_workspace_size": [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                  ctypes.POINTER(ctypes.c_size_t)],
    "hba_decode_fwd": [_i, _vp, _vp, _f, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i64,
                       _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, ctypes.c_size_t,
                       _vp, _vp, _vp, _vp],
    "hba_decode_fwd_noalloc": [_i, _vp, _vp, _f, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i64,
                               _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp],
}

_LIB = None


class HBAError(RuntimeError):
    """A nonzero status from the C-ABI."""


def lib():
    """Load the library once.  Raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                              "or `python -m hba_amd.build`; there is no fallback path")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_char_p if name == "hba_status_string" else ctypes.c_int
        _LIB = L
    return _LIB


def check(status, what):
    if status != 0:
        msg = lib().hba_status_string(status).decode()
        raise HBAError(f"{what}: {msg} (status {status})")


def strides3(t):
    """First three strides (elements) of a 4-D [B, n, H, d] view as a ctypes array."""
    return (ctypes.c_int64 * 3)(*[int(s) for s in t.stride()[:3]])
