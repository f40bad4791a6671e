"""ctypes binding of libvarlen_attn.so (the C ABI declared in include/varlen_attn.h).

The library is built in-tree by `hackaton_amd.build`; there is no fallback: a missing library
raises, so nothing can silently run another attention implementation.
"""

import ctypes
import os

# VA_LIB_PATH names another build of the same library (the host-sanitized one of
# hackaton_amd.build_hostsan, for the CPU tests); by default the in-tree build.
LIB_PATH = os.environ.get("VA_LIB_PATH") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "libvarlen_attn.so")

VA_OK, VA_EINVAL, VA_ESHAPE, VA_EDTYPE, VA_ESEQ, VA_ECAPACITY = 0, -1, -2, -3, -4, -5
VA_F16, VA_BF16, VA_F32 = 0, 1, 2
VA_PLAN_FWD, VA_PLAN_BWD, VA_PLAN_BWD_HEADS, VA_PLAN_BWD_PAIRS = 0, 1, 2, 3
VA_PLAN_BWD_GROUPS, VA_PLAN_BWD_GROUPS_ALL, VA_PLAN_FWD_NARROW = 4, 5, 6
VA_BWD_PAIR_MIN_ITEMS = 1024
VA_LAYOUT_PACKED, VA_LAYOUT_PADDED = 0, 1
VA_BWD_MAIN, VA_BWD_FINISH, VA_BWD_FINISH_HEADS, VA_BWD_STATS, VA_BWD_MAIN_STATS = 1, 2, 3, 4, 5
VA_BWD_STATS_MIN_TILES = 3
VA_FWD_MANY_ITEMS = 512
VA_FWD_AUTO, VA_FWD_WIDE, VA_FWD_MANY = 0, 1, 2

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_pi32 = ctypes.POINTER(ctypes.c_int32)
_pi64 = ctypes.POINTER(ctypes.c_int64)

class RopeTables(ctypes.Structure):
    """va_rope_tables: the rotary tables of va_bwd_rotary_stage's epilogues."""
    _fields_ = [("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p),
                ("cos_batch_stride", ctypes.c_int64), ("cos_seq_stride", ctypes.c_int64),
                ("b_idx", ctypes.c_void_p), ("t_idx", ctypes.c_void_p)]


# name -> (restype, argtypes); the same list the header declares.
SIGNATURES = {
    "va_last_error": (ctypes.c_char_p, []),
    "va_abi_version": (_i32, []),
    "va_head_dim": (_i32, []),
    "va_plan_size": (ctypes.c_int, [_pi32, _i32, _i32, _i32, _i32, _pi64]),
    "va_plan_build": (ctypes.c_int, [_pi32, _i32, _i32, _i32, _i32, _pi32, _i64, _pi64]),
    "va_plan_bwd_row_stats": (ctypes.c_int, [_pi32, _i32, _pi32]),
    "va_plan_capacity": (ctypes.c_int, [_i64, _i32, _i32, _i32, _pi64]),
    "va_plan_build_device": (ctypes.c_int, [_p, _i32, _i64, _i32, _i32, _i32, _p, _i64, _p]),
    "va_plan_build_device_lengths": (ctypes.c_int, [_p, _i32, _i64, _i32, _i32, _p, _i64, _p,
                                                    _i64, _p, _p]),
    "va_stream_capture_id": (ctypes.c_int, [_p, ctypes.POINTER(ctypes.c_uint64)]),
    "va_fwd": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32, _f32, _i32,
                              _p]),
    "va_fwd_kernel": (ctypes.c_int, [_i32, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32,
                                     _f32, _i32, _p]),
    "va_bwd_workspace_layout": (ctypes.c_int, [_i64, _i32, _i32, _i32, _pi64, _pi64]),
    "va_bwd": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32, _f32,
                              _i32, _p, _p, _p, _p, _i64, _p]),
    "va_bwd_noalloc_max_bytes": (_i64, []),
    "va_bwd_noalloc": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32,
                                      _f32, _i32, _p, _p, _p, _p]),
    "va_bwd_stage": (ctypes.c_int, [_i32, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32,
                                    _f32, _i32, _p, _p, _p, _p, _i64, _p]),
    "va_bwd_rotary_stage": (ctypes.c_int, [_i32, ctypes.POINTER(RopeTables), _p, _p, _p, _p, _p,
                                           _p, _p, _i64, _i64, _i32, _i32, _i32, _f32, _i32, _p,
                                           _p, _p, _p, _i64, _p]),
    "va_rope_fwd": (ctypes.c_int, [_p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _i64, _i32,
                                   _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p]),
    "va_rope_bwd": (ctypes.c_int, [_p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _i64, _i32,
                                   _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p]),
    "va_pack_rows": (ctypes.c_int, [_p, _p, _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _p]),
    "va_probe_mfma": (ctypes.c_int, [_i32, _i32, _i32, _p, _p]),
    "va_probe_copy": (ctypes.c_int, [_p, _p, _i64, _i32, _p]),
}

_LIB = None


class VarlenAttnError(RuntimeError):
    """A C-ABI call returned an error code (argument error < 0, HIP error > 0)."""

    def __init__(self, code, message):
        super().__init__(f"{message} (code {code})")
        self.code = code


def lib():
    """The loaded library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP kernels first "
                "(python -m hackaton_amd.build or __graft_entry__.build())")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def fwd_many_items(n_tokens, hq):
    """Whether va_fwd runs its many-item kernel for these sizes (ceil(N / 128) Hq >=
    VA_FWD_MANY_ITEMS)."""
    return -(-int(n_tokens) // 128) * int(hq) >= VA_FWD_MANY_ITEMS


def check(rc, what):
    """Raise VarlenAttnError with the library's message when rc != 0."""
    if rc != VA_OK:
        msg = lib().va_last_error()
        raise VarlenAttnError(rc, f"{what}: {msg.decode() if msg else 'error'}")
