"""ctypes binding of the C ABI (include/cascade_kernels.h) -- the reference-side
binding a Python caller would use instead of the torch ops.

Every function takes device pointers (ints, e.g. ``tensor.data_ptr()``), POD
sizes and a ``hipStream_t`` (int; ``torch.cuda.current_stream().cuda_stream``)
and returns the ABI's status code (0 = success). ``check`` turns a non-zero
code into a RuntimeError carrying ``ck_error_string``.
"""
import ctypes
import os
import re

from . import KERNEL_LIB

_HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))),
                       "include", "cascade_kernels.h")

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p
_f32 = ctypes.c_float
_p64 = ctypes.POINTER(ctypes.c_int64)
_f64 = ctypes.c_double

SIGNATURES = {
    "ck_error_string": (ctypes.c_char_p, [_int]),
    "ck_lse_merge": (_int, [_vp, _int, _vp, _int, _vp, _i64, _vp, _i64, _vp, _int, _vp, _i64, _i64, _vp]),
    "ck_fa_fp32_stage1_plan": (_int, [_i64, _i64, _i64, _i64, _i64, _i64, _p64, _p64]),
    "ck_fa_fp32_stage1": (_int, [_vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                                 _i64, _i64, _i64, _f32, _i64, _i64, _vp, _vp, _vp, _i64, _vp]),
    "ck_suffix_decode_plan": (_int, [_i64, _i64, _i64, _i64, _i64, _p64, _p64]),
    "ck_suffix_decode": (_int, [_vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32,
                                _i64, _i64, _vp, _vp, _vp, _i64, _vp]),
    "ck_f3_gateup_epilogue": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp]),
    "ck_cascade_decode_plan": (_int, [_i64, _i64, _i64, _i64, _i64, _i64, _p64]),
    "ck_cascade_decode": (_int, [_vp, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64,
                                 _i64, _i64, _i64, _i64, _f32, _i64, _i64, _vp, _vp, _vp, _i64, _vp]),
    "ck_cascade_decode_noalloc": (_int, [_vp, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _i64,
                                         _i64, _i64, _i64, _i64, _i64, _f32, _i64, _i64, _vp, _vp, _vp]),
    "ck_add_rms_norm_stats": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _int, _i64, _f64, _vp]),
    "ck_wait_giveups": (_int, [ctypes.POINTER(ctypes.c_uint64), _int]),
    "ck_bw_probe": (_int, [_vp, _vp, _i64, _int, _vp, _i64, _vp]),
    "ck_mfma_probe": (_int, [_i64, _vp, _i64, ctypes.POINTER(ctypes.c_double), _vp]),
}
PROBE_SINK_BYTES = 2 << 20

CK_DTYPE_BF16 = 0
CK_DTYPE_F32 = 1
CK_DTYPE_F16 = 2
CK_E_SCRATCH_LIMIT = -5
CASCADE_NOALLOC_SCRATCH_BYTES = 32 << 20
CK_KV_NHD = 0
CK_KV_BNSD = 1

_lib = None


def lib():
    """The loaded libcascade_hip.so with argtypes/restype set for every ABI symbol."""
    global _lib
    if _lib is None:
        if not os.path.exists(KERNEL_LIB):
            raise ImportError("cascade_amd: %s not built" % KERNEL_LIB)
        handle = ctypes.CDLL(KERNEL_LIB)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def header_symbols(path=_HEADER):
    """Function names declared in include/cascade_kernels.h."""
    text = open(path).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char \*)\s*(ck_\w+)\s*\(", text, flags=re.M)))


def error_string(code):
    return lib().ck_error_string(code).decode()


def check(code, what="ck"):
    if code != 0:
        raise RuntimeError("%s failed: %s (code %d)" % (what, error_string(code), code))


def stage1_plan(batch, max_q_len, num_heads, kv_heads, head_dim, kv_cap):
    s, w = ctypes.c_int64(0), ctypes.c_int64(0)
    check(lib().ck_fa_fp32_stage1_plan(batch, max_q_len, num_heads, kv_heads, head_dim, kv_cap,
                                       ctypes.byref(s), ctypes.byref(w)), "ck_fa_fp32_stage1_plan")
    return s.value, w.value


def suffix_plan(batch, num_heads, kv_heads, head_dim, kv_cap):
    s, w = ctypes.c_int64(0), ctypes.c_int64(0)
    check(lib().ck_suffix_decode_plan(batch, num_heads, kv_heads, head_dim, kv_cap, ctypes.byref(s),
                                      ctypes.byref(w)), "ck_suffix_decode_plan")
    return s.value, w.value


def wait_giveups(reset=False):
    """Bounded waits of the suffix / fused cascade kernels that ran out on the
    current device (0 unless an invariant broke); call after a synchronise."""
    n = ctypes.c_uint64(0)
    check(lib().ck_wait_giveups(ctypes.byref(n), 1 if reset else 0), "ck_wait_giveups")
    return n.value


def cascade_plan(batch, num_heads, kv_heads, head_dim, prefix_cap, suffix_cap):
    w = ctypes.c_int64(0)
    check(lib().ck_cascade_decode_plan(batch, num_heads, kv_heads, head_dim, prefix_cap, suffix_cap,
                                       ctypes.byref(w)), "ck_cascade_decode_plan")
    return w.value
