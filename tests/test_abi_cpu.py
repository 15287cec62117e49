"""CPU checks of the C-ABI library: it loads without a GPU, exports every symbol
include/cascade_kernels.h declares, and rejects bad arguments before any launch."""
import ctypes

import pytest

from cascade_amd import abi


def test_library_exports_every_header_symbol():
    names = abi.header_symbols()
    assert names == sorted(abi.SIGNATURES), (names, sorted(abi.SIGNATURES))
    handle = ctypes.CDLL(abi.KERNEL_LIB)
    for n in names:
        assert hasattr(handle, n), n


def test_probe_argument_validation_without_launch():
    L = abi.lib()
    p = ctypes.c_void_p(256)  # never dereferenced: every call below fails validation first
    assert L.ck_bw_probe(p, None, 8, 0, p, abi.PROBE_SINK_BYTES, None) == -1           # bytes < 16
    assert L.ck_bw_probe(p, None, 24, 0, p, abi.PROBE_SINK_BYTES, None) == -1          # bytes % 16
    assert L.ck_bw_probe(p, None, 1024, 2, p, abi.PROBE_SINK_BYTES, None) == -1        # variant
    assert L.ck_bw_probe(p, None, 1024, 1, None, 0, None) == -2                        # copy needs dst
    assert L.ck_bw_probe(p, None, 1024, 0, p, abi.PROBE_SINK_BYTES - 4, None) == -3    # short sink
    f = ctypes.c_double(0)
    assert L.ck_mfma_probe(0, p, abi.PROBE_SINK_BYTES, ctypes.byref(f), None) == -1
    assert L.ck_mfma_probe(16, p, 1024, ctypes.byref(f), None) == -3


def test_error_strings():
    assert abi.error_string(0) == "success"
    for code in (-1, -2, -3, -4):
        assert abi.error_string(code) and abi.error_string(code) != "unknown error"


def test_merge_argument_validation_without_launch():
    L = abi.lib()
    p = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation first
    assert L.ck_lse_merge(p, 0, p, 0, p, 1, p, 1, p, 0, None, 4, 15, None) == -1   # dim % 16
    assert L.ck_lse_merge(p, 0, p, 0, p, 65, p, 1, p, 0, None, 4, 16, None) == -1  # stride > 64
    assert L.ck_lse_merge(p, 2, p, 0, p, 1, p, 1, p, 0, None, 4, 16, None) == -1   # dtype tag
    assert L.ck_lse_merge(None, 0, p, 0, p, 1, p, 1, p, 0, None, 4, 16, None) == -2
    assert L.ck_lse_merge(None, 0, None, 0, None, 1, None, 1, None, 0, None, 0, 16, None) == 0  # empty


def test_stage1_plan_and_validation():
    s, w = abi.stage1_plan(1, 64, 32, 8, 128, 8192)        # config 2, flattened
    assert s > 1 and w == s * 64 * 32 * 129 * 4
    s, w = abi.stage1_plan(64, 1, 32, 8, 128, 8192)        # per-request decode: no split
    assert s == 1 and w == 0
    s, w = abi.stage1_plan(1, 256, 64, 8, 128, 32768)      # config 5 prefix
    assert s >= 1
    out = ctypes.c_int64(0)
    L = abi.lib()
    assert L.ck_fa_fp32_stage1_plan(1, 1, 30, 8, 128, 100, ctypes.byref(out), ctypes.byref(out)) == -1  # H % KVH
    assert L.ck_fa_fp32_stage1_plan(1, 1, 32, 8, 64, 100, ctypes.byref(out), ctypes.byref(out)) == -4   # D != 128
    p = ctypes.c_void_p(16)
    # block size 64 unsupported; kv_cap beyond the table: both refused before launch
    assert L.ck_fa_fp32_stage1(p, p, p, p, 1, p, p, None, 1, 1, 1, 1, 8, 8, 128, 1, 64, 0.1, 128, 1, p, p,
                               None, 0, None) == -4
    assert L.ck_fa_fp32_stage1(p, p, p, p, 1, p, p, None, 1, 1, 1, 1, 8, 8, 128, 1, 128, 0.1, 256, 1, p, p,
                               None, 0, None) == -1
    # a split plan without a workspace
    assert L.ck_fa_fp32_stage1(p, p, p, p, 64, p, p, None, 1, 64, 64, 64, 32, 8, 128, 64, 128, 0.1, 8192, 0,
                               p, p, None, 0, None) == -3
    # the softmax scale must be finite and > 0 (the row max is taken before scaling)
    for bad in (0.0, -0.1, float("inf"), float("nan")):
        assert L.ck_fa_fp32_stage1(p, p, p, p, 1, p, p, None, 1, 1, 1, 1, 8, 8, 128, 1, 128, bad, 128, 1, p, p,
                                   None, 0, None) == -1, bad


def test_suffix_plan_and_validation():
    s, w = abi.suffix_plan(64, 32, 8, 128, 4096)
    assert s >= 1 and (w == 0) == (s == 1)
    # the grid holds 512 workgroups (two per CU on 256 CUs) over all kv head groups
    assert abi.suffix_plan(64, 32, 8, 128, 4096)[0] == 512 // 8
    assert abi.suffix_plan(64, 40, 8, 128, 4096)[0] == 512 // 8
    assert abi.suffix_plan(64, 64, 8, 128, 4096)[0] == 512 // 8
    assert abi.suffix_plan(64, 8, 1, 128, 4096)[0] == 512
    L = abi.lib()
    out = ctypes.c_int64(0)
    # 16 query heads per kv head: two kv head groups of 8 per kv head
    assert abi.suffix_plan(4, 64, 4, 128, 128)[0] == 512 // 8
    # 12 per kv head: two groups of 6; 11 (prime): eleven groups of 1
    assert abi.suffix_plan(4, 48, 4, 128, 128)[0] == 512 // 8
    assert abi.suffix_plan(4, 11, 1, 128, 128)[0] == 512 // 11
    p = ctypes.c_void_p(16)
    assert L.ck_suffix_decode(p, p, p, p, 1, p, 0, 8, 8, 128, 1, 128, 0, 0.1, 128, 1, p, p, None, 0, None) == 0
    assert L.ck_suffix_decode(p, p, p, p, 1, p, 4, 8, 8, 128, 1, 128, 2, 0.1, 128, 1, p, p, p, 1 << 20, None) == -1


def test_alignment_rejected_before_launch():
    """Operand pointers the kernels would read or write 16 bytes at a time must be
    16-byte aligned; a misaligned one is refused with CK_E_INVALID_ARG (nothing launched)."""
    L = abi.lib()
    p, odd = ctypes.c_void_p(16), ctypes.c_void_p(24)
    # stage-1: misaligned q, then misaligned (padded) lse
    assert L.ck_fa_fp32_stage1(odd, p, p, p, 1, p, p, None, 1, 1, 1, 1, 8, 8, 128, 1, 128, 0.1, 128, 1, p, p,
                               None, 0, None) == -1
    assert L.ck_fa_fp32_stage1(p, p, p, p, 1, p, p, None, 1, 1, 1, 1, 8, 8, 128, 1, 128, 0.1, 128, 1, p, odd,
                               None, 0, None) == -1
    # suffix decode: misaligned k; bf16 out 4- but not 8-aligned (the fix-up stores 8 bytes)
    assert L.ck_suffix_decode(p, odd, p, p, 1, p, 4, 8, 8, 128, 1, 128, 0, 0.1, 128, 1, p, p, p, 1 << 20,
                              None) == -1
    assert L.ck_suffix_decode(p, p, p, p, 1, p, 4, 8, 8, 128, 1, 128, 0, 0.1, 128, 1, ctypes.c_void_p(20), p, p,
                              1 << 20, None) == -1
    # lse_merge: misaligned o2
    assert L.ck_lse_merge(p, 0, odd, 0, p, 1, p, 1, p, 0, None, 4, 16, None) == -1
    # cascade: misaligned suffix v
    assert L.ck_cascade_decode(p, p, p, p, 1, p, 1, p, odd, p, 1, p, 1, 0, 4, 32, 8, 128, 128, 0.088, 128, 128,
                               p, p, p, 1 << 30, None) == -1


def test_gemm_validation():
    L = abi.lib()
    p = ctypes.c_void_p(16)
    assert L.ck_f3_gateup_epilogue(p, p, p, p, 16, 100, 128, 1, 100, None) == -1  # I % 128
    assert L.ck_f3_gateup_epilogue(p, p, p, p, 16, 128, 72, 1, 128, None) == -1   # K % 16
    assert L.ck_f3_gateup_epilogue(p, p, p, p, 16, 128, 128, 6, 128, None) == -1  # mode 6
    assert L.ck_f3_gateup_epilogue(p, p, None, p, 16, 128, 128, 0, 128, None) == -2  # mode 0 needs C
    assert L.ck_f3_gateup_epilogue(p, p, p, p, 0, 128, 128, 1, 128, None) == -1   # M = 0
    odd8, odd4 = ctypes.c_void_p(24), ctypes.c_void_p(20)  # 8- but not 16-aligned; 4-aligned
    assert L.ck_f3_gateup_epilogue(odd8, p, p, p, 16, 128, 128, 1, 128, None) == -1   # a alignment
    assert L.ck_f3_gateup_epilogue(p, odd8, p, p, 16, 128, 128, 1, 128, None) == -1   # b alignment
    assert L.ck_f3_gateup_epilogue(p, p, p, odd4, 16, 128, 128, 1, 128, None) == -1   # d alignment
    assert L.ck_f3_gateup_epilogue(p, p, odd4, p, 16, 128, 128, 0, 128, None) == -1   # C alignment
    assert L.ck_f3_gateup_epilogue(p, p, p, p, 16, 128, 128, 1, 130, None) == -1   # d_stride % 4


def test_cascade_plan_and_validation():
    w = abi.cascade_plan(64, 32, 8, 128, 8192, 4096)        # the benchmark's cascade shape
    s1, w1 = abi.stage1_plan(1, 64, 32, 8, 128, 8192)
    assert w >= w1 + 64 * 32 * (128 * 2 + 4)                 # stage-1 partials + suffix scratch
    assert abi.cascade_plan(0, 32, 8, 128, 8192, 4096) == 0
    L = abi.lib()
    out = ctypes.c_int64(0)
    assert L.ck_cascade_decode_plan(4, 64, 4, 128, 128, 128, ctypes.byref(out)) == 0    # 16 heads per kv head
    assert L.ck_cascade_decode_plan(4, 11, 1, 128, 128, 128, ctypes.byref(out)) == 0    # 11 heads per kv head
    assert L.ck_cascade_decode_plan(4, 32, 8, 64, 128, 128, ctypes.byref(out)) == -4    # D != 128
    assert L.ck_cascade_decode_plan(4, 30, 8, 128, 128, 128, ctypes.byref(out)) == -1   # H % KVH
    assert L.ck_cascade_decode_plan(4, 32, 8, 128, 128, 128, None) == -2
    # sequence indices are 32-bit: a batch of 2^31 sequences is refused by both plans
    assert L.ck_cascade_decode_plan(1 << 31, 32, 8, 128, 128, 128, ctypes.byref(out)) == -1
    assert L.ck_suffix_decode_plan(1 << 31, 32, 8, 128, 128, ctypes.byref(out), ctypes.byref(out)) == -1
    p = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation first

    def call(batch=4, block=128, pcols=1, pcap=128, scols=1, scap=128, ws=None, wsb=0, q=p, layout=0):
        return L.ck_cascade_decode(q, p, p, p, pcols, p, 1, p, p, p, scols, p, 1, layout, batch, 32, 8, 128, block,
                                   0.088, pcap, scap, p, p, ws, wsb, None)
    assert call(block=64) == -4                     # block size
    assert call(pcap=256) == -1                     # prefix bound beyond its table
    assert call(scap=256) == -1                     # suffix bound beyond its table
    assert call(q=None) == -2
    assert call(layout=2) == -1                     # unknown suffix pool layout
    need = abi.cascade_plan(4, 32, 8, 128, 128, 128)
    assert call(ws=p, wsb=need - 1) == -3           # short workspace, nothing launched
    assert call(batch=0) == 0                       # empty batch: nothing to do


def test_add_rms_norm_validation_without_launch():
    L = abi.lib()
    p = ctypes.c_void_p(16)
    bf16, f16, f32 = abi.CK_DTYPE_BF16, abi.CK_DTYPE_F16, abi.CK_DTYPE_F32
    assert L.ck_add_rms_norm_stats(p, p, p, None, p, p, p, 4, 40, bf16, 0, 1e-6, None) == -1    # K % 16
    assert L.ck_add_rms_norm_stats(p, p, p, None, p, p, p, 4, 5136, bf16, 0, 1e-6, None) == -1  # K > 5120
    assert L.ck_add_rms_norm_stats(p, p, p, None, p, p, p, 4, 64, f32, 0, 1e-6, None) == -1     # dtype
    assert L.ck_add_rms_norm_stats(p, p, p, None, p, p, p, 4, 64, f16, 3, 1e-6, None) == -1     # mode
    assert L.ck_add_rms_norm_stats(p, p, p, None, p, p, p, 4, 64, bf16, 0, 0.0, None) == -1     # eps
    assert L.ck_add_rms_norm_stats(p, None, p, None, p, p, p, 4, 64, bf16, 0, 1e-6, None) == -2  # x2 in mode 0
    assert L.ck_add_rms_norm_stats(p, p, None, None, p, p, p, 4, 64, bf16, 1, 1e-6, None) == -2  # gamma in mode 1
    assert L.ck_add_rms_norm_stats(None, None, None, None, None, None, None, 0, 64, bf16, 1, 1e-6, None) == 0
    odd = ctypes.c_void_p(24)
    assert L.ck_add_rms_norm_stats(odd, p, p, None, p, p, p, 4, 64, bf16, 0, 1e-6, None) == -1  # x1 alignment
    assert L.ck_add_rms_norm_stats(p, p, odd, None, p, p, p, 4, 64, bf16, 1, 1e-6, None) == -1  # gamma alignment
