"""MI355X (gfx950) cascade-decode operator set.

``import cascade_amd`` loads ``_lib/libcascade_torch.so``, which registers the
reference's custom ops under ``torch.ops.npu`` (the loader of
``ascend-kernel/python/ascend_kernel/ascend_kernel/__init__.py:9-15``):

* ``torch.ops.npu.fa_fp32_stage1(query, key, value, block_table, actual_q_seqlens,
  actual_kv_seqlens, q_seqlen_value=0) -> (out fp32 [T,H,D], lse fp32 [T*H*8])``
* ``torch.ops.npu.lse_merge(o1, o2, lse1, lse2, out_code=0) -> out``
* ``torch.ops.npu.f3_gateup_epilogue(a, b, workspace, out_d, mode) -> (d, workspace)``
* ``torch.ops.npu.add_rms_norm_stats(x1, x2, gamma, beta, eps, mode) -> (x_out, rstd, y)``
* additive: ``torch.ops.npu.suffix_decode(query, key, value, block_table,
  actual_kv_seqlens, kv_layout=0) -> (out bf16 [B,H,D], lse fp32 [B*H])``,
  ``torch.ops.npu.lse_merge_with_lse(o1, o2, lse1, lse2, out_code=0) -> (out, lse)`` and
  ``torch.ops.npu.cascade_decode(query, prefix_key, prefix_value, prefix_block_table,
  prefix_kv_seqlens, suffix_key, suffix_value, suffix_block_table, suffix_kv_seqlens,
  suffix_kv_layout=0) -> (out bf16 [B,H,D], merged lse fp32 [B*H])``.

``cascade_amd.gate`` holds the cascade-vs-full decision harness.

The libraries are built in-tree by ``build.py``. There is no CPU fallback: if the
libraries are missing, the import raises.
"""
import os

import torch

_LIBDIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib")
KERNEL_LIB = os.path.join(_LIBDIR, "libcascade_hip.so")
TORCH_LIB = os.path.join(_LIBDIR, "libcascade_torch.so")


def _load():
    missing = [p for p in (KERNEL_LIB, TORCH_LIB) if not os.path.exists(p)]
    if missing:
        raise ImportError(
            "cascade_amd: native libraries not built (missing: %s); run "
            "`python vllm-hust-cascade-kernel_amd/build.py`" % ", ".join(missing))
    torch.ops.load_library(TORCH_LIB)


_load()

from . import ops  # noqa: E402,F401  (Python-facing helpers over torch.ops.npu)

__all__ = ["ops", "KERNEL_LIB", "TORCH_LIB"]
