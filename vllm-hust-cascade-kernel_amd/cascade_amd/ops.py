"""Python-facing wrappers over ``torch.ops.npu.*`` (names follow the reference).

``cascade_decode`` is the caller-side composition the reference documents
(ascend-kernel/README.md:160-201) -- stage-1 over the shared prefix in the
flattened form (one request, q_len = batch), the per-sequence suffix attention
and the LSE merge -- as one fused op; ``cascade_decode_unfused`` composes the
three separate ops the same way the reference does.
"""
import torch


def fa_fp32_stage1(query, key, value, block_table, actual_q_seqlens, actual_kv_seqlens, q_seqlen_value=0):
    return torch.ops.npu.fa_fp32_stage1(query, key, value, block_table, actual_q_seqlens,
                                        actual_kv_seqlens, q_seqlen_value)


def lse_merge(o1, o2, lse1, lse2, out_code=0):
    return torch.ops.npu.lse_merge(o1, o2, lse1, lse2, out_code)


def lse_merge_with_lse(o1, o2, lse1, lse2, out_code=0):
    return torch.ops.npu.lse_merge_with_lse(o1, o2, lse1, lse2, out_code)


def suffix_decode(query, key, value, block_table, actual_kv_seqlens, kv_layout=0):
    """kv_layout 0: key/value [numBlocks, 128, KVH, D] (NHD); 1: [numBlocks, KVH, 128, D] (BNSD)."""
    return torch.ops.npu.suffix_decode(query, key, value, block_table, actual_kv_seqlens, kv_layout)


def f3_gateup_epilogue(a, b, workspace=None, out_d=None, mode=1):
    return torch.ops.npu.f3_gateup_epilogue(a, b, workspace, out_d, mode)


def add_rms_norm_stats(x1, x2, gamma=None, beta=None, eps=1e-6, mode=0):
    """Residual add + RMSNorm statistics (+ apply); see include/cascade_kernels.h."""
    return torch.ops.npu.add_rms_norm_stats(x1, x2, gamma, beta, eps, mode)


def swiglu_gate_up(a, b):
    """D = silu(a @ b[:I].T) * (a @ b[I:].T) in one fused GEMM (mode 1)."""
    return torch.ops.npu.f3_gateup_epilogue(a, b, None, None, 1)[0]


def cascade_decode(query, prefix_key, prefix_value, prefix_block_table, prefix_kv_seqlens,
                   suffix_key, suffix_value, suffix_block_table, suffix_kv_seqlens, suffix_kv_layout=0):
    """Shared-prefix cascade decode for a batch of B single-token queries, fused.

    query [B,H,D] bf16; prefix pages shared by all B sequences (prefix_block_table
    [1, cols], prefix_kv_seqlens int64 [1] on the device); each sequence's suffix
    through its own suffix_block_table row and suffix_kv_seqlens entry; the suffix
    pool may be NHD (suffix_kv_layout 0, the prefix pool's layout) or BNSD (1).
    Returns (out bf16 [B,H,D], merged LSE fp32 [B*H]).
    """
    return torch.ops.npu.cascade_decode(query, prefix_key, prefix_value, prefix_block_table, prefix_kv_seqlens,
                                        suffix_key, suffix_value, suffix_block_table, suffix_kv_seqlens,
                                        suffix_kv_layout)


def cascade_decode_unfused(query, prefix_key, prefix_value, prefix_block_table, prefix_kv_seqlens,
                           suffix_key, suffix_value, suffix_block_table, suffix_kv_seqlens, out_code=1):
    """The same cascade as the reference composes it (ascend-kernel/README.md:160-201):
    stage-1 flattened (one request, q_len = B), suffix attention, lse_merge."""
    B = query.shape[0]
    qlens = torch.full((1,), B, dtype=torch.int64, device=query.device)
    o1, l1 = torch.ops.npu.fa_fp32_stage1(query, prefix_key, prefix_value, prefix_block_table, qlens,
                                          prefix_kv_seqlens, B)
    o2, l2 = torch.ops.npu.suffix_decode(query, suffix_key, suffix_value, suffix_block_table, suffix_kv_seqlens)
    return torch.ops.npu.lse_merge(o1, o2, l1, l2, out_code)
