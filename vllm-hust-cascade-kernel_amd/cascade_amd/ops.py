"""The cascade compositions over ``torch.ops.npu.*``; the single ops are called as
``torch.ops.npu.<name>`` directly, as in the reference.

``cascade_decode`` is the caller-side composition the reference documents
(ascend-kernel/README.md:160-201) -- stage-1 over the shared prefix in the
flattened form (one request, q_len = batch), the per-sequence suffix attention
and the LSE merge -- as one fused op; ``cascade_decode_unfused`` composes the
three separate ops the same way the reference does.
"""
import torch


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
