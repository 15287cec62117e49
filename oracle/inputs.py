"""Seeded input generators. Test infrastructure only.

``paged_inputs`` follows ``ascend-kernel/csrc/ops/fa_fp32_stage1/test/fa_fp32_ref.py:30-61``
(numpy ``default_rng(seed)`` standard normals for k, v, q in that order, per-request
distinct blocks by default, identical rows for ``share_blocks``) and adds a seeded
physical-block permutation (``permute=True``) so block_table indexing is exercised
beyond the identity / contiguous tables the reference uses.

``merge_inputs`` follows ``ascend-kernel/csrc/ops/lse_merge/test/lse_merge_cases.py:32-42``
(torch CPU generator seeded per case; o1, o2, l1, l2 drawn in that order).
"""
import numpy as np

from .bf16 import bf16_bits, bits_to_f32

BLOCK_SIZE = 128


def paged_inputs(batch, kv_seqlens, num_heads, kv_heads, head_dim=128, seed=0, q_len=1,
                 block_cols=None, share_blocks=False, permute=False, pad_value=0,
                 extra_blocks=0, dist="normal"):
    """Returns a dict with bf16 bit arrays (q16, k16, v16: uint16), their float32
    values (q, k, v), block_table int32 [B, cols], q_seqlens/kv_seqlens int64."""
    rng = np.random.default_rng(seed)
    kv_seqlens = [int(x) for x in kv_seqlens]
    assert len(kv_seqlens) == batch
    blocks_per_req = [(kv + BLOCK_SIZE - 1) // BLOCK_SIZE for kv in kv_seqlens]
    if block_cols is None:
        block_cols = max(max(blocks_per_req), 1)
    num_blocks = (max(blocks_per_req) if share_blocks else sum(blocks_per_req)) + extra_blocks
    num_blocks = max(num_blocks, 1)
    shape = (num_blocks, BLOCK_SIZE, kv_heads, head_dim)
    if dist == "normal":
        k = rng.standard_normal(shape).astype(np.float32)
        v = rng.standard_normal(shape).astype(np.float32)
        q = rng.standard_normal((batch * q_len, num_heads, head_dim)).astype(np.float32)
    else:
        k = rng.uniform(-1, 1, shape).astype(np.float32)
        v = rng.uniform(-1, 1, shape).astype(np.float32)
        q = rng.uniform(-1, 1, (batch * q_len, num_heads, head_dim)).astype(np.float32)
    phys = rng.permutation(num_blocks).astype(np.int32) if permute else \
        np.arange(num_blocks, dtype=np.int32)
    bt = np.full((batch, block_cols), pad_value, dtype=np.int32)
    nxt = 0
    for b, nb in enumerate(blocks_per_req):
        if share_blocks:
            bt[b, :nb] = phys[:nb]
        else:
            bt[b, :nb] = phys[nxt:nxt + nb]
            nxt += nb
    q16, k16, v16 = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    return dict(q16=q16, k16=k16, v16=v16, q=bits_to_f32(q16), k=bits_to_f32(k16),
                v=bits_to_f32(v16), block_table=bt,
                q_seqlens=np.full(batch, q_len, dtype=np.int64),
                kv_seqlens=np.asarray(kv_seqlens, dtype=np.int64),
                num_tokens=batch * q_len)


def merge_inputs(T, H, D, o1_f32, padded, seed):
    """lse_merge_cases.make_inputs restated. Returns torch CPU tensors
    (o1, o2, l1c, l2c, l1, l2): o1 fp32 or bf16, o2 bf16, compact l1/l2 and, when
    ``padded``, their 8-copy padded forms l1c/l2c."""
    import torch
    g = torch.Generator(device="cpu").manual_seed(seed)
    o1 = torch.randn(T, H, D, generator=g, dtype=torch.float32)
    o1 = o1 if o1_f32 else o1.to(torch.bfloat16)
    o2 = torch.randn(T, H, D, generator=g, dtype=torch.float32).to(torch.bfloat16)
    l1 = torch.randn(T, H, generator=g, dtype=torch.float32)
    l2 = torch.randn(T, H, generator=g, dtype=torch.float32)
    l1c, l2c = l1, l2
    if padded:
        l1c = l1.unsqueeze(-1).expand(T, H, 8).contiguous().reshape(T, H * 8)
        l2c = l2.unsqueeze(-1).expand(T, H, 8).contiguous().reshape(T, H * 8)
    return o1, o2, l1c, l2c, l1, l2
