"""Pins oracle.torch_cpu (the CPU baseline's torch restatement) against the numpy
oracle on small inputs, with planted mistakes it must not hide."""
import numpy as np
import torch

from oracle import attention as A
from oracle import gemm as G
from oracle import torch_cpu as TC
from oracle.inputs import paged_inputs
from oracle.merge import merge_fp64


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x))


def test_stage1_flattened_matches_numpy_oracle():
    inp = paged_inputs(1, [1300], 16, 4, seed=7, q_len=12, permute=True)
    O, L = TC.stage1(_t(inp["q"]), _t(inp["k"]), _t(inp["v"]), _t(inp["block_table"][0]), 1300)
    O_ref, L_ref = A.stage1(inp["q"], inp["k"], inp["v"], inp["block_table"], inp["q_seqlens"], inp["kv_seqlens"])
    # fp32 products against fp64: a handful of P elements round to the other bf16
    # neighbour; each moves O by at most 2^-8 p |v| / l
    assert np.abs(O.numpy() - O_ref).max() < 2e-4
    assert np.abs(L.numpy() - L_ref).max() < 1e-5
    # planted mistake: interleaved GQA head mapping
    q2 = inp["q"].reshape(12, 4, 4, 128).transpose(0, 2, 1, 3).reshape(12, 16, 128)
    Ow, _ = TC.stage1(_t(q2), _t(inp["k"]), _t(inp["v"]), _t(inp["block_table"][0]), 1300)
    assert np.abs(Ow.numpy() - O_ref).max() > 1e-2


def test_suffix_matches_numpy_oracle_with_empty_sequences():
    inp = paged_inputs(4, [0, 200, 513, 1], 8, 2, seed=3, permute=True)
    O, L = TC.suffix(_t(inp["q"]), _t(inp["k"]), _t(inp["v"]), _t(inp["block_table"]), inp["kv_seqlens"])
    O_ref, L_ref = A.stage1(inp["q"], inp["k"], inp["v"], inp["block_table"], np.ones(4, np.int64),
                            inp["kv_seqlens"], quantize_p=False)
    assert np.abs(O.numpy() - O_ref).max() < 1e-5
    fin = np.isfinite(L_ref)
    assert np.array_equal(np.isfinite(L.numpy()), fin)
    assert np.abs(L.numpy()[fin] - L_ref[fin]).max() < 1e-5


def test_merge_and_swiglu_match_numpy_oracle():
    rng = np.random.default_rng(1)
    o1, o2 = rng.standard_normal((2, 50, 128))
    l1, l2 = rng.standard_normal((2, 50)) * 2
    l2[::7] = -np.inf
    l1[3] = l2[3] = -np.inf
    out, lse = TC.merge(_t(o1).float(), _t(o2).float(), _t(l1).float(), _t(l2).float())
    ref, ref_l = merge_fp64(o1, o2, l1, l2)
    assert np.abs(out.numpy() - ref).max() < 1e-5
    assert np.all(out.numpy()[3] == 0) and np.isneginf(lse.numpy()[3])
    fin = np.isfinite(ref_l)
    assert np.abs(lse.numpy()[fin] - ref_l[fin]).max() < 1e-5
    a = rng.standard_normal((5, 256)).astype(np.float32)
    w = (rng.standard_normal((2 * 128, 256)) * 0.05).astype(np.float32)
    _, exact = G.swiglu(a, w)
    assert np.abs(TC.swiglu(_t(a), _t(w)).numpy() - exact).max() < 1e-4 * np.abs(exact).max()
