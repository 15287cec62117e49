"""LSE merge oracle (numpy). Test infrastructure only.

* ``merge_fp64``   -- the fp64 reference of ``ascend-kernel/csrc/ops/lse_merge/test/
                      lse_merge_cases.py:45-50``: m = max(l1, l2),
                      out = (o1 e^(l1-m) + o2 e^(l2-m)) / (e^(l1-m) + e^(l2-m)),
                      extended with the merged LSE m + ln(w1 + w2) and a defined result
                      when both sides are -inf (out = 0, lse = -inf; the reference
                      kernel has no guard and yields NaN there).
* ``merge_fp32``   -- the kernel's fp32 operation order
                      (``.../lse_merge/op_kernel/kernel_lse_merge.cpp:237-289``):
                      Max, Sub, Exp, Exp, Add, then per row sInv = 1/s and
                      out = (o1*w1 + o2*w2) * sInv, each step rounded to fp32.
* ``merge_many``   -- the N-way generalisation (split-KV partials):
                      lse = log sum_i e^(lse_i), O = sum_i e^(lse_i - lse) O_i.
"""
import numpy as np


def merge_fp64(o1, o2, l1, l2):
    """Returns (out fp64 [...,D], lse fp64 [...])."""
    o1 = np.asarray(o1, dtype=np.float64)
    o2 = np.asarray(o2, dtype=np.float64)
    l1 = np.asarray(l1, dtype=np.float64)
    l2 = np.asarray(l2, dtype=np.float64)
    m = np.maximum(l1, l2)
    empty = np.isneginf(m)
    ms = np.where(empty, 0.0, m)
    with np.errstate(invalid='ignore', divide='ignore'):
        w1 = np.exp(l1 - ms)
        w2 = np.exp(l2 - ms)
        s = w1 + w2
        out = (o1 * w1[..., None] + o2 * w2[..., None]) / s[..., None]
        lse = m + np.log(s)
    out = np.where(empty[..., None], 0.0, out)
    lse = np.where(empty, -np.inf, lse)
    return out, lse


def merge_fp32(o1, o2, l1, l2):
    """fp32 restatement of the kernel's operation order. Returns (out fp32, lse fp32)."""
    f = np.float32
    o1 = np.asarray(o1, dtype=f)
    o2 = np.asarray(o2, dtype=f)
    l1 = np.asarray(l1, dtype=f)
    l2 = np.asarray(l2, dtype=f)
    m = np.maximum(l1, l2)
    empty = np.isneginf(m)
    ms = np.where(empty, f(0), m).astype(f)
    with np.errstate(invalid='ignore', divide='ignore', over='ignore'):
        w1 = np.exp((l1 - ms).astype(f)).astype(f)
        w2 = np.exp((l2 - ms).astype(f)).astype(f)
        s = (w1 + w2).astype(f)
        sinv = (f(1) / s).astype(f)
        acc = ((o1 * w1[..., None]).astype(f) + (o2 * w2[..., None]).astype(f)).astype(f)
        out = (acc * sinv[..., None]).astype(f)
        lse = (m + np.log(s).astype(f)).astype(f)
    out = np.where(empty[..., None], f(0), out).astype(f)
    lse = np.where(empty, f(-np.inf), lse).astype(f)
    return out, lse


def merge_many(os_, lses):
    """N-way merge. os_ [N, ..., D], lses [N, ...] -> (out fp64, lse fp64)."""
    o = np.asarray(os_, dtype=np.float64)
    l = np.asarray(lses, dtype=np.float64)
    m = l.max(axis=0)
    empty = np.isneginf(m)
    ms = np.where(empty, 0.0, m)
    w = np.exp(l - ms[None])
    s = w.sum(axis=0)
    with np.errstate(invalid='ignore', divide='ignore'):
        out = (o * w[..., None]).sum(axis=0) / s[..., None]
        lse = m + np.log(s)
    return np.where(empty[..., None], 0.0, out), np.where(empty, -np.inf, lse)
