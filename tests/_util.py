"""Shared test helpers (numpy <-> torch, tolerances)."""
import zlib

import numpy as np

BF16_EPS = 2.0 ** -8

# (case, max |O error|, O bound, max LSE relative error, LSE bound) of every parity
# case that records its margin; conftest prints the table after the run.
MARGINS = []


def record_margin(case, o_err, o_bound, l_rel=None, l_bound=None):
    MARGINS.append((case, float(o_err), float(o_bound), None if l_rel is None else float(l_rel),
                    None if l_bound is None else float(l_bound)))


def torch_bf16(bits, device):
    """uint16 bfloat16 bit patterns (numpy) -> torch.bfloat16 tensor on device."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)
    return t.to(device)


def bf16_to_np(t):
    """torch.bfloat16 tensor -> float32 numpy (exact)."""
    import torch
    return t.detach().to("cpu").view(torch.int16).numpy().view(np.uint16).astype(np.uint32) \
        .__lshift__(16).view(np.float32)


def case_seed(name):
    return zlib.crc32(name.encode()) % 2 ** 31


def merge_metrics(out, ref, mare_floor=0.0):
    """MERE / MARE / MaxAbsErr as defined by the reference's lse_merge tests
    (ascend-kernel/csrc/ops/lse_merge/test/test_lse_merge_precision.py:86-97)."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    diff = np.abs(out - ref)
    rel = diff / (np.abs(ref) + 1e-7)
    if mare_floor > 0:
        dom = np.abs(ref) >= mare_floor
        mare = float((rel * dom).max()) if dom.any() else 0.0
    else:
        mare = float(rel.max())
    return {"MERE": float(rel.mean()), "MARE": mare, "MaxAbsErr": float(diff.max())}


# (o1 fp32?, out_code, padded, MERE tol, MARE tol, MARE floor): lse_merge_cases.py:14-20
MERGE_MODES = {
    "A_tier0": (False, 0, False, 7.81e-3, 7.81e-2, 0.0),
    "B_fp32out": (True, 2, False, 1.22e-4, 1.22e-3, 1e-2),
    "Bp_fp32out_pad": (True, 2, True, 1.22e-4, 1.22e-3, 1e-2),
    "C_hybrid_bf16": (True, 1, False, 7.81e-3, 7.81e-2, 0.0),
    "D_tier0_pad": (False, 0, True, 7.81e-3, 7.81e-2, 0.0),
}
# lse_merge_cases.py:22-29
MERGE_SHAPES = [("production", (64, 40, 128)), ("0.5B", (56, 8, 128)), ("tiny", (7, 4, 16)),
                ("odd-rows", (13, 8, 128)), ("single-row", (1, 40, 128)), ("small-tile", (32, 32, 64))]


def merge_boundary(name, o1, o2, l1, l2):
    """The six boundary mutators of lse_merge_cases.py:53-70 (torch tensors, in place)."""
    if name == "equal_weights":
        l2.copy_(l1)
    elif name == "dlse_p40":
        l2.copy_(l1 - 40.0)
    elif name == "dlse_m40":
        l2.copy_(l1 + 40.0)
    elif name == "large_mag_30_35":
        l1.fill_(30.0)
        l2.fill_(35.0)
    elif name == "o2_zero":
        o2.zero_()
    elif name == "o1_zero":
        o1.zero_()
    else:
        raise KeyError(name)


MERGE_BOUNDARY = ["equal_weights", "dlse_p40", "dlse_m40", "large_mag_30_35", "o2_zero", "o1_zero"]
