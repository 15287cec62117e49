"""CPU checks of the cascade-vs-full gate's host logic (cascade_amd/gate.py) with an
injected timer: bucketing, one measurement per bucket, the margin rule, JSON
persistence and the FULL-form block table."""
import json

import pytest
import torch

from cascade_amd import gate as G


def test_buckets():
    g = G.CascadeGate(32, 8, timer=lambda *a: 1.0)
    assert g.bucket(1, 1) == (1, 1024)
    assert g.bucket(50, 5000) == (64, 5120)
    assert g.bucket(64, 8192) == (64, 8192)
    assert g.bucket(65, 8193) == (128, 9216)


def test_one_measurement_per_bucket_and_choice():
    calls = []

    def timer(form, batch, shared):
        calls.append((form, batch, shared))
        # cascade wins for long shared prefixes, loses for short ones (README.md:245,258)
        if form == G.CASCADE:
            return 10.0 + 0.001 * shared
        return 5.0 + 0.004 * shared

    g = G.CascadeGate(32, 8, timer=timer)
    assert g.choose(64, 8192) == G.CASCADE
    assert g.choose(60, 8000) == G.CASCADE          # same bucket: no new measurement
    assert g.choose(64, 1024) == G.FULL
    assert len(calls) == 4
    g2 = G.CascadeGate(32, 8, timer=timer, margin=3.0)   # cascade must win by 3x
    assert g2.choose(64, 8192) == G.FULL


def test_json_round_trip():
    g = G.CascadeGate(32, 8, timer=lambda form, b, s: 1.0 if form == G.CASCADE else 2.0)
    g.choose(8, 2048)
    g.choose(256, 32768)
    text = g.to_json()
    h = G.CascadeGate(32, 8, timer=lambda *a: pytest.fail("must not re-measure"))
    h.load_json(text)
    assert h.choose(8, 2048) == G.CASCADE and h.choose(200, 32000) == G.CASCADE
    bad = json.loads(text)
    bad["shape"] = [64, 8, 128]
    with pytest.raises(ValueError):
        h.load_json(json.dumps(bad))


def test_full_block_table():
    pre = torch.tensor([[7, 3, 9, 100]], dtype=torch.int32)
    suf = torch.tensor([[1, 2], [5, 6], [8, 0]], dtype=torch.int32)
    bt = G.full_block_table(pre, 3, suf)
    assert bt.tolist() == [[7, 3, 9, 1, 2], [7, 3, 9, 5, 6], [7, 3, 9, 8, 0]]
    with pytest.raises(ValueError):
        G.full_decode(None, None, None, pre, 100, suf, None)
