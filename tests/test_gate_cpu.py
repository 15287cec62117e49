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


def _meta_case(B=4, H=32, KVH=8, P=1000):
    import cascade_amd  # noqa: F401  (registers the ops; Meta kernels need no GPU)
    m = "meta"
    bf = dict(dtype=torch.bfloat16, device=m)
    q = torch.empty(B, H, 128, **bf)
    kv = torch.empty(40, 128, KVH, 128, **bf)
    btp = torch.empty(1, 8, dtype=torch.int32, device=m)
    bts = torch.empty(B, 4, dtype=torch.int32, device=m)
    sl = torch.empty(B, dtype=torch.int64, device=m)
    return q, kv, btp, bts, sl


def test_unaligned_prefix_takes_cascade_without_measuring():
    g = G.CascadeGate(32, 8, timer=lambda *a: pytest.fail("an unaligned prefix must not be measured"))
    q, kv, btp, bts, sl = _meta_case()
    out, lse = g.decode(q, kv, kv, btp, 1000, bts, sl)
    assert out.shape == q.shape and lse.shape == (4 * 32,)
    assert not g.decisions


def test_capture_needs_decisions_and_prefix_tensors(monkeypatch):
    """Under capture an unmeasured bucket and an unseen prefix length are refused
    with a clear error; measured decisions and a cached (or passed) prefix tensor
    dispatch without a host round trip."""
    q, kv, btp, bts, sl = _meta_case()
    g = G.CascadeGate(32, 8, timer=lambda form, b, s: 1.0 if form == G.CASCADE else 2.0)
    monkeypatch.setattr(G, "_capturing", lambda: True)
    with pytest.raises(RuntimeError, match="no decision"):
        g.decode(q, kv, kv, btp, 1024, bts, sl)
    monkeypatch.setattr(G, "_capturing", lambda: False)
    g.choose(4, 1024)
    monkeypatch.setattr(G, "_capturing", lambda: True)
    with pytest.raises(RuntimeError, match="prefix length 1024"):
        g.decode(q, kv, kv, btp, 1024, bts, sl)
    out, _ = g.decode(q, kv, kv, btp, 1024, bts, sl, prefix_len_tensor=torch.empty(1, dtype=torch.int64,
                                                                                    device="meta"))
    assert out.shape == q.shape
    monkeypatch.setattr(G, "_capturing", lambda: False)
    g.decode(q, kv, kv, btp, 1024, bts, sl)              # eager call makes the tensor once
    monkeypatch.setattr(G, "_capturing", lambda: True)
    out, _ = g.decode(q, kv, kv, btp, 1024, bts, sl)     # now capture-safe
    assert out.shape == q.shape


def test_prefix_tensor_cache_is_bounded_and_keeps_captured_entries(monkeypatch):
    """The gate keeps at most PLEN_CACHE prefix-length tensors, evicting the least
    recently used, but never one a captured graph has read (the graph holds its
    address); a reused length is served from the cache."""
    g = G.CascadeGate(32, 8, timer=lambda *a: 1.0)
    monkeypatch.setattr(G, "_capturing", lambda: False)
    first = g._prefix_tensor(128, "meta")
    monkeypatch.setattr(G, "_capturing", lambda: True)
    assert g._prefix_tensor(128, "meta") is first          # read under capture: pinned
    monkeypatch.setattr(G, "_capturing", lambda: False)
    for n in range(1, G.PLEN_CACHE + 50):
        g._prefix_tensor(128 * (n + 1), "meta")
        g._prefix_tensor(128 * 2, "meta")                  # kept recent: never evicted
    assert len(g._plens) == G.PLEN_CACHE
    assert g._prefix_tensor(128, "meta") is first
    assert ("meta", 256) in g._plens
    assert ("meta", 384) not in g._plens                   # the oldest unpinned ones went
