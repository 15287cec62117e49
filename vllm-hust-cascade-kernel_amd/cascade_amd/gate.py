"""Adaptive cascade-vs-full gate for shared-prefix decode.

The reference's caller decides per (batch, shared length) bucket whether the
two-stage cascade pays off, by micro-benchmarking both forms on the bucket's
shape and falling back to plain per-sequence decode where the cascade loses
(ascend-kernel/README.md:244-245 "自适应 gate ... 按 (B, shared) 桶实测决定走不走
cascade，亏区自动回落 FULL"; the losing region, e.g. 4k shared x B=64 x suffix 260,
README.md:258). This module is that harness for the MI355X ops:

* ``full_decode`` - the FULL form: one ``suffix_decode`` over each sequence's whole
  context, its block-table row being the shared prefix pages followed by its own
  suffix pages (the shared prefix must be page aligned, as vLLM's common-prefix
  blocks are).
* ``CascadeGate`` - buckets (batch rounded up to a power of two, shared length
  rounded up to a multiple of ``shared_quantum`` tokens), times both forms once per
  bucket on synthetic inputs of the bucket's shape and caches the faster form;
  ``decode`` dispatches a real call to the chosen form. Decisions can be saved to
  and loaded from JSON so a serving process does not re-measure.

The timing function is injectable (``timer=``) so the bucketing and caching logic
is testable without a GPU.

HIP-graph capture: measuring a bucket synchronises the device and creating the
device-side prefix length copies from the host, and neither may happen while a
stream is being captured. ``decode`` therefore raises during capture for a bucket
without a decision and for a prefix length it has no device tensor for: measure
(``choose``) or ``load_json`` the buckets, and make one eager call per prefix
length (or pass ``prefix_len_tensor``), before capturing.
"""
import collections
import json
import math

import torch

CASCADE = "cascade"
PLEN_CACHE = 256  # device tensors of prefix lengths kept by a gate (plus any a captured graph read)
FULL = "full"
PAGE = 128


def full_block_table(prefix_block_table, prefix_pages, suffix_block_table):
    """[B, prefix_pages + suffix_cols] int32: the shared prefix pages, then each
    sequence's own suffix pages."""
    B = suffix_block_table.shape[0]
    pre = prefix_block_table[:1, :prefix_pages].expand(B, prefix_pages)
    return torch.cat([pre, suffix_block_table], dim=1).contiguous()


def full_decode(query, key, value, prefix_block_table, prefix_len, suffix_block_table, suffix_kv_seqlens):
    """Per-sequence decode over prefix + suffix without the cascade split.

    ``prefix_len`` is a host int (the bucketing key; a multiple of 128).
    Returns (out bf16 [B,H,D], lse fp32 [B*H]) like ``cascade_decode``.
    """
    if prefix_len % PAGE:
        raise ValueError("full_decode: the shared prefix must be page aligned (%d tokens)" % prefix_len)
    bt = full_block_table(prefix_block_table, prefix_len // PAGE, suffix_block_table)
    kv = (suffix_kv_seqlens + prefix_len).contiguous()
    return torch.ops.npu.suffix_decode(query, key, value, bt, kv)


def _capturing():
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def _bucket(batch, shared_len, shared_quantum):
    b = 1 << max(0, math.ceil(math.log2(max(1, batch))))
    s = max(shared_quantum, -(-shared_len // shared_quantum) * shared_quantum)
    return b, s


def _cuda_timer(fn, reps=20, warmup=3):
    """Mean time (ms) of `reps` back-to-back calls, events only at the two ends."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


class CascadeGate:
    """Per-bucket choice between ``cascade_decode`` and ``full_decode``.

    num_heads / kv_heads / head_dim fix the attention shape; ``suffix_len`` is the
    representative per-sequence suffix length used when measuring a bucket (the
    decision is made per (batch, shared) bucket, as the reference's gate does).
    """

    def __init__(self, num_heads, kv_heads, head_dim=128, suffix_len=256, shared_quantum=1024,
                 device="cuda:0", timer=None, margin=1.0):
        self.shape = (num_heads, kv_heads, head_dim)
        self.suffix_len = suffix_len
        self.shared_quantum = shared_quantum
        self.device = device
        self.timer = timer
        self.margin = margin  # cascade must be faster than full by this factor to be chosen
        self.decisions = {}   # (batch bucket, shared bucket) -> {"choice", "cascade_ms", "full_ms"}
        # (device, prefix length) -> int64 [1] device tensor, made on first use; least
        # recently used first. At most PLEN_CACHE entries, except that an entry a
        # captured graph has read is never evicted (the graph holds its address).
        self._plens = collections.OrderedDict()
        self._plens_captured = set()

    # ---- buckets and decisions ---------------------------------------------------
    def bucket(self, batch, shared_len):
        return _bucket(batch, shared_len, self.shared_quantum)

    def choose(self, batch, shared_len):
        key = self.bucket(batch, shared_len)
        if key not in self.decisions:
            c_ms, f_ms = self.measure(*key)
            self.decisions[key] = {"choice": CASCADE if c_ms * self.margin < f_ms else FULL,
                                   "cascade_ms": c_ms, "full_ms": f_ms}
        return self.decisions[key]["choice"]

    def measure(self, batch, shared_len):
        """(cascade ms, full ms) on synthetic inputs of the bucket's shape."""
        if self.timer is not None:
            return self.timer(CASCADE, batch, shared_len), self.timer(FULL, batch, shared_len)
        H, KVH, D = self.shape
        npre = shared_len // PAGE
        nsuf = -(-self.suffix_len // PAGE)
        nblocks = npre + batch * nsuf
        g = torch.Generator(device=self.device).manual_seed(batch * 131 + shared_len)
        k = torch.randn(nblocks, PAGE, KVH, D, generator=g, device=self.device).to(torch.bfloat16)
        v = torch.randn(nblocks, PAGE, KVH, D, generator=g, device=self.device).to(torch.bfloat16)
        q = torch.randn(batch, H, D, generator=g, device=self.device).to(torch.bfloat16)
        perm = torch.randperm(nblocks, generator=torch.Generator().manual_seed(7)).to(torch.int32)
        btp = perm[:npre].view(1, npre).to(self.device)
        bts = perm[npre:].view(batch, nsuf).to(self.device)
        plen = torch.tensor([shared_len], dtype=torch.int64, device=self.device)
        sl = torch.full((batch,), self.suffix_len, dtype=torch.int64, device=self.device)
        c_ms = _cuda_timer(lambda: torch.ops.npu.cascade_decode(q, k, v, btp, plen, k, v, bts, sl))
        f_ms = _cuda_timer(lambda: full_decode(q, k, v, btp, shared_len, bts, sl))
        return c_ms, f_ms

    # ---- dispatch ---------------------------------------------------------------------
    def decode(self, query, key, value, prefix_block_table, prefix_len, suffix_block_table, suffix_kv_seqlens,
               prefix_len_tensor=None):
        """Shared-prefix decode through the bucket's chosen form.

        ``prefix_len`` is the host-side shared length (the bucketing key). The
        cascade's device-side prefix length is ``prefix_len_tensor`` when given,
        else a tensor this gate makes once per (device, length) and reuses. A
        prefix that is not page aligned always takes the cascade (the FULL form
        needs whole prefix pages), without measuring.
        """
        if prefix_len % PAGE:
            choice = CASCADE
        else:
            bk = self.bucket(query.shape[0], prefix_len)
            if bk not in self.decisions and _capturing():
                raise RuntimeError("CascadeGate.decode: bucket (batch %d, shared %d) has no decision and the "
                                   "stream is being captured; measure it with choose() or load_json() before "
                                   "capture" % bk)
            choice = self.choose(query.shape[0], prefix_len)
        if choice == CASCADE:
            plen = prefix_len_tensor if prefix_len_tensor is not None else \
                self._prefix_tensor(prefix_len, query.device)
            return torch.ops.npu.cascade_decode(query, key, value, prefix_block_table, plen, key, value,
                                                suffix_block_table, suffix_kv_seqlens)
        return full_decode(query, key, value, prefix_block_table, prefix_len, suffix_block_table,
                           suffix_kv_seqlens)

    def _prefix_tensor(self, prefix_len, device):
        k = (str(device), int(prefix_len))
        t = self._plens.get(k)
        if t is None:
            if _capturing():
                raise RuntimeError("CascadeGate.decode: no device tensor for prefix length %d yet and the stream "
                                   "is being captured; make one eager call with this length first, or pass "
                                   "prefix_len_tensor" % prefix_len)
            t = torch.tensor([int(prefix_len)], dtype=torch.int64, device=device)
            self._plens[k] = t
            self._evict_prefix_tensors()
        else:
            self._plens.move_to_end(k)
        if _capturing():
            self._plens_captured.add(k)
        return t

    def _evict_prefix_tensors(self):
        while len(self._plens) > PLEN_CACHE:
            old = next((key for key in self._plens if key not in self._plens_captured), None)
            if old is None:
                return
            del self._plens[old]

    # ---- persistence ------------------------------------------------------------------
    def to_json(self):
        return json.dumps({"shape": list(self.shape), "suffix_len": self.suffix_len,
                           "shared_quantum": self.shared_quantum,
                           "decisions": [{"batch": b, "shared": s, **d} for (b, s), d in
                                         sorted(self.decisions.items())]})

    def load_json(self, text):
        data = json.loads(text)
        if tuple(data["shape"]) != self.shape or data["shared_quantum"] != self.shared_quantum:
            raise ValueError("CascadeGate.load_json: decisions were measured for another shape/quantum")
        for d in data["decisions"]:
            self.decisions[(d["batch"], d["shared"])] = {k: d[k] for k in ("choice", "cascade_ms", "full_ms")}


def main(argv=None):
    """Measure a grid of buckets and print the decision table (markdown):
    python -m cascade_amd.gate --heads 32 --kv-heads 8 --suffix 256 --batches 8,64 --shared 1024,8192"""
    import argparse
    ap = argparse.ArgumentParser(description=main.__doc__)
    ap.add_argument("--heads", type=int, default=32)
    ap.add_argument("--kv-heads", type=int, default=8)
    ap.add_argument("--suffix", type=int, default=256)
    ap.add_argument("--batches", default="8,16,32,64,128,256")
    ap.add_argument("--shared", default="1024,2048,4096,8192,16384,32768")
    ap.add_argument("--json", default=None, help="also write the decisions here")
    args = ap.parse_args(argv)
    g = CascadeGate(args.heads, args.kv_heads, suffix_len=args.suffix)
    print("| batch | shared | cascade (us) | full (us) | choice |")
    print("|---:|---:|---:|---:|---|")
    for b in (int(x) for x in args.batches.split(",")):
        for s in (int(x) for x in args.shared.split(",")):
            g.choose(b, s)
            d = g.decisions[g.bucket(b, s)]
            print("| %d | %d | %.1f | %.1f | %s |" % (b, s, d["cascade_ms"] * 1e3, d["full_ms"] * 1e3, d["choice"]),
                  flush=True)
    if args.json:
        with open(args.json, "w") as f:
            f.write(g.to_json())


if __name__ == "__main__":
    import cascade_amd  # noqa: F401  (registers torch.ops.npu)
    main()
