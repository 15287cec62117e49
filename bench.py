"""Benchmark of the cascade-decode operator set on one MI355X.

The step (timed exactly --steps times after --warmup untimed steps, which follow
--settle-ms of untimed steps that bring the clocks to their sustained state) is one fused
npu.cascade_decode call at BASELINE config 2's attention shapes, end to end:
  32 query heads, 8 kv heads, head dim 128, bf16; a shared 8192-token prefix (64
  pages of 128 tokens, permuted physical pages) read by stage-1 in the flattened
  form (one request, q_len = 64); 64 sequences whose own suffixes have geometric
  lengths (mean 512, clipped to [1, 4096]); the two partial results merged into
  bf16 O and the merged LSE.
value = algorithmic bytes of one step (q, prefix K/V read once, every suffix
K/V, block tables, seqlens, final bf16 O and merged LSE) x steps / the timed
region. Inputs are resident in HBM; the K/V pools rotate through enough copies
(>= 2 GiB distinct) that the 256 MB Infinity Cache cannot serve them.

Reported beside it (extra keys, each op launched back to back on the stream its
kernels run on, HIP events only at a loop's two ends):
  * each op of the reference's three-op composition, and the composition;
  * lse_merge of two fp32 partials [8192, 128] (5% of the
    suffix LSEs -inf) into bf16 + merged LSE over rotated inputs, reported by
    one HIP graph of the rotated calls replayed (GPU time per call), with the
    host-bound back-to-back loop beside it;
  * measured denominators beside the published peaks: the library's
    benchmark-only probes (a streaming HBM read and copy, back-to-back
    register-operand MFMAs), a 256 MiB torch copy and a bf16 8192^3
    torch.matmul;
  * the fused SwiGLU gate_up GEMM at M = 4096 (MFMA-bound) and
    at M = 1, 16, 256 (weight-stream bound);
  * the 70B-class cascade (H 64 / KVH 8, 32768-token prefix,
    256 sequences) followed by the SwiGLU GEMM M = 256, K = 8192, I = 28672;
  * add_rms_norm_stats, a HIP-graph batch of the cascade, and the CPU baseline
    (the torch CPU restatement of the same cascade on the host's cores).
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "vllm-hust-cascade-kernel_amd"))

HBM_PEAK_GBS = 8000.0        # MI355X published HBM3E bandwidth
BF16_PEAK_TFLOPS = 2500.0    # MI355X published dense bf16 MFMA peak

B, H, KVH, D, PREFIX, PAGE = 64, 32, 8, 128, 8192, 128
GEMM_M, GEMM_K, GEMM_I = 4096, 4096, 14336
C5 = dict(B=256, H=64, KVH=8, PREFIX=32768, GEMM_M=256, GEMM_K=8192, GEMM_I=28672)
MERGE_ROWS = 256 * 32        # [B=256, H=32] rows of D = 128
NORM_M, NORM_K = 2048, 5120  # add_rms_norm_stats at the reference's prefill-main shape
ROTATE_BYTES = 2 << 30
# the kernels each op launches (an op's HIP-event time covers all of them)
OP_KERNELS = {"cascade_decode": "cascade_fused_kernel + cascade_epilogue_kernel",
              "fa_fp32_stage1": "stage1_narrow_kernel + stage1_combine_kernel",
              "suffix_decode": "suffix_stream_kernel + suffix_fixup_kernel",
              "lse_merge": "lse_merge_kernel"}
CPU_THREADS_MAX = 16         # the GPU box's host-core share for one GPU


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--settle-ms", type=float, default=100.0,
                    help="untimed steps run back to back for this long before the warm-up steps, "
                         "so the GPU clocks reach their sustained state")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="only the step loop and the cascade's ops")
    return ap.parse_args()


def kernel_sources_sha256():
    """Hash of the HIP kernel sources (csrc/*.hip, *.h): ties a committed traffic profile to
    the code it was measured on."""
    import glob
    import hashlib
    h = hashlib.sha256()
    csrc = os.path.join(REPO, "vllm-hust-cascade-kernel_amd", "csrc")
    for f in sorted(glob.glob(os.path.join(csrc, "*.hip")) + glob.glob(os.path.join(csrc, "*.h"))):
        h.update(os.path.basename(f).encode())
        h.update(open(f, "rb").read())
    return h.hexdigest()


def geometric_suffixes(n, seed):
    import numpy as np
    rng = np.random.default_rng(seed)
    return np.clip(rng.geometric(1.0 / 512, size=n), 1, 4096).astype(np.int64)


def kv_tok_bytes(kvh):
    return kvh * D * 2 * 2  # K and V rows of one token, bf16


def build_cascade(torch, dev, b, h, kvh, prefix, suf, seed):
    """Pools rotated over >= ROTATE_BYTES of distinct copies, permuted pages."""
    import numpy as np
    nsb = [(int(s) + PAGE - 1) // PAGE for s in suf]
    npages = prefix // PAGE + sum(nsb)
    rng = np.random.default_rng(seed)
    perm = rng.permutation(npages).astype(np.int32)
    bt_pre = torch.from_numpy(perm[:prefix // PAGE][None, :].copy()).to(dev)
    bt_suf_np = np.zeros((b, max(nsb)), dtype=np.int32)
    off = prefix // PAGE
    for i in range(b):
        bt_suf_np[i, :nsb[i]] = perm[off:off + nsb[i]]
        off += nsb[i]
    bt_suf = torch.from_numpy(bt_suf_np).to(dev)
    pool_bytes = npages * PAGE * kv_tok_bytes(kvh)
    copies = max(2, -(-ROTATE_BYTES // pool_bytes))
    g = torch.Generator(device=dev).manual_seed(seed)
    pools = []
    for _ in range(copies):
        k = torch.randn(npages, PAGE, kvh, D, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
        v = torch.randn(npages, PAGE, kvh, D, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
        q = torch.randn(b, h, D, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
        pools.append((q, k, v))
    c = dict(pools=pools, bt_pre=bt_pre, bt_suf=bt_suf, copies=copies, suf_np=suf, B=b, H=h, KVH=kvh,
             PREFIX=prefix, qlens=torch.tensor([b], dtype=torch.int64, device=dev),
             kvlens=torch.tensor([prefix], dtype=torch.int64, device=dev), suf=torch.from_numpy(suf).to(dev))
    kt = kv_tok_bytes(kvh)
    c["bytes_end_to_end"] = (b * h * D * 2 + prefix * kt + int(suf.sum()) * kt
                             + (bt_pre.numel() + bt_suf.numel()) * 4 + (b + 1) * 8 + b * h * D * 2 + b * h * 4)
    c["bytes_stage1"] = (b * h * D * 2 + prefix * kt + bt_pre.numel() * 4 + 16
                         + b * h * D * 4 + b * h * 8 * 4)            # reads + fp32 O + padded LSE
    c["bytes_suffix"] = (b * h * D * 2 + int(suf.sum()) * kt + bt_suf.numel() * 4 + b * 8
                         + b * h * D * 2 + b * h * 4)                # reads + bf16 O + LSE
    c["bytes_merge"] = b * h * D * (4 + 2 + 2) + b * h * (8 + 1) * 4
    c["flops_stage1"] = 4 * b * h * D * prefix
    return c


def cpu_baseline(torch, w, gpu_out):
    """The torch CPU restatement of the cascade (oracle/torch_cpu.py: 512-column
    online softmax with bf16 P for stage-1, per-sequence suffix attention, LSE
    merge) on full steps of the benchmark workload -- the GPU step's own inputs
    (its first K/V pool copy, q, the permuted block tables, the suffix lengths),
    copied to the host -- with the host's allowed cores, at most the 16-core
    share of the box's CPUs that goes with one GPU. One warm-up step, then the
    median of at least 5 steps and at least 10 s of work (at most ~30 s). The
    warm-up step's output is compared with the GPU step's on the same inputs."""
    import numpy as np
    sys.path.insert(0, REPO)
    from oracle import torch_cpu as TC
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = os.cpu_count() or 1
    cores = max(1, min(allowed, CPU_THREADS_MAX))
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    q, k, v = (x.cpu() for x in w["pools"][0])
    bt_pre = w["bt_pre"][0].cpu()
    bt_suf = w["bt_suf"].cpu()
    suf = w["suf_np"]

    def step():
        O1, L1 = TC.stage1(q, k, v, bt_pre, PREFIX)
        O2, L2 = TC.suffix(q, k, v, bt_suf, suf)
        out, _ = TC.merge(O1, O2, L1, L2)
        return out.to(torch.bfloat16)

    first = step()  # warm-up
    diff = float((first.float() - gpu_out.float().cpu()).abs().max())
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < 12.0 and len(times) < 2000):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > 30.0:
            break
    torch.set_num_threads(prev)
    dt = float(np.median(times))
    kt = kv_tok_bytes(KVH)
    nbytes = B * H * D * 2 + PREFIX * kt + int(suf.sum()) * kt + B * H * D * 2 + B * H * 4
    return {"value": round(nbytes / dt / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "max_abs_diff_vs_gpu": diff,
            "sample": "full cascade steps of the benchmark workload on the GPU step's own inputs (first K/V "
                      "copy, q, permuted block tables, suffix lengths) through the torch CPU restatement "
                      "(oracle/torch_cpu.py, fp32, %d threads: the host cores allowed to this process, %d, "
                      "capped at the 16-core share of the box that goes with one GPU; os.cpu_count() = %d): "
                      "median of %d steps (%.3f s each, %.1f s total) after one warm-up; its bf16 output is "
                      "within %.2e of the GPU step's" % (cores, allowed, os.cpu_count() or 0, len(times), dt,
                                                          sum(times), diff)}


def measured_peaks(torch, timed, dev):
    """Achievable rates on this GPU beside the published peaks, from the library's
    benchmark-only probes (csrc/probe.hip): a 2 GiB streaming read and a 1 GiB
    copy (8 workgroups of 4 waves per CU), and back-to-back register-operand bf16
    MFMAs; beside them a plain 256 MiB torch copy (also the known-size dispatch
    that calibrates the FETCH_SIZE / WRITE_SIZE counters) and a bf16 torch.matmul
    (hipBLASLt, 8192^3)."""
    import ctypes
    from cascade_amd import abi
    L = abi.lib()
    st = torch.cuda.current_stream().cuda_stream
    sink = torch.empty(abi.PROBE_SINK_BYTES, dtype=torch.uint8, device=dev)
    buf = torch.ones(1 << 30, dtype=torch.int16, device=dev)  # 2 GiB
    dst = torch.empty(1 << 29, dtype=torch.int16, device=dev)  # 1 GiB

    def read(i):
        abi.check(L.ck_bw_probe(buf.data_ptr(), None, buf.numel() * 2, 0, sink.data_ptr(), sink.numel(), st))

    def copy(i):
        abi.check(L.ck_bw_probe(buf.data_ptr(), dst.data_ptr(), dst.numel() * 2, 1, None, 0, st))
    for _ in range(3):
        read(0)
        copy(0)
    read_gbs = buf.numel() * 2 / (timed(read, 10, warm=False) * 1e-3) / 1e9
    copy_gbs = 2 * dst.numel() * 2 / (timed(copy, 10, warm=False) * 1e-3) / 1e9
    del buf, dst
    src = torch.zeros(128 << 20, dtype=torch.int16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch_copy_gbs = 2 * src.numel() * 2 / (timed(lambda i: dst.copy_(src), 50, warm=False) * 1e-3) / 1e9
    del src, dst
    flops = ctypes.c_double(0)
    iters = 4096

    def mfma(i):
        abi.check(L.ck_mfma_probe(iters, sink.data_ptr(), sink.numel(), ctypes.byref(flops), st))
    for _ in range(10):  # ~20 ms: the clocks settle under the MFMA load first
        mfma(0)
    mfma_tflops = flops.value / (timed(mfma, 20, warm=False) * 1e-3) / 1e12
    n = 8192
    a = torch.randn(n, n, device=dev, dtype=torch.float32).to(torch.bfloat16)
    b = torch.randn(n, n, device=dev, dtype=torch.float32).to(torch.bfloat16)
    for _ in range(10):
        torch.matmul(a, b)
    mm_tflops = 2.0 * n ** 3 / (timed(lambda i: torch.matmul(a, b), 20, warm=False) * 1e-3) / 1e12
    del a, b
    return {"hbm_spec_gbs": HBM_PEAK_GBS, "hbm_read_gbs": round(read_gbs, 1), "hbm_copy_gbs": round(copy_gbs, 1),
            "torch_copy_gbs": round(torch_copy_gbs, 1),
            "bf16_spec_tflops": BF16_PEAK_TFLOPS, "bf16_mfma_probe_tflops": round(mfma_tflops, 1),
            "bf16_matmul_tflops": round(mm_tflops, 1),
            "method": "ck_bw_probe: 2 GiB streaming read / 1 GiB copy, 10 back to back; torch copy_ of 256 MiB, 50 "
                      "back to back; ck_mfma_probe: %d rounds of 16 independent 32x32x16 bf16 MFMAs per wave, 2 "
                      "waves per SIMD, 20 back to back after 10; bf16 torch.matmul 8192^3, 20 back to back" % iters}


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU; --gpus %d is not supported "
              "(the cascade-decode path would shard by kv head, with no exchange between GPUs)" % args.gpus,
              file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    import cascade_amd  # noqa: F401
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()

    def timed(fn, n, first=0, warm=True):
        """Mean GPU time (ms) of n back-to-back calls, HIP events on `stream` at
        the loop's two ends only. With `warm`, one untimed call first (a kernel's
        first launch in the process loads its code object)."""
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        if warm:
            fn(first + n)
        torch.cuda.synchronize()
        e0.record(stream)
        for i in range(n):
            fn(first + i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    # ---- the step: fused cascade decode at config 2 shapes ------------------------
    w = build_cascade(torch, dev, B, H, KVH, PREFIX, geometric_suffixes(B, 0), 1)

    def cascade(i, c=w):
        q, k, v = c["pools"][i % c["copies"]]
        return torch.ops.npu.cascade_decode(q, k, v, c["bt_pre"], c["kvlens"], k, v, c["bt_suf"], c["suf"])

    # Clock settle: from idle the GPU needs some tens of ms of sustained load before
    # its clocks stop ramping (20-step windows of this step measured 57-61 us from a
    # cold start and a steady 54 us after ~20 ms); then the --warmup steps and the
    # timed steps follow without a pause.
    settle_steps = 0
    t_settle = time.perf_counter()
    while (time.perf_counter() - t_settle) * 1e3 < args.settle_ms:
        for _ in range(50):
            cascade(settle_steps)
            settle_steps += 1
        torch.cuda.synchronize()
    settle_ms = (time.perf_counter() - t_settle) * 1e3
    for i in range(args.warmup):
        cascade(i)
    torch.cuda.synchronize()
    # timed region: synchronize on both sides (one rank: no barrier to take)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms_step = timed(cascade, args.steps, args.warmup, warm=False)
    wall = time.perf_counter() - t0
    value = w["bytes_end_to_end"] / (ms_step * 1e-3) / 1e9

    # measured denominators, outside every timed region; the 256 MiB copy is also the
    # known-size dispatch (__amd_rocclr_copyBuffer) that calibrates the FETCH_SIZE /
    # WRITE_SIZE counters
    peaks = measured_peaks(torch, timed, dev)

    # ---- the cascade's ops: the reference's three-op composition -----------------------
    def stage1(i, c=w):
        q, k, v = c["pools"][i % c["copies"]]
        return torch.ops.npu.fa_fp32_stage1(q, k, v, c["bt_pre"], c["qlens"], c["kvlens"], c["B"])

    def suffix(i, c=w):
        q, k, v = c["pools"][i % c["copies"]]
        return torch.ops.npu.suffix_decode(q, k, v, c["bt_suf"], c["suf"])

    parts = [(stage1(i), suffix(i)) for i in range(w["copies"])]

    def merge(i):
        (o1, l1), (o2, l2) = parts[i % len(parts)]
        return torch.ops.npu.lse_merge(o1, o2, l1, l2, 1)

    def cascade_unfused(i):
        o1, l1 = stage1(i)
        o2, l2 = suffix(i)
        return torch.ops.npu.lse_merge(o1, o2, l1, l2, 1)

    n = max(args.steps, 100)
    ms = {"cascade_unfused": timed(cascade_unfused, n), "stage1": timed(stage1, n), "suffix": timed(suffix, n),
          "merge": timed(merge, n)}
    del parts
    per_op = {"fa_fp32_stage1": (ms["stage1"], w["bytes_stage1"]),
              "suffix_decode": (ms["suffix"], w["bytes_suffix"]),
              "lse_merge": (ms["merge"], w["bytes_merge"])}
    dom = max(per_op, key=lambda k: per_op[k][0])
    dom_gbs = per_op[dom][1] / (per_op[dom][0] * 1e-3) / 1e9
    # HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    # (calibrated against a plain copy of known size); used only while the kernel
    # sources are the ones that profile was taken from
    traffic = {}
    traffic_note = "no profile"
    tpath = os.path.join(REPO, "profiles", "pmc_traffic.json")
    if os.path.exists(tpath):
        prof = json.load(open(tpath))
        if prof.get("sources_sha256") == kernel_sources_sha256():
            traffic = prof
            traffic_note = "rocprofv3 FETCH_SIZE/WRITE_SIZE of these kernel sources (profiles/pmc_traffic.md)"
        else:
            traffic_note = "profile predates the current kernel sources: traffic not reported"

    line = {
        "metric": "cascade-decode attn HBM GB/s (% of peak) + SwiGLU GEMM TFLOP/s at 1 MI355X",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"steps": settle_steps, "ms": round(settle_ms, 1)},
        "ms_per_step": round(ms_step, 5),
        "wall_ms_per_step": round(wall * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) bf16 q/k/v, N(0,0.02) weights, seeded)",
        "config": {
            "workload": "BASELINE config 2 end to end: cascade decode H32/KVH8/D128, shared prefix 8192 "
                        "(flattened stage-1, q_len 64), 64 suffixes ~Geometric(mean 512) clipped [1,4096] "
                        "(%d tokens), page 128, permuted pages, merge to bf16 + merged LSE; one fused "
                        "cascade_decode call per step" % int(w["suf_np"].sum()),
            "kv_rotation_copies": w["copies"],
            "bytes_per_step": w["bytes_end_to_end"],
        },
        "cascade_pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "cascade_us": round(ms_step * 1e3, 2),
        "cascade_unfused_us": round(ms["cascade_unfused"] * 1e3, 2),
        "per_op_us": {k: round(v[0] * 1e3, 2) for k, v in per_op.items()},
        # the step's own launches: the fused kernel (stage-1 units and suffix streams
        # side by side, most of the step's time) and its epilogue, timed together
        "roofline": {"kernel": "cascade_decode op (" + OP_KERNELS["cascade_decode"] + ")", "bound": "hbm",
                     "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic.get("cascade_decode"),
                     "traffic_source": traffic_note, "peak_measured": peaks["hbm_read_gbs"],
                     "peak_measured_kind": "ck_bw_probe streaming read (the step is read-dominated)",
                     "frac_of_measured": round(value / peaks["hbm_read_gbs"], 4)},
        "peaks": peaks,
        # the slowest op of the reference's three-op composition, for comparison
        "roofline_ops": {"kernel": dom + " op (" + OP_KERNELS[dom] + ")", "bound": "hbm",
                         "achieved": round(dom_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": traffic.get(dom)},
    }
    if args.no_extras:
        print(json.dumps(line), flush=True)
        return

    # ---- the merge alone, fp32 partials into bf16 + merged LSE ------
    merge_bytes = MERGE_ROWS * D * (4 + 4 + 2) + MERGE_ROWS * 4 * 3
    m_copies = -(-ROTATE_BYTES // merge_bytes)
    gm = torch.Generator(device=dev).manual_seed(3)
    m_in = []
    for _ in range(m_copies):
        o1 = torch.randn(MERGE_ROWS, D, generator=gm, device=dev)
        o2 = torch.randn(MERGE_ROWS, D, generator=gm, device=dev)
        l1 = torch.randn(MERGE_ROWS, generator=gm, device=dev) * 2.0
        l2 = torch.randn(MERGE_ROWS, generator=gm, device=dev) * 2.0
        l2[torch.rand(MERGE_ROWS, generator=gm, device=dev) < 0.05] = -float("inf")
        m_in.append((o1, o2, l1, l2))

    def merge3(i):
        return torch.ops.npu.lse_merge_with_lse(*m_in[i % m_copies], 1)

    def merge3_hot(i):
        return torch.ops.npu.lse_merge_with_lse(*m_in[0], 1)
    t_m3, t_m3_hot = timed(merge3, n), timed(merge3_hot, n)
    # The kernel is shorter than the host's per-call op dispatch, so the loop above
    # measures the host as much as the GPU. The same rotated calls replayed from
    # one HIP graph give the GPU time per call.
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        merge3(0)
    stream.wait_stream(side)
    torch.cuda.synchronize()
    g3 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g3):
        for i in range(m_copies):
            merge3(i)
    g3.replay()
    torch.cuda.synchronize()
    reps3 = max(1, n // 20)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps3):
        g3.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    t_m3_graph = e0.elapsed_time(e1) / (reps3 * m_copies)
    del g3, m_in
    # reported by the graph replay (GPU time per call); the host loop is kept beside
    # it, labelled: it measures the host's per-call op dispatch as much as the kernel
    line["config3_merge"] = {
        "rows": MERGE_ROWS, "bytes": merge_bytes, "rotation_copies": m_copies,
        "timing": "HIP graph of %d rotated calls, replayed; GPU time per call" % m_copies,
        "us": round(t_m3_graph * 1e3, 2), "gbs": round(merge_bytes / (t_m3_graph * 1e-3) / 1e9, 1),
        "frac_of_hbm_peak": round(merge_bytes / (t_m3_graph * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "host_loop_us": round(t_m3 * 1e3, 2),
        "host_loop_note": "back-to-back op calls from the host: bound by the host's op dispatch, not the kernel",
        "cache_hot_host_loop_us": round(t_m3_hot * 1e3, 2)}

    # ---- the fused SwiGLU GEMM ------------------------------------------
    a = torch.randn(GEMM_M, GEMM_K, device=dev, dtype=torch.float32).to(torch.bfloat16)
    wt = (torch.randn(2 * GEMM_I, GEMM_K, device=dev, dtype=torch.float32) * 0.02).to(torch.bfloat16)
    d_out = torch.empty(GEMM_M, GEMM_I, device=dev, dtype=torch.bfloat16)

    def gemm(i):
        torch.ops.npu.f3_gateup_epilogue(a, wt, None, d_out, 1)
    for _ in range(40):  # let the clocks settle under a sustained MFMA load (~30 ms) before timing
        gemm(0)
    t_gemm = timed(gemm, max(20, n // 5))
    gemm_tflops = 2.0 * GEMM_M * GEMM_K * 2 * GEMM_I / (t_gemm * 1e-3) / 1e12
    line["swiglu_gemm"] = {"M": GEMM_M, "K": GEMM_K, "I": GEMM_I, "tflops": round(gemm_tflops, 1),
                           "us": round(t_gemm * 1e3, 1), "pct_of_bf16_peak": round(100.0 * gemm_tflops /
                                                                                    BF16_PEAK_TFLOPS, 2)}
    line["roofline_gemm"] = {"kernel": "f3_gateup_epilogue mode 1", "bound": "mfma", "achieved": round(gemm_tflops, 1),
                             "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(gemm_tflops / BF16_PEAK_TFLOPS, 4),
                             "traffic": traffic.get("f3_gateup_epilogue"),
                             "peak_measured": peaks["bf16_mfma_probe_tflops"],
                             "peak_measured_kind": "ck_mfma_probe: register-operand MFMAs, no memory traffic",
                             "frac_of_measured": round(gemm_tflops / peaks["bf16_mfma_probe_tflops"], 4),
                             "vs_library_matmul": round(gemm_tflops / peaks["bf16_matmul_tflops"], 4)}
    # decode-sized M over two weight copies (470 MB together, beyond the Infinity Cache)
    wt_pair = [wt, (torch.randn(2 * GEMM_I, GEMM_K, device=dev, dtype=torch.float32) * 0.02).to(torch.bfloat16)]
    small_m = {}
    for mm in (1, 16, 256):
        a_m = torch.randn(mm, GEMM_K, device=dev, dtype=torch.float32).to(torch.bfloat16)
        d_m = torch.empty(mm, GEMM_I, device=dev, dtype=torch.bfloat16)

        def gemm_m(i, a_m=a_m, d_m=d_m):
            torch.ops.npu.f3_gateup_epilogue(a_m, wt_pair[i % 2], None, d_m, 1)
        t = timed(gemm_m, n)
        wbytes = 2 * GEMM_I * GEMM_K * 2
        small_m[str(mm)] = {"us": round(t * 1e3, 1), "weight_gbs": round(wbytes / (t * 1e-3) / 1e9, 1),
                            "frac_of_hbm_peak": round((wbytes + mm * (GEMM_K + GEMM_I) * 2) / (t * 1e-3) / 1e9
                                                      / HBM_PEAK_GBS, 4)}
    line["swiglu_gemm_small_m"] = small_m
    del wt_pair, a, wt, d_out

    # ---- 70B-class cascade + SwiGLU GEMM -------------------------
    c5 = build_cascade(torch, dev, C5["B"], C5["H"], C5["KVH"], C5["PREFIX"], geometric_suffixes(C5["B"], 5), 5)
    a5 = torch.randn(C5["GEMM_M"], C5["GEMM_K"], device=dev, dtype=torch.float32).to(torch.bfloat16)
    w5 = (torch.randn(2 * C5["GEMM_I"], C5["GEMM_K"], device=dev, dtype=torch.float32) * 0.02).to(torch.bfloat16)
    d5 = torch.empty(C5["GEMM_M"], C5["GEMM_I"], device=dev, dtype=torch.bfloat16)

    def c5_cascade(i):
        return cascade(i, c5)

    def c5_gemm(i):
        torch.ops.npu.f3_gateup_epilogue(a5, w5, None, d5, 1)

    def c5_step(i):
        c5_cascade(i)
        c5_gemm(i)
    t5 = {"cascade": timed(c5_cascade, 30), "gemm": timed(c5_gemm, 30), "step": timed(c5_step, 30)}
    g5_flops = 2.0 * C5["GEMM_M"] * C5["GEMM_K"] * 2 * C5["GEMM_I"]
    g5_bytes = 2 * C5["GEMM_I"] * C5["GEMM_K"] * 2 + C5["GEMM_M"] * (C5["GEMM_K"] + C5["GEMM_I"]) * 2
    line["config5"] = {
        "workload": "H64/KVH8/D128, shared prefix 32768, 256 suffixes ~Geometric(mean 512) clipped [1,4096] "
                    "(%d tokens); then SwiGLU GEMM M=256 K=8192 I=28672" % int(c5["suf_np"].sum()),
        "kv_rotation_copies": c5["copies"],
        "cascade_us": round(t5["cascade"] * 1e3, 1),
        "cascade_gbs": round(c5["bytes_end_to_end"] / (t5["cascade"] * 1e-3) / 1e9, 1),
        "cascade_bytes": c5["bytes_end_to_end"],
        "stage1_flops": c5["flops_stage1"],
        "gemm_us": round(t5["gemm"] * 1e3, 1),
        "gemm_tflops": round(g5_flops / (t5["gemm"] * 1e-3) / 1e12, 1),
        "gemm_frac_of_hbm_peak": round(g5_bytes / (t5["gemm"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "step_us": round(t5["step"] * 1e3, 1),
    }
    del c5, a5, w5, d5

    # ---- add_rms_norm_stats (adjacent op), rotated over 8 input pairs ----------------
    norm_copies = 8
    norm_in = [(torch.randn(NORM_M, NORM_K, device=dev) * 0.5).to(torch.bfloat16) for _ in range(2 * norm_copies)]
    norm_gamma = (1.0 + torch.randn(NORM_K, device=dev) * 0.1).to(torch.bfloat16)

    def norm0(i):
        j = 2 * (i % norm_copies)
        return torch.ops.npu.add_rms_norm_stats(norm_in[j], norm_in[j + 1], None, None, 1e-6, 0)

    def norm1(i):
        j = 2 * (i % norm_copies)
        return torch.ops.npu.add_rms_norm_stats(norm_in[j], norm_in[j], norm_gamma, None, 1e-6, 1)
    t_n0, t_n1 = timed(norm0, n), timed(norm1, n)
    line["add_rms_norm_stats"] = {
        "shape": [NORM_M, NORM_K], "dtype": "bf16",
        "mode0_us": round(t_n0 * 1e3, 2),
        "mode0_gbs": round((3 * NORM_M * NORM_K * 2 + NORM_M * 4) / (t_n0 * 1e-3) / 1e9, 1),
        "mode1_us": round(t_n1 * 1e3, 2),
        "mode1_gbs": round((2 * NORM_M * NORM_K * 2 + NORM_K * 2 + NORM_M * 4) / (t_n1 * 1e-3) / 1e9, 1)}
    del norm_in

    # ---- HIP-graph batch: one graph holding one cascade call per pool copy -----------
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        cascade(0)
    stream.wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(w["copies"]):
            cascade(i)
    graph.replay()
    torch.cuda.synchronize()
    reps = max(1, n // 2)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    t_graph = e0.elapsed_time(e1) / (reps * w["copies"])
    del graph
    line["cascade_graph_us"] = round(t_graph * 1e3, 2)
    line["cascade_graph_gbs"] = round(w["bytes_end_to_end"] / (t_graph * 1e-3) / 1e9, 2)

    if not args.no_cpu_baseline:
        gpu_out, _ = cascade(0)
        line["cpu_baseline"] = cpu_baseline(torch, w, gpu_out)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
