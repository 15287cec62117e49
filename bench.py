"""Benchmark of the cascade-decode operator set on one MI355X.

Workload (BASELINE config 2 end-to-end, plus config 4 at M=4096):
  * cascade decode, Llama-3-8B attention shapes: 32 query heads, 8 kv heads,
    head dim 128, bf16; a shared 8192-token prefix (64 pages of 128 tokens,
    permuted physical pages) read by stage-1 in the flattened form (one request,
    q_len = 64); 64 sequences whose own suffixes have geometric lengths (mean 512,
    clipped to [1, 4096]); the two partial results merged into bf16. The step
    runs the fused npu.cascade_decode op (stage-1, suffix, merge epilogue); the
    reference's three-op composition (fa_fp32_stage1, suffix_decode, lse_merge)
    is timed beside it, and each op alone.
  * the fused SwiGLU gate_up GEMM, activations [4096, 4096], weight
    [2*14336, 4096] bf16, fp32 accumulation, d = silu(g) * u in bf16.

value = end-to-end cascade HBM throughput: algorithmic bytes (q, prefix K/V read
once, every suffix K/V, block tables, seqlens, final bf16 O and merged LSE) /
measured time of one fused cascade decode. Inputs are resident in HBM; K/V pools rotate through enough copies
(>= 2 GiB distinct) that the 256 MB Infinity Cache cannot serve them.
Each timing loop launches its op back to back on the stream the kernels run on
(the step loop exactly --steps times, each component op at least 100 times),
with HIP events only at the loop's two ends (an event recorded between two
kernels delays the second by several microseconds).
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
NORM_M, NORM_K = 2048, 5120  # add_rms_norm_stats at the reference's prefill-main shape
ROTATE_BYTES = 2 << 30
# the kernels each op launches (an op's HIP-event time covers all of them)
OP_KERNELS = {"fa_fp32_stage1": "stage1_kernel + stage1_combine_kernel",
              "suffix_decode": "suffix_stream_kernel + suffix_fixup_kernel",
              "lse_merge": "lse_merge_kernel"}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    return ap.parse_args()


def suffix_lengths():
    import numpy as np
    rng = np.random.default_rng(0)
    return np.clip(rng.geometric(1.0 / 512, size=B), 1, 4096).astype(np.int64)


def build_workload(torch, dev):
    import numpy as np
    suf = suffix_lengths()
    nsb = [(int(s) + PAGE - 1) // PAGE for s in suf]
    npages = PREFIX // PAGE + sum(nsb)
    rng = np.random.default_rng(1)
    perm = rng.permutation(npages).astype(np.int32)
    bt_pre = torch.from_numpy(perm[:PREFIX // PAGE][None, :].copy()).to(dev)
    bt_suf_np = np.zeros((B, max(nsb)), dtype=np.int32)
    off = PREFIX // PAGE
    for b in range(B):
        bt_suf_np[b, :nsb[b]] = perm[off:off + nsb[b]]
        off += nsb[b]
    bt_suf = torch.from_numpy(bt_suf_np).to(dev)
    pool_bytes = 2 * npages * PAGE * KVH * D * 2
    copies = max(2, -(-ROTATE_BYTES // pool_bytes))
    g = torch.Generator(device=dev).manual_seed(0)
    pools = []
    for _ in range(copies):
        k = torch.randn(npages, PAGE, KVH, D, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
        v = torch.randn(npages, PAGE, KVH, D, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
        q = torch.randn(B, H, D, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
        pools.append((q, k, v))
    w = dict(
        pools=pools, bt_pre=bt_pre, bt_suf=bt_suf,
        qlens=torch.tensor([B], dtype=torch.int64, device=dev),
        kvlens=torch.tensor([PREFIX], dtype=torch.int64, device=dev),
        suf=torch.from_numpy(suf).to(dev), suf_np=suf, npages=npages, copies=copies,
    )
    # algorithmic bytes of one cascade step (inputs read once, final output written once)
    kv_tok = KVH * D * 2 * 2
    w["bytes_prefix_kernel"] = (B * H * D * 2 + PREFIX * kv_tok + bt_pre.numel() * 4 + 16
                                + B * H * D * 4 + B * H * 8 * 4)       # stage-1 reads + fp32 O + padded LSE
    w["bytes_suffix_kernel"] = (B * H * D * 2 + int(suf.sum()) * kv_tok + bt_suf.numel() * 4 + B * 8
                                + B * H * D * 2 + B * H * 4)            # suffix reads + bf16 O + LSE
    w["bytes_merge_kernel"] = B * H * D * (4 + 2 + 2) + B * H * (8 + 1) * 4
    w["bytes_end_to_end"] = (B * H * D * 2 + PREFIX * kv_tok + int(suf.sum()) * kv_tok
                             + (bt_pre.numel() + bt_suf.numel()) * 4 + (B + 1) * 8 + B * H * D * 2 + B * H * 4)
    w["flops_prefix"] = 4 * B * H * D * PREFIX
    return w


def cpu_baseline(torch):
    """Times the CPU oracle (numpy restatement, test infrastructure) on full
    cascade steps of the same workload: einsum loops, one thread (numpy's
    einsum without optimize= does not call BLAS). One warm-up step, then at
    least 5 timed steps and at least 10 s of work (at most ~30 s); the median
    step is reported."""
    import numpy as np
    sys.path.insert(0, REPO)
    from oracle import attention as A
    from oracle.merge import merge_fp64
    suf = suffix_lengths()
    rng = np.random.default_rng(2)
    nsb = [(int(s) + PAGE - 1) // PAGE for s in suf]
    npages = PREFIX // PAGE + sum(nsb)
    k = rng.standard_normal((npages, PAGE, KVH, D)).astype(np.float32)
    v = rng.standard_normal((npages, PAGE, KVH, D)).astype(np.float32)
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    bt_pre = np.arange(PREFIX // PAGE, dtype=np.int32)[None]
    bt_suf = np.zeros((B, max(nsb)), dtype=np.int32)
    off = PREFIX // PAGE
    for b in range(B):
        bt_suf[b, :nsb[b]] = np.arange(off, off + nsb[b])
        off += nsb[b]

    def step():
        O1, L1 = A.stage1(q, k, v, bt_pre, [B], [PREFIX])
        O2, L2 = A.suffix(q, k, v, bt_suf, suf)
        merge_fp64(O1, O2, L1, L2)

    step()  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < 10.0 and len(times) < 64):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > 30.0:
            break
    dt = float(np.median(times))
    kv_tok = KVH * D * 2 * 2
    nbytes = B * H * D * 2 + PREFIX * kv_tok + int(suf.sum()) * kv_tok + B * H * D * 2
    return {"value": round(nbytes / dt / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": "full cascade steps of the benchmark workload (stage-1 + suffix + merge) through "
                      "the numpy oracle: median of %d steps (%.2f s each, %.1f s total) after one warm-up"
                      % (len(times), dt, sum(times))}


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU; --gpus %d is not supported "
              "(the cascade-decode path would shard by kv head, with no exchange between GPUs)" % args.gpus,
              file=sys.stderr)
        sys.exit(2)
    import torch
    import cascade_amd  # noqa: F401
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()

    w = build_workload(torch, dev)
    a = torch.randn(GEMM_M, GEMM_K, device=dev, dtype=torch.float32).to(torch.bfloat16)
    wt = (torch.randn(2 * GEMM_I, GEMM_K, device=dev, dtype=torch.float32) * 0.02).to(torch.bfloat16)
    d_out = torch.empty(GEMM_M, GEMM_I, device=dev, dtype=torch.bfloat16)
    ws = torch.empty(GEMM_M, 2 * GEMM_I, device=dev, dtype=torch.bfloat16)

    # calibration copy of known size (read 256 MiB + write 256 MiB) for the PMC
    # traffic scale factor; outside the timed region
    src = torch.empty(128 << 20, dtype=torch.int16, device=dev).fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst

    def stage1(i):
        q, k, v = w["pools"][i % w["copies"]]
        return torch.ops.npu.fa_fp32_stage1(q, k, v, w["bt_pre"], w["qlens"], w["kvlens"], B)

    def suffix(i):
        q, k, v = w["pools"][i % w["copies"]]
        return torch.ops.npu.suffix_decode(q, k, v, w["bt_suf"], w["suf"])

    o1_fix, l1_fix = stage1(0)
    o2_fix, l2_fix = suffix(0)

    def merge(i):
        return torch.ops.npu.lse_merge(o1_fix, o2_fix, l1_fix, l2_fix, 1)

    def cascade(i):
        q, k, v = w["pools"][i % w["copies"]]
        return torch.ops.npu.cascade_decode(q, k, v, w["bt_pre"], w["kvlens"], k, v, w["bt_suf"], w["suf"])

    def cascade_unfused(i):
        o1, l1 = stage1(i)
        o2, l2 = suffix(i)
        return torch.ops.npu.lse_merge(o1, o2, l1, l2, 1)

    def gemm(i):
        torch.ops.npu.f3_gateup_epilogue(a, wt, ws, d_out, 1)

    # add_rms_norm_stats inputs, rotated over enough copies to leave the Infinity Cache
    norm_copies = 8
    norm_in = [(torch.randn(NORM_M, NORM_K, device=dev) * 0.5).to(torch.bfloat16) for _ in range(2 * norm_copies)]
    norm_gamma = (1.0 + torch.randn(NORM_K, device=dev) * 0.1).to(torch.bfloat16)

    def norm0(i):
        j = 2 * (i % norm_copies)
        return torch.ops.npu.add_rms_norm_stats(norm_in[j], norm_in[j + 1], None, None, 1e-6, 0)

    def norm1(i):
        j = 2 * (i % norm_copies)
        return torch.ops.npu.add_rms_norm_stats(norm_in[j], norm_in[j], norm_gamma, None, 1e-6, 1)

    def step(i):
        cascade(i)
        gemm(i)

    def timed(fn, n, first, warm=True):
        """Mean GPU time (ms) of n back-to-back calls, HIP events only at the two
        ends (an event between kernels costs the stream several microseconds).
        With `warm`, one untimed call first: a kernel's first launch in the
        process loads its code object (the step itself has its warmup steps)."""
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

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # the timed region: exactly `steps` full steps
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms_step = timed(step, args.steps, args.warmup, warm=False)
    wall = time.perf_counter() - t0

    # component timings: each op over the same number of back-to-back launches, at
    # least 100, so the start-up gap between the first event and the first kernel
    # (a host launch latency) is a small share of the loop
    n = max(args.steps, 100)
    ms = {"cascade": timed(cascade, n, 0), "cascade_unfused": timed(cascade_unfused, n, 0), "gemm": timed(gemm, n, 0),
          "stage1": timed(stage1, n, 0), "suffix": timed(suffix, n, 0), "merge": timed(merge, n, 0),
          "norm0": timed(norm0, n, 0), "norm1": timed(norm1, n, 0)}

    # decode-sized SwiGLU GEMMs (BASELINE config 4's other M values) over two weight
    # copies (470 MB together, beyond the Infinity Cache), so the weight stream is
    # measured from HBM
    wt_pair = [wt, (torch.randn(2 * GEMM_I, GEMM_K, device=dev, dtype=torch.float32) * 0.02).to(torch.bfloat16)]
    small_m = {}
    for mm in (1, 16, 256):
        a_m = torch.randn(mm, GEMM_K, device=dev, dtype=torch.float32).to(torch.bfloat16)
        d_m = torch.empty(mm, GEMM_I, device=dev, dtype=torch.bfloat16)

        def gemm_m(i, a_m=a_m, d_m=d_m):
            torch.ops.npu.f3_gateup_epilogue(a_m, wt_pair[i % 2], None, d_m, 1)
        t = timed(gemm_m, n, 0)
        small_m[str(mm)] = {"us": round(t * 1e3, 1),
                            "weight_gbs": round(2 * GEMM_I * GEMM_K * 2 / (t * 1e-3) / 1e9, 1)}
    del wt_pair

    # HIP-graph batch: one graph holding one fused cascade call per K/V pool copy,
    # replayed back to back (the plugin's graph mode); launch gaps disappear
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
    ms["cascade_graph"] = e0.elapsed_time(e1) / (reps * w["copies"])
    del graph

    cascade_gbs = w["bytes_end_to_end"] / (ms["cascade"] * 1e-3) / 1e9
    gemm_flops = 2.0 * GEMM_M * GEMM_K * 2 * GEMM_I
    gemm_tflops = gemm_flops / (ms["gemm"] * 1e-3) / 1e12
    per_kernel = {
        "fa_fp32_stage1": (ms["stage1"], w["bytes_prefix_kernel"]),
        "suffix_decode": (ms["suffix"], w["bytes_suffix_kernel"]),
        "lse_merge": (ms["merge"], w["bytes_merge_kernel"]),
    }
    dom = max(per_kernel, key=lambda n: per_kernel[n][0])
    dom_gbs = per_kernel[dom][1] / (per_kernel[dom][0] * 1e-3) / 1e9
    # HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    # (calibrated against a plain copy of known size)
    traffic = gemm_traffic = None
    tpath = os.path.join(REPO, "profiles", "pmc_traffic.json")
    if os.path.exists(tpath):
        tj = json.load(open(tpath))
        traffic = tj.get(dom)
        gemm_traffic = tj.get("f3_gateup_epilogue")

    line = {
        "metric": "cascade-decode attn HBM GB/s (% of peak) + SwiGLU GEMM TFLOP/s at 1 MI355X",
        "value": round(cascade_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "wall_ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) bf16 q/k/v, N(0,0.02) weights, seeded)",
        "config": {
            "workload": "cascade decode H32/KVH8/D128, shared prefix 8192 (flattened stage-1, q_len 64), "
                        "64 suffixes ~Geometric(mean 512) clipped [1,4096] (%d tokens), page 128, permuted "
                        "pages, merge to bf16; plus fused SwiGLU gate_up GEMM M=%d K=%d I=%d"
                        % (int(w["suf_np"].sum()), GEMM_M, GEMM_K, GEMM_I),
            "kv_rotation_copies": w["copies"],
        },
        "cascade_pct_of_hbm_peak": round(100.0 * cascade_gbs / HBM_PEAK_GBS, 2),
        "cascade_us": round(ms["cascade"] * 1e3, 2),
        "cascade_unfused_us": round(ms["cascade_unfused"] * 1e3, 2),
        "cascade_graph_us": round(ms["cascade_graph"] * 1e3, 2),
        "cascade_graph_gbs": round(w["bytes_end_to_end"] / (ms["cascade_graph"] * 1e-3) / 1e9, 2),
        "per_op_us": {n: round(v[0] * 1e3, 2) for n, v in per_kernel.items()},
        "add_rms_norm_stats": {
            "shape": [NORM_M, NORM_K], "dtype": "bf16",
            "mode0_us": round(ms["norm0"] * 1e3, 2),
            "mode0_gbs": round((3 * NORM_M * NORM_K * 2 + NORM_M * 4) / (ms["norm0"] * 1e-3) / 1e9, 1),
            "mode1_us": round(ms["norm1"] * 1e3, 2),
            "mode1_gbs": round((2 * NORM_M * NORM_K * 2 + NORM_K * 2 + NORM_M * 4) / (ms["norm1"] * 1e-3) / 1e9, 1)},
        "swiglu_gemm": {"tflops": round(gemm_tflops, 1), "us": round(ms["gemm"] * 1e3, 1),
                        "pct_of_bf16_peak": round(100.0 * gemm_tflops / BF16_PEAK_TFLOPS, 2)},
        "swiglu_gemm_small_m": small_m,
        "roofline": {"kernel": dom + " op (" + OP_KERNELS[dom] + ")", "bound": "hbm", "achieved": round(dom_gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": traffic},
        "roofline_gemm": {"kernel": "f3_gateup_epilogue mode 1", "bound": "mfma", "achieved": round(gemm_tflops, 1),
                          "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                          "frac": round(gemm_tflops / BF16_PEAK_TFLOPS, 4), "traffic": gemm_traffic},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(torch)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
