#!/usr/bin/env python3
"""Benchmark of the WUSH INT4 W4A4 layer on one MI355X.

Metric: microseconds per layer, and speedup vs hipBLASLt bf16,
for the Llama-70B FFN shape K=8192, N=57344 at M = 1 / 8 / 32 / 4096.

A "step" is one forward pass of the layer's hot path over one batch of
synthetic activations, chained as the reference's official bench does
(reference bench/exp_p13_official.py:31-39; my_int4.chain.make_chain):
  M == 1 : fused_transform_quant_int4_smallm -> w4a4_gemv
  M <= 4 : fused_transform_quant_int4_smallm -> w4a4_gemv_multi
  M <= 32: fused_transform_quant_int4_smallm -> w4a4_gemm_s4
  else   : fused_transform_quant_int4_v3     -> w4a4_gemm_s4
with the weights pre-quantized (W' = W T^-1, sigma-clip s4 + bf16 scales) and
resident in HBM; every step works on its own layer's weights and transform,
cycling over --copies distinct weight copies that together exceed the 256 MB
MALL, so every step streams its weights from HBM.

Timing of each M (the headline `value` is M = 1):
  * `us`: exactly --steps layer steps in 5 groups (sizes differ by at most
    one), each group one replay of a HIP graph that holds the group's steps,
    timed with HIP events on the replay stream; the median per-step time over
    the groups.  The device is synchronized before and after.
  * `us_graph12`: a graph of 12 layer steps (a decoder stack's per-token
    graph), median per step over 5 groups of replays.
  * `us_1step`: the reference's method (exp_p13_official.py:15-29): a graph of
    one step, median per step over 5 groups of replays, so every step also pays
    the replay launch cost (about 5 us on this part).
hipBLASLt bf16 at the same shape is timed the same three ways.

Also reported: the roofline of the dominant kernel at M=1 (gemv_int4, HBM-
bound; timed alone with HIP events on its launch stream), and the CPU
baseline -- the reference's CPU path (rtn_int4 quant + dequantized fp32
matmul) restated with the same torch ops in oracle/rtn_torch.py, on this
host's cores: the L70 layer at M=1 on a bounded weight sample, and BASELINE
config 1 (X fp16 16x4096, W fp16 4096x4096, seed 0) at full size.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--sweep]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "µs/layer + speedup vs hipBLASLt bf16, K=8192 N=57344 at M=1/8/32/4096"
K_L70, N_L70 = 8192, 57344
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_int4_l70_m1_traffic.txt")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--ms", default="1,8,32,64,4096", help="comma-separated M values")
    ap.add_argument("--copies", type=int, default=3, help="distinct weight copies (MALL defeat)")
    ap.add_argument("--graph-steps", type=int, default=12, help="layer steps captured in one HIP graph")
    ap.add_argument("--no-blas", action="store_true", help="skip the hipBLASLt bf16 baseline")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--K", type=int, default=K_L70)
    ap.add_argument("--N", type=int, default=N_L70)
    ap.add_argument("--counter-workload", action="store_true",
                    help="launch every kernel of the path 3 times, then a 512 MiB copy (rocprofv3 --pmc)")
    ap.add_argument("--sweep", action="store_true",
                    help="the reference's shape x M matrix (bench/exp_p13_matrix.py): a table, one JSON line")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only launch the M=1 dominant kernel (for rocprofv3 runs)")
    return ap.parse_args()


FP16_PEAK_TFLOPS = 2500.0       # dense fp16 MFMA (the prefill kernel's instruction)
F32_MFMA_PEAK_TFLOPS = 157.3    # fp32 MFMA (the fused transform's instruction)


def capture(fns):
    """One HIP graph holding one call of each function, after two eager passes."""
    import torch
    for _ in range(2):
        for fn in fns:
            fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for fn in fns:
            fn()
    return g


def group_sizes(steps: int, groups: int = 5):
    """`steps` split into `groups` (at most `steps`) sizes that differ by at most one."""
    n = max(1, min(groups, steps))
    base, extra = divmod(steps, n)
    return [base + (1 if i < extra else 0) for i in range(n)]


def time_steps(make_graph, steps: int, warmup: int):
    """Exactly `steps` layer steps in 5 groups, each group one replay of a graph
    holding the group's steps (make_graph(n) -> graph of n steps), timed with
    HIP events on the current stream, the device synchronized before and after.
    Returns the median per-step seconds over the groups and the per-group values."""
    import torch
    sizes = group_sizes(steps)
    graphs = {n: make_graph(n) for n in sorted(set(sizes))}
    g0, done = graphs[sizes[0]], 0
    while done < warmup:
        g0.replay()
        done += sizes[0]
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    marks = []
    for n in sizes:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        graphs[n].replay()
        e1.record(stream)
        marks.append((e0, e1, n))
    torch.cuda.synchronize()
    per = [e0.elapsed_time(e1) * 1e-3 / n for e0, e1, n in marks]
    del graphs
    return statistics.median(per), per


def time_med5(graph, steps_per_replay: int, reps: int):
    """The reference's med5 (bench/exp_p13_official.py:15-23): 3 warm-up
    replays, then 5 groups of `reps` replays, each group timed with HIP events;
    median per-step seconds."""
    import torch
    for _ in range(3):
        graph.replay()
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    marks = []
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            graph.replay()
        e1.record(stream)
        marks.append((e0, e1))
    torch.cuda.synchronize()
    return statistics.median(e0.elapsed_time(e1) * 1e-3 / (reps * steps_per_replay) for e0, e1 in marks)


def ref_reps(M: int) -> int:
    """Replays per timing group of a one-step graph (bench/exp_p13_matrix.py:65)."""
    return 100 if M <= 8 else (30 if M <= 64 else 8)


def prefill_mfma(M: int, N: int, K: int) -> str:
    """MFMA type of the w4a4_gemm_s4 kernel for M rows at the bench's shapes:
    the fp16 tiles from M = 256 when K % 256 == 0 (every bench shape has at
    least 16 column tiles of 256, which with M >= 256 meets the planner's
    tile-count condition, except Qwen3-8B K=N=4096 below M = 2048), the fp16
    streaming kernel at 32 < M <= 64 when 224 to 256 workgroups of 224
    columns cover N and K % 1024 == 0, int8 otherwise."""
    wgs = -(-N // 224)
    if (M >= 256 and K % 256 == 0) or (32 < M <= 64 and 224 <= wgs <= 256 and K % 1024 == 0):
        return "fp16"
    return "int8"


SWEEP_SHAPES = [("Qwen3-8B", 4096, 4096), ("Qwen3-8B", 4096, 24576), ("Qwen3-8B", 12288, 4096),
                ("Llama-70B", 8192, 8192), ("Llama-70B", 8192, 57344)]
SWEEP_MS = [1, 2, 4, 8, 16, 32, 64, 128, 256, 1024, 2048, 4096]
# bench/exp_p13_matrix.py:32 (GEMM alone, K = 4096) and :53-54 (9 layer shapes, K = 4096)
REF_GEMM_SHAPES = [(8, 4096), (64, 4096), (2048, 512), (4096, 4096)]
REF_E2E_SHAPES = [(1, 4096), (2, 4096), (4, 4096), (8, 4096), (16, 4096), (32, 4096), (64, 4096),
                  (2048, 512), (4096, 4096)]


def sweep(args):
    """The reference's performance matrices:
    * bench/exp_p13_official.py:42-44 -- five FFN shapes x M = 1..4096, the
      layer step of my_int4.chain (its dispatch by M) against hipBLASLt fp16
      (the reference's baseline) and bf16, --graph-steps steps per HIP graph
      over enough distinct weight copies to exceed the 256 MB MALL (the
      reference replays one warm weight set), median of 5 groups;
    * bench/exp_p13_matrix.py:32-45 -- w4a4_gemm_s4 alone at (M, N) = (8,
      4096), (64, 4096), (2048, 512), (4096, 4096), K = 4096, one step per
      graph replay, median of 5 groups (the reference's method), against the
      hipBLASLt GEMMs at the same shape;
    * bench/exp_p13_matrix.py:53-73 -- the 9 layer shapes at K = 4096
      (M = 1..64 at N = 4096, 2048 x 512, 4096 x 4096), one step per replay.
    A table goes to stderr and one JSON line to stdout."""
    import torch
    from my_int4 import _C
    from my_int4.chain import make_chain
    from wush_int4_kernel_amd.wush_transform import compute_wush_transform, transform_weights

    dev = torch.device("cuda:0")
    torch.backends.cuda.preferred_blas_library("hipblaslt")
    gen = torch.Generator(device=dev).manual_seed(0)

    def weights(K, N, copies_bytes=300_000_000):
        W = (torch.randn(N, K, generator=gen, device=dev) * 0.02).to(torch.bfloat16)
        Xc = torch.randn(256, K, generator=gen, device=dev)
        T64 = compute_wush_transform(Xc.double(), W.double())
        wq, ws = _C.quant_int4(transform_weights(W.double(), T64).to(torch.bfloat16).contiguous())
        T = T64.to(torch.bfloat16).contiguous()
        nc = max(2, min(8, -(-copies_bytes // (N * K * 9 // 16))))
        copies = [(wq, ws, T)] + [(wq.clone(), ws.clone(), T.clone()) for _ in range(nc - 1)]
        nb = max(2, min(8, -(-copies_bytes // (N * K * 2))))
        blas_w = [W] + [W.clone() for _ in range(nb - 1)]
        return copies, blas_w, [w.half() for w in blas_w]

    def graph_of(fns_for_step, n):
        return capture([fns_for_step(i) for i in range(n)])

    rows = []
    for model, K, N in SWEEP_SHAPES:
        copies, blas_w, half_w = weights(K, N)
        nc, nb = len(copies), len(blas_w)
        for M in SWEEP_MS:
            X = torch.randn(M, K, generator=gen, device=dev).to(torch.bfloat16)
            X16 = X.half()
            gs = args.graph_steps
            reps = max(1, -(-args.steps // gs)) if M <= 64 else 1
            t4 = time_med5(graph_of(lambda i: make_chain(X, copies[i % nc][2], copies[i % nc][0],
                                                         copies[i % nc][1], M), gs), gs, reps)
            tb = time_med5(graph_of(lambda i: (lambda Wc=blas_w[i % nb]: torch.matmul(X, Wc.t())), gs), gs, reps)
            th = time_med5(graph_of(lambda i: (lambda Wc=half_w[i % nb]: torch.matmul(X16, Wc.t())), gs), gs, reps)
            tf = 2 * M * N * K / 1e12
            rows.append({"model": model, "K": K, "N": N, "M": M, "int4_us": round(t4 * 1e6, 2),
                         "int4_tflops": round(tf / t4, 2), "hipblaslt_fp16_us": round(th * 1e6, 2),
                         "hipblaslt_bf16_us": round(tb * 1e6, 2), "speedup_vs_fp16": round(th / t4, 3),
                         "speedup_vs_bf16": round(tb / t4, 3)})
            log(f"{model:9s} K={K:5d} N={N:5d} M={M:5d} | int4 {t4 * 1e6:9.2f} us {tf / t4:7.1f} TF/s | "
                f"fp16 {th * 1e6:9.2f} us | bf16 {tb * 1e6:9.2f} us | {th / t4:5.2f}x {tb / t4:5.2f}x")
        del copies, blas_w, half_w
        torch.cuda.empty_cache()

    # the reference's GEMM-alone table and 9 layer shapes, K = 4096, one step per replay
    K = 4096
    gemm_rows, e2e_rows = [], []
    for M, N in REF_GEMM_SHAPES:
        copies, blas_w, half_w = weights(K, N)
        wq, ws, T = copies[0]
        X = torch.randn(M, K, generator=gen, device=dev).to(torch.bfloat16)
        xq, xs = _C.fused_transform_quant_int4_v3(X, T)
        reps = ref_reps(M)
        t4 = time_med5(capture([lambda: _C.w4a4_gemm_s4(xq, xs, wq, ws)]), 1, reps)
        tb = time_med5(capture([lambda: torch.matmul(X, blas_w[0].t())]), 1, reps)
        X16 = X.half()
        th = time_med5(capture([lambda: torch.matmul(X16, half_w[0].t())]), 1, reps)
        # the same with graph_steps calls per replay, over the weight copies
        gs = args.graph_steps
        r12 = max(1, reps // gs)
        t4g = time_med5(graph_of(lambda i: (lambda c=copies[i % len(copies)]: _C.w4a4_gemm_s4(xq, xs, c[0], c[1])),
                                 gs), gs, r12)
        tbg = time_med5(graph_of(lambda i: (lambda Wc=blas_w[i % len(blas_w)]: torch.matmul(X, Wc.t())), gs), gs, r12)
        gemm_rows.append({"M": M, "N": N, "K": K, "w4a4_gemm_s4_us": round(t4 * 1e6, 2),
                          "tflops": round(2 * M * N * K / t4 / 1e12, 2), "hipblaslt_fp16_us": round(th * 1e6, 2),
                          "hipblaslt_bf16_us": round(tb * 1e6, 2), "speedup_vs_fp16": round(th / t4, 3),
                          "speedup_vs_bf16": round(tb / t4, 3), "w4a4_gemm_s4_us_graph": round(t4g * 1e6, 2),
                          "hipblaslt_bf16_us_graph": round(tbg * 1e6, 2),
                          "speedup_vs_bf16_graph": round(tbg / t4g, 3)})
        log(f"GEMM alone {M:5d}x{N:5d}x{K}: {t4 * 1e6:8.2f} us | fp16 {th * 1e6:8.2f} | bf16 {tb * 1e6:8.2f} | "
            f"{th / t4:5.2f}x {tb / t4:5.2f}x | {gs} per replay: {t4g * 1e6:8.2f} us vs bf16 {tbg * 1e6:8.2f}")
        del copies, blas_w, half_w
        torch.cuda.empty_cache()
    for M, N in REF_E2E_SHAPES:
        copies, blas_w, half_w = weights(K, N)
        wq, ws, T = copies[0]
        X = torch.randn(M, K, generator=gen, device=dev).to(torch.bfloat16)
        X16 = X.half()
        reps = ref_reps(M)
        t4 = time_med5(capture([make_chain(X, T, wq, ws, M)]), 1, reps)
        tb = time_med5(capture([lambda: torch.matmul(X, blas_w[0].t())]), 1, reps)
        th = time_med5(capture([lambda: torch.matmul(X16, half_w[0].t())]), 1, reps)
        gs = args.graph_steps
        r12 = max(1, reps // gs)
        t4g = time_med5(graph_of(lambda i: make_chain(X, copies[i % len(copies)][2], copies[i % len(copies)][0],
                                                      copies[i % len(copies)][1], M), gs), gs, r12)
        tbg = time_med5(graph_of(lambda i: (lambda Wc=blas_w[i % len(blas_w)]: torch.matmul(X, Wc.t())), gs), gs, r12)
        e2e_rows.append({"M": M, "N": N, "K": K, "layer_us": round(t4 * 1e6, 2),
                         "hipblaslt_fp16_us": round(th * 1e6, 2), "hipblaslt_bf16_us": round(tb * 1e6, 2),
                         "speedup_vs_fp16": round(th / t4, 3), "speedup_vs_bf16": round(tb / t4, 3),
                         "layer_us_graph": round(t4g * 1e6, 2), "hipblaslt_bf16_us_graph": round(tbg * 1e6, 2),
                         "speedup_vs_bf16_graph": round(tbg / t4g, 3)})
        log(f"layer {M:5d}x{N:5d}x{K}: {t4 * 1e6:8.2f} us | fp16 {th * 1e6:8.2f} | bf16 {tb * 1e6:8.2f} | "
            f"{th / t4:5.2f}x {tb / t4:5.2f}x | {gs} per replay: {t4g * 1e6:8.2f} us vs bf16 {tbg * 1e6:8.2f}")
        del copies, blas_w, half_w
        torch.cuda.empty_cache()
    print(json.dumps({"sweep": "reference matrices (bench/exp_p13_official.py, bench/exp_p13_matrix.py)",
                      "rows": rows, "gemm_alone_k4096": gemm_rows, "layers_k4096": e2e_rows}))


def layer_bytes(M, N, K):
    """Algorithmic HBM bytes of one layer: x bf16 + T bf16 + W4 codes/scales + y fp16."""
    return 2 * M * K + 64 * K + N * K // 2 + N * K // 16 + 2 * M * N


def gemv_bytes(M, N, K):
    """Algorithmic bytes of one gemv_int4 launch: x codes/scales, W4 codes/scales, y fp16."""
    return M * K // 2 + M * K // 16 + N * K // 2 + N * K // 16 + 2 * M * N


def read_traffic():
    """HBM bytes per launch of gemv_int4 at L70 M=1 from the committed rocprofv3 summary."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs on one GPU: the W4A4 layer path has no "
                          "multi-GPU mode (it would shard the weight rows along N, column-"
                          "parallel, with one all-gather of y); run with --gpus 1"}))
        sys.exit(2)

    if args.sweep:
        return sweep(args)

    import torch
    from my_int4 import _C
    from wush_int4_kernel_amd import capi
    from my_int4.chain import make_chain, route
    from wush_int4_kernel_amd.wush_transform import compute_wush_transform, transform_weights

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    K, N = args.K, args.N
    Ms = [int(m) for m in args.ms.split(",") if m]

    # ---------------------------------------------------------------- inputs
    t0 = time.time()
    gcpu = torch.Generator().manual_seed(0)
    n_out = int(round(0.01 * K))
    out_ch = torch.randperm(K, generator=gcpu)[:n_out].to(dev)
    gdev = torch.Generator(device=dev).manual_seed(0)

    def activations(M, gen):
        x = torch.randn(M, K, generator=gen, device=dev, dtype=torch.float32)
        x[:, out_ch] *= 50.0
        return x

    W = torch.randn(N, K, generator=gdev, device=dev, dtype=torch.float32) * 0.02
    Xcal = activations(512, gdev)
    T64 = compute_wush_transform(Xcal.double(), W.double())
    T = T64.to(torch.bfloat16).contiguous()
    Wt = transform_weights(W.double(), T64).to(torch.bfloat16).contiguous()
    wq, ws = _C.quant_int4(Wt)
    del W, Xcal
    torch.cuda.synchronize()
    copies = [(wq, ws, T)] + [(wq.clone(), ws.clone(), T.clone()) for _ in range(args.copies - 1)]
    log(f"[bench] weights ready: N={N} K={K}, {args.copies} copies x "
        f"{(wq.numel() + ws.numel() * 2) / 1e6:.1f} MB ({time.time() - t0:.1f}s)")

    stream = torch.cuda.current_stream()

    # -------------------------------------------------------- kernel-only mode
    if args.kernel_only:
        M = 1
        X = activations(M, gdev).to(torch.bfloat16)
        xq, xs = _C.fused_transform_quant_int4_smallm(X, T)
        y = torch.empty(M, N, dtype=torch.float16, device=dev)
        for i in range(args.warmup + args.steps):
            cq, cs, _ = copies[i % len(copies)]
            capi.gemv_int4(xq.data_ptr(), xs.data_ptr(), cq.data_ptr(), cs.data_ptr(), y.data_ptr(),
                           M, N, K, stream.cuda_stream)
        torch.cuda.synchronize()
        # calibration kernel for the HBM counters: a plain 512 MiB device copy
        src = torch.empty(256 << 20, dtype=torch.int16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"kernel_only": "gemv_int4", "launches": args.warmup + args.steps,
                          "gemv_algorithmic_bytes": gemv_bytes(M, N, K),
                          "copy_bytes_each_way": src.numel() * 2}))
        return

    # ------------------------------------------------- hardware-counter workload
    if args.counter_workload:
        # Each kernel of the path three times on bench shapes, then the copy
        # that calibrates FETCH_SIZE / WRITE_SIZE.  For rocprofv3 --pmc passes.
        def launch_product(kind, M_, N_, K_, wq_, ws_, reps=3):
            xq_, xs_ = _C.quant_int4(activations_k(M_, K_))
            y_ = torch.empty(M_, N_, dtype=torch.float16, device=dev)
            wsb = capi.gemm_s4_workspace_bytes(M_, N_, K_)
            work = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
            for _ in range(reps):
                if kind == "gemv":
                    capi.gemv_int4(xq_.data_ptr(), xs_.data_ptr(), wq_.data_ptr(), ws_.data_ptr(), y_.data_ptr(),
                                   M_, N_, K_, stream.cuda_stream)
                else:
                    capi.gemm_s4(xq_.data_ptr(), xs_.data_ptr(), wq_.data_ptr(), ws_.data_ptr(), y_.data_ptr(),
                                 M_, N_, K_, work.data_ptr() if wsb else None, wsb, stream.cuda_stream)

        def activations_k(M_, K_):
            return torch.randn(M_, K_, generator=gdev, device=dev).to(torch.bfloat16)

        launch_product("gemv", 1, N, K, wq, ws)            # L70 M=1 decode
        launch_product("gemv", 8, N, K, wq, ws)            # L70 M=8 decode
        launch_product("gemm", 32, N, K, wq, ws)           # L70 M=32 (in-workgroup K-split streaming GEMM)
        launch_product("gemm", 64, N, K, wq, ws)           # L70 M=64 (fp16-MFMA streaming GEMM)
        for _ in range(3):
            _C.fused_transform_quant_int4_smallm(activations(1, gdev).to(torch.bfloat16), T)
            _C.fused_transform_quant_int4(activations(4096, gdev).to(torch.bfloat16), T)
            _C.quant_int4(Wt)
        Wq8, Ws8 = _C.quant_int4((torch.randn(24576, 4096, generator=gdev, device=dev) * 0.02).to(torch.bfloat16))
        launch_product("gemm", 8, 24576, 4096, Wq8, Ws8)   # Qwen3-8B M=8 (K-split streaming GEMM, 8 rows)
        W3, S3 = _C.quant_int4((torch.randn(4096, 4096, generator=gdev, device=dev) * 0.02).to(torch.bfloat16))
        launch_product("gemm", 4096, 4096, 4096, W3, S3)  # 4096^3 prefill tiles
        del W3, S3
        # L70 M=4096 prefill and hipBLASLt bf16 at the same shape: the clock
        # (GRBM_GUI_ACTIVE) and MFMA-busy comparison of the two
        launch_product("gemm", 4096, N, K, wq, ws)
        torch.backends.cuda.preferred_blas_library("hipblaslt")
        Xp = activations_k(4096, K)
        for _ in range(3):
            torch.matmul(Xp, Wt.t())
        del Xp
        torch.cuda.synchronize()
        src = torch.empty(256 << 20, dtype=torch.int16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"counter_workload": "done", "copy_bytes_each_way": src.numel() * 2}))
        return

    # ------------------------------------------------------------- layer sweep
    torch.backends.cuda.preferred_blas_library("hipblaslt")
    blas_w = None if args.no_blas else [Wt, Wt.clone()]
    layers = {}
    gs = args.graph_steps
    for M in Ms:
        X = activations(M, gdev).to(torch.bfloat16).contiguous()

        def chain_graph(n):
            return capture([make_chain(X, copies[i % len(copies)][2], copies[i % len(copies)][0],
                                       copies[i % len(copies)][1], M) for i in range(n)])

        t_int4, per_group = time_steps(chain_graph, args.steps, args.warmup)
        reps12 = max(1, -(-args.steps // gs)) if M <= 64 else 1
        t12 = time_med5(chain_graph(gs), gs, reps12)
        t1 = time_med5(chain_graph(1), 1, ref_reps(M))
        mfma = prefill_mfma(M, N, K)
        peak = FP16_PEAK_TFLOPS if mfma == "fp16" else INT8_PEAK_TOPS
        tflops = 2 * M * N * K / t_int4 / 1e12
        entry = {
            "us": round(t_int4 * 1e6, 2),
            "us_groups": [round(t * 1e6, 2) for t in per_group],
            "us_graph12": round(t12 * 1e6, 2),
            "us_1step": round(t1 * 1e6, 2),
            "chain": " -> ".join(route(M)),
            "layer_bytes": layer_bytes(M, N, K),
            "hbm_gbs": round(layer_bytes(M, N, K) / t_int4 / 1e9, 1),
            "hbm_frac": round(layer_bytes(M, N, K) / t_int4 / 1e9 / HBM_PEAK_GBS, 4),
            "mfma": mfma,
            "mfma_tops": round(tflops, 2),
            "mfma_frac": round(tflops / peak, 4),
            # the north star's roofline for prefill-sized GEMM: the int8 MFMA peak
            "int8_peak_frac": round(tflops / INT8_PEAK_TOPS, 4),
        }
        if blas_w is not None:
            def blas_graph(n):
                return capture([lambda Wc=blas_w[i % len(blas_w)]: torch.matmul(X, Wc.t()) for i in range(n)])

            tb, _ = time_steps(blas_graph, args.steps, args.warmup)
            tb12 = time_med5(blas_graph(gs), gs, reps12)
            tb1 = time_med5(blas_graph(1), 1, ref_reps(M))
            entry.update({
                "hipblaslt_bf16_us": round(tb * 1e6, 2),
                "hipblaslt_bf16_us_graph12": round(tb12 * 1e6, 2),
                "hipblaslt_bf16_us_1step": round(tb1 * 1e6, 2),
                "speedup_vs_hipblaslt": round(tb / t_int4, 3),
                "speedup_vs_hipblaslt_graph12": round(tb12 / t12, 3),
                "speedup_vs_hipblaslt_1step": round(tb1 / t1, 3),
            })
        layers[f"M={M}"] = entry
        log(f"[bench] M={M}: {entry}")
        torch.cuda.empty_cache()

    # ---------------------------------------- the path's other ops, timed alone
    ops = {}
    # fused transform + quant of X 2048x4096 (1% outlier channels x50),
    # T from this build's WUSH solve on a 512-row calibration draw; VALU-bound when bit-exact
    Mc, Kc = 2048, 4096
    gc = torch.Generator(device=dev).manual_seed(1)
    och = torch.randperm(Kc, generator=gcpu)[:int(round(0.01 * Kc))].to(dev)

    def acts_c(m):
        x = torch.randn(m, Kc, generator=gc, device=dev, dtype=torch.float32)
        x[:, och] *= 50.0
        return x

    # 20 distinct X copies (336 MB, more than the 256 MB MALL), so each call
    # reads its X from HBM as a layer's fresh activations would be
    Xc2s = [acts_c(Mc).to(torch.bfloat16) for _ in range(20)]
    Wc2 = torch.randn(Kc, Kc, generator=gc, device=dev, dtype=torch.float32) * 0.02
    Tc2 = compute_wush_transform(acts_c(512).double(), Wc2.double()).to(torch.bfloat16).contiguous()
    # 40 calls per graph replay, as the layer steps: a replay costs about 10 us
    # beyond its kernels on this part, 1 us per call at 10 calls
    t = time_med5(capture([lambda Xc=Xc2s[i % len(Xc2s)]: _C.fused_transform_quant_int4(Xc, Tc2)
                           for i in range(40)]), 40, 1)
    del Xc2s
    tq_bytes = 2 * Mc * Kc + 64 * Kc + Mc * Kc // 2 + Mc * Kc // 16
    tq_macs = 32 * Mc * Kc              # 32 MACs per element, on the fp32 matrix cores
    ops["fused_tq_cfg2"] = {
        "us": round(t * 1e6, 2), "shape": f"X {Mc}x{Kc} bf16 (20 copies in turn), T {Kc // 32}x32x32",
        "hbm_bytes": tq_bytes, "hbm_gbs": round(tq_bytes / t / 1e9, 1),
        "hbm_frac": round(tq_bytes / t / 1e9 / HBM_PEAK_GBS, 4),
        "fp32_macs": tq_macs, "mfma_f32_frac": round(2 * tq_macs / t / (F32_MFMA_PEAK_TFLOPS * 1e12), 4),
    }
    # a2/a3: quant_int4 of one Llama-70B weight tensor (N x K bf16), HBM-bound
    # 8 calls per replay (1.2 GB each): the replay's own cost spread as in the other op timings
    t = time_med5(capture([lambda: _C.quant_int4(Wt)] * 8), 8, 1)
    q_bytes = N * K * 2 + N * K // 2 + N * K // 16
    ops["quant_int4_l70_weights"] = {
        "us": round(t * 1e6, 2), "shape": f"{N}x{K} bf16", "hbm_bytes": q_bytes,
        "hbm_gbs": round(q_bytes / t / 1e9, 1), "hbm_frac": round(q_bytes / t / 1e9 / HBM_PEAK_GBS, 4),
    }
    log(f"[bench] ops: {ops}")
    del blas_w
    torch.cuda.empty_cache()

    # --------------------------------------------- roofline of the M=1 kernel
    M = 1
    X = activations(M, gdev).to(torch.bfloat16)
    xq, xs = _C.fused_transform_quant_int4_smallm(X, T)
    y = torch.empty(M, N, dtype=torch.float16, device=dev)
    launches = max(50, args.steps)

    def launch(i):
        cq, cs, _ = copies[i % len(copies)]
        capi.gemv_int4(xq.data_ptr(), xs.data_ptr(), cq.data_ptr(), cs.data_ptr(), y.data_ptr(),
                       M, N, K, stream.cuda_stream)

    for i in range(10):
        launch(i)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(launches):
        launch(i)
    e1.record(stream)
    torch.cuda.synchronize()
    t_kernel = e0.elapsed_time(e1) / 1e3 / launches
    alg = gemv_bytes(M, N, K)
    achieved = alg / t_kernel / 1e9
    roofline = {
        "kernel": "gemv_int4_kernel<1> (L70, M=1)",
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": read_traffic(),
        "algorithmic_bytes": alg,
        "avg_launch_us": round(t_kernel * 1e6, 2),
    }
    log(f"[bench] roofline: {roofline}")

    # ------------------------------------------------------------ CPU baseline
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(wq, ws, X, N, K)
        log(f"[bench] cpu baseline: {cpu}")

    head = layers.get("M=1") or next(iter(layers.values()))
    out = {
        "metric": METRIC,
        "value": head["us"],
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us"] / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4",
        "data": "synthetic: seeded N(0,1) activations with 1% outlier channels x50, N(0,0.02) weights "
                "transformed by this build's WUSH T and sigma-clip quantized",
        "config": {
            "workload": f"Llama-70B FFN layer K={K} N={N}, M=1: fused_transform_quant_int4_smallm + w4a4_gemv; "
                        f"{args.steps} layer steps timed as 5 graph replays of {'/'.join(map(str, sorted(set(group_sizes(args.steps)))))} "
                        f"steps each (median per step), each step on its own weights cycling over {args.copies} "
                        f"distinct copies",
            "K": K, "N": N, "M": 1,
        },
        "layers": layers,
        "ops": ops,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "device": torch.cuda.get_device_name(0),
    }
    print(json.dumps(out))


def _median_time(fn, reps=5):
    fn()
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return statistics.median(ts)


def cpu_config1(threads: int):
    """BASELINE config 1 at full size on the host: X fp16 16x4096 ~ N(0,1) with
    1% of the K channels x50, W fp16 4096x4096 ~ N(0,0.02), seed 0; quant(X),
    quant(W) and dequant + fp32 matmul (my_int4/rtn_int4.py:33-75, restated in
    oracle/rtn_torch.py), each the median of 5 after a warm-up, on `threads`
    torch threads.  Returns seconds."""
    import torch

    from oracle import rtn_torch

    g = torch.Generator().manual_seed(0)
    M1, K1, N1 = 16, 4096, 4096
    ch = torch.randperm(K1, generator=g)[:int(round(0.01 * K1))]
    X = torch.randn(M1, K1, generator=g)
    X[:, ch] *= 50.0
    X = X.half()
    W = (torch.randn(N1, K1, generator=g) * 0.02).half()
    torch.set_num_threads(threads)
    t_qx = _median_time(lambda: rtn_torch.quant(X))
    t_qw = _median_time(lambda: rtn_torch.quant(W))
    xq, xs = rtn_torch.quant(X)
    wq, ws = rtn_torch.quant(W)
    t_mm = _median_time(lambda: rtn_torch.w4a4_matmul(xq, xs, wq, ws))
    return t_qx, t_qw, t_mm


def cpu_baseline(wq, ws, X, N, K):
    """The reference CPU path on this host (my_int4/rtn_int4.py:33-75, restated
    with the same eager torch CPU ops in oracle/rtn_torch.py, bit-identical to
    the C oracle), on the host's cores (at most 16, the box's share per GPU):
    * the headline: the L70 layer at M=1 -- rtn quant of x, dequant of the
      weights and the fp32 matmul -- on a bounded sample, the first 16384 of
      the N weight rows, median of 5 after a warm-up, scaled by N/16384
      (dequant and matmul are linear in N; the x quant is counted once); a
      single-thread figure on a 2048-row sample beside it;
    * BASELINE config 1 at full size (cpu_config1), on all threads and on one."""
    import torch

    from oracle import rtn_torch

    threads = max(1, min(os.cpu_count() or 1, 16))
    S = min(16384, N)
    wq_c = wq[:S].cpu()
    ws_c = ws[:S].cpu()
    x_c = X.cpu()

    torch.set_num_threads(threads)
    xq, xs = rtn_torch.quant(x_c)
    t_qx = _median_time(lambda: rtn_torch.quant(x_c))
    t_dw = _median_time(lambda: rtn_torch.dequant(wq_c, ws_c))
    wd = rtn_torch.dequant(wq_c, ws_c)
    xd = rtn_torch.dequant(xq, xs)
    t_mm = _median_time(lambda: xd @ wd.T)
    del wd
    per_layer = t_qx + (t_dw + t_mm) * (N / S)
    S1 = min(2048, N)
    torch.set_num_threads(1)
    t1 = t_qx + _median_time(lambda: rtn_torch.w4a4_matmul(xq, xs, wq_c[:S1], ws_c[:S1]), reps=3) * (N / S1)
    c1_one = cpu_config1(1)
    c1_all = cpu_config1(threads)
    torch.set_num_threads(threads)
    try:
        cpu_model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except Exception:
        cpu_model = platform.processor()

    def ms(v):
        return round(v * 1e3, 3)

    return {
        "value": round(per_layer * 1e6, 1),
        "unit": "us/layer",
        "cores": threads,
        "kind": "port",
        "sample": f"L70 layer at M=1 (K={K}, N={N}): torch CPU rtn quant of x + dequant of {S} weight rows + "
                  f"fp32 matmul (oracle/rtn_torch.py, the reference's ops), {threads} threads, median of 5, "
                  f"scaled by N/{S}; per sample: quant {t_qx * 1e6:.0f} us, dequant {t_dw * 1e3:.1f} ms, "
                  f"matmul {t_mm * 1e3:.2f} ms; 1 thread: {t1 * 1e3:.0f} ms/layer ({S1}-row sample)",
        "config1": {
            "workload": "BASELINE config 1, full size: X fp16 16x4096 (1% channels x50), W fp16 4096x4096 "
                        "N(0,0.02), seed 0; median of 5 after a warm-up each",
            "threads": {str(threads): {"quant_x_ms": ms(c1_all[0]), "quant_w_ms": ms(c1_all[1]),
                                       "dequant_matmul_ms": ms(c1_all[2])},
                        "1": {"quant_x_ms": ms(c1_one[0]), "quant_w_ms": ms(c1_one[1]),
                              "dequant_matmul_ms": ms(c1_one[2])}},
        },
        "host": {"cpu_model": cpu_model, "os_cpu_count": os.cpu_count(), "torch_threads": threads},
    }


if __name__ == "__main__":
    main()
