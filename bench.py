#!/usr/bin/env python3
"""Benchmark of the MI355X FP8 quantized-linear path (one GPU).

Workloads (synthetic data, seeded host generator luisaml_amd.synth):
  * small-M decode linear (the headline line): x[M,4096] fp32 N(0,1) with
    M in {1,4,16}, dynamically QuantizeLinear'd to E4M3 per tensor, times a
    4096x11008 E4M3 weight (N(0,0.02), per-output-channel fp32 scales), bf16
    out.  One step = the three linears, each one lcml_fp8_gemm_dynamic call.
    Ten distinct copies of the packed weight (451 MB, 1.76x the 256 MB MALL)
    are rotated so that every launch streams its weights from HBM.
  * 8192^3 GEMM: A, B E4M3 quantised from N(0,1) with per-tensor scales
    (amax/448), fp32 accumulate, bf16 out, fused scalar dequant scale.
  * transformer-block linears (M = 4096), the ResNet 3x3 conv as an
    implicit-im2col GEMM, and the 3-layer W8A32 MLP, as sub-lines.
  * the CPU baseline: the oracle (the reference's arithmetic restated in C)
    on the host cores, on bounded samples of each workload.

Prints ONE JSON line.  `value` is the small-M whole-step throughput (GB/s of
algorithmic bytes with inputs resident in HBM); the 8192^3 GEMM TFLOP/s and
both roofline fractions ride along in the same line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

METRIC = "FP8 GEMM TFLOPS (% of MFMA peak) at 8192³; small-M linear GB/s (% HBM peak)"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
FP8_PEAK_TFLOPS = 5000.0       # dense FP8 MFMA
BF16_PEAK_TFLOPS = 2500.0      # dense bf16 MFMA (the exact kernel's instruction)
SMALL_K, SMALL_N, SMALL_MS = 4096, 11008, (1, 4, 16)
MEDIUM_MS = (32, 64, 128, 256)  # the same linear past decode sizes (a sub-benchmark, not the value)
BIG = 8192
N_WEIGHT_COPIES = 10


def channel_scales_np(w: np.ndarray, axis: int) -> np.ndarray:
    """Per-channel E4M3 scales amax/448 (1.0 when not a positive finite number)."""
    amax = np.max(np.abs(np.nan_to_num(w, nan=0.0)), axis=axis).astype(np.float32)
    s = (amax / np.float32(448.0)).astype(np.float32)
    bad = ~(s > 0) | ~np.isfinite(s)
    s[bad] = 1.0
    return s


def small_m_bytes(M: int) -> int:
    """Algorithmic HBM bytes of one small-M linear (quantize + GEMM):
    E4M3 weights + fp32 per-channel scales + fp32 activations in + bf16 out."""
    return SMALL_K * SMALL_N + 4 * SMALL_N + 4 * M * SMALL_K + 2 * M * SMALL_N


def gemm_kernel_bytes(M: int) -> int:
    """Algorithmic bytes of the small-M GEMM kernel alone (E4M3 activations in)."""
    return SMALL_K * SMALL_N + 4 * SMALL_N + M * SMALL_K + 2 * M * SMALL_N


def oracle_free_dynamic_scale(w: np.ndarray) -> np.float32:
    """Per-tensor E4M3 scale amax/448 (1.0 when not a positive finite number)."""
    s = np.float32(np.max(np.abs(np.nan_to_num(w, nan=0.0)))) / np.float32(448.0)
    return np.float32(s) if (s > 0 and np.isfinite(s)) else np.float32(1.0)


def cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, int(os.environ.get("OMP_NUM_THREADS", n))))


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-big", action="store_true", help="skip the 8192^3 GEMM")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run one plain 256 MiB device copy (profiler byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only (the kernels run on one GPU's share; there is no "
              "multi-GPU path); run with --gpus 1", file=sys.stderr)
        return 2

    import torch
    from luisaml_amd import capi, synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    out = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "e4m3",
           "data": "synthetic (seeded splitmix64 + Box-Muller, random-init weights)"}

    cpu_in = {}  # host copies of each workload's operands for the CPU leg

    # ------------------------------------------------------------ small-M --
    K, N = SMALL_K, SMALL_N
    w = synth.normal(101, (K, N), std=0.02)  # [K, N] (MatMul layout)
    sw = channel_scales_np(w, axis=0)
    d_sw = torch.from_numpy(sw).to(dev)
    qw = capi.quantize(torch.from_numpy(w).to(dev), d_sw, axis=1)
    packed = [capi.pack_weight(qw, w_is_nk=False)]
    for _ in range(N_WEIGHT_COPIES - 1):
        packed.append(packed[0].clone())
    del qw
    xs, qxs, sxs, ys = {}, {}, {}, {}
    for M in SMALL_MS:
        xs[M] = torch.from_numpy(synth.normal(200 + M, (M, K))).to(dev)
        qxs[M] = torch.empty((M, K), dtype=torch.uint8, device=dev)
        sxs[M] = torch.empty(1, dtype=torch.float32, device=dev)
        ys[M] = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    # workspace of the unfused path that AUTO takes for larger M*K
    wss = {M: torch.empty(max(256, capi.lib().lcml_fp8_gemm_dynamic_workspace_bytes(M, K, capi.KERNEL_AUTO)),
                          dtype=torch.uint8, device=dev) for M in SMALL_MS}

    def linear(M, copy):
        """One linear, one call: DynamicQuantizeLinear + DQ + Gemm (fused into
        one launch where that is cheaper, else quantize + GEMM)."""
        capi.gemm_dynamic(xs[M], packed[copy], d_sw, N, K, out=ys[M], kernel=capi.KERNEL_AUTO, workspace=wss[M])

    def linear_two_kernel(M, copy, gemm_only=False):
        """The same linear as two launches: dynamic quantize, then the GEMM."""
        if not gemm_only:
            capi.quantize_dynamic(xs[M], out=qxs[M], scale_out=sxs[M])
        capi.gemm(qxs[M], sxs[M], packed[copy], d_sw, N, K, out=ys[M], kernel=capi.KERNEL_AUTO)

    def step(i):
        for j, M in enumerate(SMALL_MS):
            linear(M, (3 * i + j) % N_WEIGHT_COPIES)

    def step_two_kernel(i, gemm_only=False):
        for j, M in enumerate(SMALL_MS):
            linear_two_kernel(M, (3 * i + j) % N_WEIGHT_COPIES, gemm_only)

    def capture(fn, n):
        """HIP graph of n calls of fn(i) on a side stream (kernels only, no memsets)."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(2):
                fn(i)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                fn(i)
        torch.cuda.synchronize()
        return g

    def timed(fn):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    def warm(fn, ms: float = 40.0):
        """Untimed repeats of fn for about `ms` of GPU time, so the sub-benchmarks
        below are timed at steady clocks rather than on the ramp."""
        t = timed(fn)
        for _ in range(max(1, min(200, int(ms / max(t, 1e-3))))):
            fn()
        torch.cuda.synchronize()

    # eager warmup, then the timed region: one replay of a graph holding
    # exactly `steps` steps (launch gaps of the Python/ctypes caller removed)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    g_steps = capture(step, args.steps)
    g_steps.replay()
    step_ms = timed(g_steps.replay) / args.steps
    eager_ms = timed(lambda: [step(i) for i in range(args.steps)]) / args.steps
    # the unfused composition (quantize kernel + GEMM kernel), and its GEMM alone
    g_two = capture(step_two_kernel, args.steps)
    g_two.replay()
    two_ms = timed(g_two.replay) / args.steps
    g_gemm = capture(lambda i: step_two_kernel(i, gemm_only=True), args.steps)
    g_gemm.replay()
    gemm_ms_total = timed(g_gemm.replay) / args.steps  # three GEMM launches per step
    bytes_step = sum(small_m_bytes(M) for M in SMALL_MS)
    # HBM bytes per launch of the GEMM kernel, from the committed counter runs
    # (FETCH_SIZE / WRITE_SIZE per dispatch, copy-calibrated); None if absent
    traffic_bytes, traffic_src = None, None
    tpath = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "skinny_gemm_small_m_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as fh:
            tj = json.load(fh)
        if tj.get("kernel_key") == "skinny_step":  # counters of the kernel launches this line reports
            traffic_bytes = tj["mean_hbm_bytes"]
            traffic_src = ("profiles/skinny_gemm_small_m_traffic.json (rocprofv3 FETCH_SIZE + WRITE_SIZE per "
                           "dispatch, copy-calibrated, mean over M)")
    value_gbs = bytes_step / (step_ms * 1e-3) / 1e9
    kbytes = sum(gemm_kernel_bytes(M) for M in SMALL_MS)
    k_gbs = kbytes / (gemm_ms_total * 1e-3) / 1e9
    # The dominant kernel is k_gemm_skinny: the fused-quantise instantiation
    # is the whole linear where AUTO fuses (fp32 activations in), the E4M3
    # instantiation after the quantise kernel elsewhere.  Per M, the average
    # duration of that kernel's launches (a graph holding only them).
    per_launch, kern_bytes, fused_m = {}, {}, {}
    for M in SMALL_MS:
        fused_m[M] = capi.lib().lcml_fp8_gemm_dynamic_workspace_bytes(M, K, capi.KERNEL_AUTO) == 0
        if fused_m[M]:
            fn, kern_bytes[str(M)] = (lambda i, M=M: linear(M, i % N_WEIGHT_COPIES)), small_m_bytes(M)
        else:
            fn, kern_bytes[str(M)] = ((lambda i, M=M: linear_two_kernel(M, i % N_WEIGHT_COPIES, gemm_only=True)),
                                      gemm_kernel_bytes(M))
        gm = capture(fn, 3 * args.steps)
        gm.replay()
        per_launch[str(M)] = round(1e3 * timed(gm.replay) / (3 * args.steps), 2)
        del gm
    kern_gbs = sum(kern_bytes.values()) / (sum(per_launch.values()) * 1e-6) / 1e9
    out.update({
        "value": round(value_gbs, 1), "unit": "GB/s", "ms_per_step": round(step_ms, 5),
        "ms_per_step_eager_launches": round(eager_ms, 5),
        "config": {"workload": "small-M FP8 linear: x[M,4096] fp32 -> dynamic per-tensor E4M3 -> "
                               "x W[4096,11008] E4M3 (per-channel scales) -> bf16, M in {1,4,16}, "
                               "one step = the three linears (lcml_fp8_gemm_dynamic each: one fused launch "
                               "for M*K <= 16384, else quantize + GEMM), timed as one HIP-graph replay",
                   "K": K, "N": N, "M": list(SMALL_MS), "weight_copies_rotated": N_WEIGHT_COPIES,
                   "bytes_per_step": bytes_step, "pct_hbm_peak": round(100 * value_gbs / HBM_PEAK_GBS, 1)},
        "roofline": {"bound": "hbm",
                     "kernel": "k_gemm_skinny, exact bf16-MFMA instantiation (fused dynamic quantisation at "
                               + ",".join(f"M={M}" for M in SMALL_MS if fused_m[M]) + ", E4M3 activations in "
                               "at " + ",".join(f"M={M}" for M in SMALL_MS if not fused_m[M]) + ")",
                     "achieved": round(kern_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kern_gbs / HBM_PEAK_GBS, 4), "traffic": traffic_bytes,
                     "traffic_source": traffic_src,
                     "bytes_per_launch": kern_bytes,
                     "bytes_per_launch_mean": round(sum(kern_bytes.values()) / len(kern_bytes)),
                     "avg_launch_us": per_launch},
        "two_kernel_composition": {
            "ms_per_step": round(two_ms, 5), "gbs": round(bytes_step / (two_ms * 1e-3) / 1e9, 1),
            "gemm_kernel_alone": {"kernel": "k_gemm_skinny (E4M3 activations in)",
                                  "avg_launch_us": round(1e3 * gemm_ms_total / 3, 2),
                                  "achieved_gbs": round(k_gbs, 1),
                                  "bytes_per_launch": {str(M): gemm_kernel_bytes(M) for M in SMALL_MS}}},
    })
    del g_steps, g_gemm, g_two

    # HBM read floor: a kernel that only reads the same packed weight bytes
    # (lcml_fp8_stream_read), rotated over the same copies, back to back in a
    # graph like the GEMM launches; best over a few grid sizes
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    floor = {}
    for wgs in (172, 256, 512, 768, 1024, 2048):
        gf = capture(lambda i, wgs=wgs: capi.stream_read(packed[i % N_WEIGHT_COPIES], sink, wgs), 3 * args.steps)
        gf.replay()
        floor[str(wgs)] = round(1e3 * timed(gf.replay) / (3 * args.steps), 2)
        del gf
    wbytes = packed[0].numel()
    best_wgs = min(floor, key=floor.get)
    out["read_floor"] = {
        "workload": f"read-only stream of one packed weight copy ({wbytes} B), {N_WEIGHT_COPIES} copies rotated, "
                    "graph of back-to-back launches; the best a kernel that only reads these bytes achieves",
        "avg_launch_us_by_workgroups": floor, "best_us": floor[best_wgs],
        "best_gbs": round(wbytes / (floor[best_wgs] * 1e-6) / 1e9, 1),
        "frac_hbm": round(wbytes / (floor[best_wgs] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "gemm_over_floor": {m: round(per_launch[m] / floor[best_wgs], 3) for m in per_launch}}

    # same-box yardstick: the vendor library (hipBLASLt through torch) on the
    # same small-M shape, E4M3 activations already quantised, per-tensor
    # scales, bf16 out, the same seven rotated weight copies
    lib_ref = {"note": "hipBLASLt via torch on this GPU: fp8 torch._scaled_mm (per-tensor scales, activations "
                       "already E4M3) and bf16 torch.matmul; a yardstick, not the reference implementation"}
    try:
        w8 = [torch.from_numpy(np.ascontiguousarray(w.T)).to(dev).to(torch.float8_e4m3fn)
              for _ in range(N_WEIGHT_COPIES)]  # [N, K]
        one = torch.ones((), dtype=torch.float32, device=dev)
        fp8_us = {}
        for M in SMALL_MS:
            x8 = xs[M].to(torch.float8_e4m3fn)
            gl = capture(lambda i, x8=x8: torch._scaled_mm(x8, w8[i % N_WEIGHT_COPIES].t(), scale_a=one,
                                                           scale_b=one, out_dtype=torch.bfloat16), 3 * args.steps)
            gl.replay()
            fp8_us[str(M)] = round(1e3 * timed(gl.replay) / (3 * args.steps), 2)
            del gl
        lib_ref["small_m_fp8_scaled_mm_us"] = fp8_us
        lib_ref["small_m_fp8_scaled_mm_gbs"] = {m: round(gemm_kernel_bytes(int(m)) / (t * 1e-6) / 1e9, 1)
                                                for m, t in fp8_us.items()}
        # medium M on the same linear: AUTO (the skinny kernel with 2 or 4
        # row blocks per workgroup, or 128x128 tiles) against the 256x256-
        # and 128x128-tile kernels and the library, E4M3 activations in, bf16
        # out
        med = {}
        for M in MEDIUM_MS:
            qx = capi.quantize(torch.from_numpy(synth.normal(400 + M, (M, K))).to(dev), one)
            x8 = qx.view(torch.float8_e4m3fn)
            yv = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            row = {}
            for name, kern in (("auto_us", capi.KERNEL_AUTO), ("tile_kernel_us", capi.KERNEL_MFMA),
                               ("tile128_kernel_us", capi.KERNEL_MFMA_128)):
                gm = capture(lambda i, kern=kern: capi.gemm(qx, one, packed[i % N_WEIGHT_COPIES], d_sw, N, K,
                                                             out=yv, kernel=kern), 3 * args.steps)
                warm(gm.replay, 20.0)  # the first kernel of a row would otherwise be timed on the clock ramp
                row[name] = round(1e3 * timed(gm.replay) / (3 * args.steps), 2)
                del gm
            gl = capture(lambda i: torch._scaled_mm(x8, w8[i % N_WEIGHT_COPIES].t(), scale_a=one, scale_b=one,
                                                    out_dtype=torch.bfloat16), 3 * args.steps)
            warm(gl.replay, 20.0)
            row["hipblaslt_fp8_us"] = round(1e3 * timed(gl.replay) / (3 * args.steps), 2)
            del gl
            row["auto_tflops"] = round(2.0 * M * K * N / (row["auto_us"] * 1e-6) / 1e12, 1)
            med[str(M)] = row
        out["medium_m"] = {"workload": f"x[M,{K}] E4M3 x W[{K},{N}] E4M3 (per-channel scales), bf16 out, "
                                       f"{N_WEIGHT_COPIES} weight copies rotated", **med}
        del w8
    except Exception as exc:  # an older torch without ROCm fp8 GEMM
        lib_ref["small_m_error"] = f"{type(exc).__name__}: {str(exc)[:120]}"
    out["library_reference"] = lib_ref

    # ------------------------------------------------------------ 8192^3 ---
    if not args.no_big:
        a = torch.from_numpy(synth.normal(301, (BIG, BIG))).to(dev)
        b = torch.from_numpy(synth.normal(302, (BIG, BIG))).to(dev)  # [K, N]
        qa, sa = capi.quantize_dynamic(a)
        qb, sb = capi.quantize_dynamic(b)
        # the standalone Q / DQ kernels on one 8192^2 operand (67.1M elements,
        # 5 algorithmic bytes each: fp32 one way, E4M3 the other)
        nq = BIG * BIG
        q_out = torch.empty_like(qa)
        ws_q = torch.empty(capi.DYNAMIC_WORKSPACE_BYTES, dtype=torch.uint8, device=dev)
        s_q = torch.empty(1, dtype=torch.float32, device=dev)
        qkern = {}
        for name, fn in (("quantize_static", lambda: capi.quantize(a, sa, out=q_out)),
                         ("quantize_dynamic", lambda: capi.quantize_dynamic(a, out=q_out, scale_out=s_q,
                                                                            workspace=ws_q)),
                         ("dequantize", lambda: capi.dequantize(qa, sa, out=b))):
            warm(fn)
            n = max(5, args.steps)
            ms = timed(lambda: [fn() for _ in range(n)]) / n
            gbs = 5.0 * nq / (ms * 1e-3) / 1e9
            qkern[name] = {"ms": round(ms, 4), "gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        qkern["quantize_dynamic"]["note"] = "two passes over x (amax partials, then encode): 9 B/elem moved"
        out["quantize_kernels_67m"] = {"workload": "8192x8192 fp32 N(0,1) <-> E4M3, per-tensor scale",
                                       "elements": nq, "bytes_per_element": 5, **qkern}
        del a, b, q_out
        bp = capi.pack_weight(qb, w_is_nk=False)
        del qb
        y = torch.empty((BIG, BIG), dtype=torch.bfloat16, device=dev)
        big = {}
        for name, kern, peak in (("exact_bf16_mfma", capi.KERNEL_MFMA, BF16_PEAK_TFLOPS),
                                 ("native_fp8_mfma", capi.KERNEL_MFMA_FP8, FP8_PEAK_TFLOPS)):
            warm(lambda: capi.gemm(qa, sa, bp, sb, BIG, BIG, out=y, kernel=kern))
            n = max(3, args.steps // 2)
            ms = timed(lambda: [capi.gemm(qa, sa, bp, sb, BIG, BIG, out=y, kernel=kern) for _ in range(n)]) / n
            tflops = 2.0 * BIG ** 3 / (ms * 1e-3) / 1e12
            big[name] = {"ms": round(ms, 4), "tflops": round(tflops, 1),
                         "pct_fp8_peak": round(100 * tflops / FP8_PEAK_TFLOPS, 1),
                         "pct_instruction_peak": round(100 * tflops / peak, 1)}
        try:
            ab = qa.view(torch.float8_e4m3fn).to(torch.bfloat16)
            bb = ab.t().contiguous()
            n = max(3, args.steps // 2)
            torch.matmul(ab, bb)
            ms_b = timed(lambda: [torch.matmul(ab, bb) for _ in range(n)]) / n
            a8, b8 = qa.view(torch.float8_e4m3fn), qa.view(torch.float8_e4m3fn).t().contiguous().t()
            one = torch.ones((), dtype=torch.float32, device=dev)
            torch._scaled_mm(a8, b8, scale_a=one, scale_b=one, out_dtype=torch.bfloat16)
            ms_8 = timed(lambda: [torch._scaled_mm(a8, b8, scale_a=one, scale_b=one, out_dtype=torch.bfloat16)
                                  for _ in range(n)]) / n
            out["library_reference"]["gemm_8192_bf16_matmul_tflops"] = round(2.0 * BIG ** 3 / (ms_b * 1e-3) / 1e12, 1)
            out["library_reference"]["gemm_8192_fp8_scaled_mm_tflops"] = round(2.0 * BIG ** 3 / (ms_8 * 1e-3) / 1e12, 1)
            del ab, bb, a8, b8
        except Exception as exc:
            out["library_reference"]["gemm_8192_error"] = f"{type(exc).__name__}: {str(exc)[:120]}"
        out["gemm_8192"] = {"workload": "8192^3 E4M3 x E4M3, per-tensor scales, fp32 accumulate, bf16 out",
                            "default_kernel": "exact_bf16_mfma",
                            "tile": "256x256, 2x2 wavefronts of 128x128 (one per SIMD), 5-stage LDS ring", **big,
                            "roofline": {"bound": "mfma", "achieved": big["exact_bf16_mfma"]["tflops"],
                                         "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                                         "frac": round(big["exact_bf16_mfma"]["tflops"] / FP8_PEAK_TFLOPS, 4)}}
        del qa, bp, y

    # ------------------------------------------ transformer-block linears ---
    if not args.no_big:
        # batch 8 x seq 512 (M = 4096), hidden 4096: QKV 4096->12288, O 4096->4096,
        # up 4096->11008 + GELU (fp32 out), down 11008->4096 on the GELU output;
        # every linear quantises its fp32 input per tensor (dynamic scale) and
        # adds an fp32 bias; weights N(0,0.02) with per-channel E4M3 scales.
        # The attention core is not part of this path: O-proj reads x.
        Mt, H = 4096, 4096
        shapes = {"qkv": (H, 3 * H), "o": (H, H), "up": (H, 11008), "down": (11008, H)}
        wts = {}
        cpu_in["transformer"] = {"x": synth.normal(420, (Mt, H)), "shapes": shapes, "w": {}}
        for i, (name, (kk, nn)) in enumerate(shapes.items()):
            wf = torch.from_numpy(synth.normal(400 + i, (kk, nn), std=0.02)).to(dev)
            sc = torch.from_numpy(channel_scales_np(wf.cpu().numpy(), axis=0)).to(dev)
            qd = capi.quantize(wf, sc, axis=1)
            bias_h = synth.normal(410 + i, (nn,), std=0.01)
            wts[name] = (capi.pack_weight(qd, w_is_nk=False), sc, torch.from_numpy(bias_h).to(dev))
            if not args.no_cpu:  # the same E4M3 codes and scales for the CPU leg
                cpu_in["transformer"]["w"][name] = (qd.cpu().numpy(), sc.cpu().numpy(), bias_h)
            del wf, qd
        xt = torch.from_numpy(cpu_in["transformer"]["x"]).to(dev)
        y_qkv = torch.empty((Mt, 3 * H), dtype=torch.bfloat16, device=dev)
        y_o = torch.empty((Mt, H), dtype=torch.bfloat16, device=dev)
        y_up = torch.empty((Mt, 11008), dtype=torch.float32, device=dev)
        y_dn = torch.empty((Mt, H), dtype=torch.bfloat16, device=dev)
        ws = torch.empty(capi.lib().lcml_fp8_gemm_dynamic_workspace_bytes(Mt, 11008, capi.KERNEL_MFMA),
                         dtype=torch.uint8, device=dev)
        flops_block = 2.0 * Mt * sum(kk * nn for kk, nn in shapes.values())

        up_part = capi.amax_parts_buffer(Mt, 11008, dev)

        def block(kern):
            def lin(x_in, name, y, act=capi.ACT_NONE, **kw):
                bp_, sc_, b_ = wts[name]
                kk, nn = shapes[name]
                return capi.gemm_dynamic_ex(x_in, bp_, sc_, nn, kk, c=b_, act=act, out=y, kernel=kern,
                                            workspace=ws, **kw)[1]
            lin(xt, "qkv", y_qkv)
            lin(xt, "o", y_o)
            # the up-projection's epilogue writes the partial maxima of its
            # GELU output, so the down-projection's quantisation needs no
            # amax pass over those 180 MB
            n_up = lin(xt, "up", y_up, act=capi.ACT_GELU_ERF, y_amax_part=up_part)
            lin(y_up, "down", y_dn, x_amax=(up_part, n_up))

        blk = {}
        for name, kern, peak in (("exact_bf16_mfma", capi.KERNEL_MFMA, BF16_PEAK_TFLOPS),
                                 ("native_fp8_mfma", capi.KERNEL_MFMA_FP8, FP8_PEAK_TFLOPS)):
            warm(lambda: block(kern))
            n = max(2, args.steps // 4)
            ms = timed(lambda: [block(kern) for _ in range(n)]) / n
            tf = flops_block / (ms * 1e-3) / 1e12
            blk[name] = {"ms": round(ms, 4), "tflops": round(tf, 1),
                         "pct_fp8_peak": round(100 * tf / FP8_PEAK_TFLOPS, 1),
                         "pct_instruction_peak": round(100 * tf / peak, 1)}
            # each linear on its own (quantisation of its input included; the
            # down-projection's scale from the up-projection's partials of
            # the last block above), so the block time splits by linear
            def lin1(which, kern=kern):
                bp_, sc_, b_ = wts[which]
                kk, nn = shapes[which]
                x_in, y, kw = {"qkv": (xt, y_qkv, {}), "o": (xt, y_o, {}),
                               "up": (xt, y_up, {"act": capi.ACT_GELU_ERF, "y_amax_part": up_part}),
                               "down": (y_up, y_dn, {"x_amax": (up_part, n_up_last[0])})}[which]
                capi.gemm_dynamic_ex(x_in, bp_, sc_, nn, kk, c=b_, out=y, kernel=kern, workspace=ws, **kw)
            n_up_last = [capi.gemm_dynamic_ex(xt, *wts["up"][:2], 11008, 4096, c=wts["up"][2], act=capi.ACT_GELU_ERF,
                                              out=y_up, kernel=kern, workspace=ws, y_amax_part=up_part)[1]]
            per = {}
            for which in ("qkv", "o", "up", "down"):
                per[which] = round(1e3 * timed(lambda: [lin1(which) for _ in range(n)]) / n, 1)
            blk[name]["per_linear_us"] = per
        out["transformer_linears_m4096"] = {
            "workload": "M=4096 (batch 8 x seq 512), hidden 4096: QKV 4096->12288, O 4096->4096, up 4096->11008 "
                        "+GELU, down 11008->4096; each linear = dynamic per-tensor quantize of its fp32 input + "
                        "FP8 GEMM with per-channel scales + fp32 bias (GELU on up); bf16 outputs except up (fp32, "
                        "re-quantised by down, whose scale comes from the partial maxima of |up| that the "
                        "up-projection's epilogue writes)", "flops": flops_block, **blk}
        del wts, xt, y_qkv, y_o, y_up, y_dn, ws

    # ------------------------------------------------------- conv as GEMM ---
    if not args.no_big:
        # ResNet-style 3x3 conv: x[32,256,56,56] fp32 N(0,1), dynamic per-tensor
        # E4M3 (written NHWC), W[256,256,3,3] N(0,0.03) per-output-channel
        # E4M3, stride 1, pad 1, bias + ReLU, NCHW fp32 out; the GEMM view is
        # M = 100352, K = 2304, N = 256 with the im2col done in the A loads
        cn, cc, ch, cw, cco = 32, 256, 56, 56, 256
        xc = torch.from_numpy(synth.normal(600, (cn, cc, ch, cw))).to(dev)
        wc = synth.normal(601, (cco, cc, 3, 3), std=0.03)
        wsc = channel_scales_np(wc.reshape(cco, -1), axis=1)
        d_wsc = torch.from_numpy(wsc).to(dev)
        qwc = capi.quantize(torch.from_numpy(wc.reshape(cco, -1)).to(dev), d_wsc, axis=0).reshape(cco, cc, 3, 3)
        bpc = capi.pack_conv_weight(qwc.contiguous())
        bc_h = synth.normal(602, (cco,), std=0.01)
        bc = torch.from_numpy(bc_h).to(dev)
        if not args.no_cpu:
            cpu_in["conv"] = {"x": xc.cpu().numpy(), "qw": qwc.cpu().numpy(), "sw": wsc, "bias": bc_h}
        xq = torch.empty((cn, ch, cw, cc), dtype=torch.uint8, device=dev)
        sxc = torch.empty(1, dtype=torch.float32, device=dev)
        wsq = torch.empty(256, dtype=torch.uint8, device=dev)
        yc = torch.empty((cn, cco, ch, cw), dtype=torch.float32, device=dev)
        conv_flops = 2.0 * cn * ch * cw * cco * cc * 9
        conv = {}

        def quant_c():
            capi.quantize_nhwc(xc, out=xq, scale_out=sxc, workspace=wsq)

        warm(quant_c)
        n = max(3, args.steps // 2)
        q_ms = timed(lambda: [quant_c() for _ in range(n)]) / n
        for name, kern, peak in (("exact_bf16_mfma", capi.KERNEL_MFMA, BF16_PEAK_TFLOPS),
                                 ("native_fp8_mfma", capi.KERNEL_MFMA_FP8, FP8_PEAK_TFLOPS)):
            def conv_c():
                capi.conv2d(xq, sxc, bpc, d_wsc, cco, (3, 3), pads=(1, 1), bias=bc, act=capi.ACT_RELU, out=yc,
                            kernel=kern)
            warm(conv_c)
            ms = timed(lambda: [conv_c() for _ in range(n)]) / n
            tf = conv_flops / (ms * 1e-3) / 1e12
            conv[name] = {"conv_ms": round(ms, 4), "tflops": round(tf, 1),
                          "pct_fp8_peak": round(100 * tf / FP8_PEAK_TFLOPS, 1),
                          "pct_instruction_peak": round(100 * tf / peak, 1),
                          "with_quantize_ms": round(ms + q_ms, 4)}
        in_bytes = cn * cc * ch * cw * 4
        out["conv3x3_resnet"] = {
            "workload": "x[32,256,56,56] fp32 -> dynamic E4M3 (NHWC) -> 3x3 conv pad 1 (implicit im2col GEMM "
                        "M=100352 K=2304 N=256, per-channel E4M3 weights) + bias + ReLU -> NCHW fp32",
            "flops": conv_flops, "quantize_nhwc_ms": round(q_ms, 4),
            "quantize_nhwc_gbs": round((in_bytes + in_bytes // 4) / (q_ms * 1e-3) / 1e9, 1), **conv}
        del xc, xq, yc, bpc

    # ---------------------------------------------------------- 3-layer MLP ---
    # 784->256 (+ReLU) -> 128 (+ReLU) -> 10, batch 64, fp32 activations, E4M3
    # weights with one per-tensor scale each through DequantizeLinear (W8A32)
    mlp = []
    cpu_in["mlp"] = {"x": synth.uniform(520, (64, 784)), "layers": []}
    for i, (kk, nn) in enumerate(((784, 256), (256, 128), (128, 10))):
        wf = synth.normal(500 + i, (nn, kk), std=0.05)  # Gemm transB=1 layout
        sc = np.array([oracle_free_dynamic_scale(wf)], np.float32)
        d_sc = torch.from_numpy(sc).to(dev)
        q = capi.quantize(torch.from_numpy(wf).to(dev), d_sc)
        b_h = synth.normal(510 + i, (nn,), std=0.01)
        mlp.append((capi.pack_weight(q, w_is_nk=True), d_sc, torch.from_numpy(b_h).to(dev), kk, nn))
        cpu_in["mlp"]["layers"].append((q.cpu().numpy(), sc, b_h))
    x_mlp = torch.from_numpy(cpu_in["mlp"]["x"]).to(dev)
    bufs = [torch.empty((64, nn), dtype=torch.float32, device=dev) for (_, _, _, _, nn) in mlp]

    def mlp_fwd(_i=0):
        h = x_mlp
        for j, (bp_, sc_, b_, kk, nn) in enumerate(mlp):
            capi.gemm_w8a32(h, bp_, sc_, nn, kk, c=b_, act=capi.ACT_RELU if j < 2 else capi.ACT_NONE, out=bufs[j])
            h = bufs[j]

    mlp_fwd()
    g_mlp = capture(mlp_fwd, 50)
    g_mlp.replay()
    mlp_us = 1e3 * timed(g_mlp.replay) / 50
    out["mlp_784_256_128_10"] = {"workload": "3-layer MLP batch 64, W8A32 (DequantizeLinear weights, fp32 "
                                             "activations), bias + ReLU fused, HIP-graph replay",
                                 "us_per_forward": round(mlp_us, 2), "flops": 2 * 64 * (784 * 256 + 256 * 128 + 128 * 10)}
    del g_mlp

    if args.calib_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        out["calib_copy_bytes"] = 256 << 20

    # --------------------------------------------------------- CPU leg -----
    if not args.no_cpu:
        import oracle  # the CPU restatement of the reference arithmetic (baseline only)
        nt = cpu_threads()
        oracle.set_threads(nt)
        wq = oracle.quantize(w, sw, axis=1)
        t = time.perf_counter()
        reps = 0
        while True:
            for M in SMALL_MS:
                x = synth.normal(200 + M, (M, K))
                s = oracle.dynamic_scale(x)
                oracle.qlinear(oracle.quantize(x, s), s, wq, sw)
            reps += 1
            if time.perf_counter() - t > 8.0 or reps >= 5:
                break
        cpu_s = (time.perf_counter() - t) / reps
        out["cpu_baseline"] = {"value": round(bytes_step / cpu_s / 1e9, 3), "unit": "GB/s", "cores": nt,
                               "kind": "port",
                               "sample": f"{reps} full steps of the small-M workload (M=1,4,16) through the "
                                         "oracle: dynamic quantize, dequantize, fp32 fma-chain Gemm "
                                         "(gemm.cpp:155-162 order), OpenMP over output tiles"}
        if not args.no_big:
            rows = 64
            a = synth.normal(301, (BIG, BIG))[:rows]
            b = synth.normal(302, (BIG, BIG))
            qa_c = oracle.quantize(a, oracle.dynamic_scale(a))
            sb_c = oracle.dynamic_scale(b)
            qb_c = oracle.quantize(b, sb_c)
            t = time.perf_counter()
            oracle.qlinear(qa_c, 1.0, qb_c, sb_c)
            dt = time.perf_counter() - t
            out["cpu_baseline"]["gemm_8192_sample"] = {
                "gflops": round(2.0 * rows * BIG * BIG / dt / 1e9, 2), "cores": nt,
                "sample": f"{rows} rows of the 8192^3 GEMM (dequantize + fma-chain Gemm)"}

        cpu_workloads(out["cpu_baseline"], cpu_in, nt)

    print(json.dumps(out), flush=True)
    return 0


def cpu_workloads(cb: dict, cpu_in: dict, nt: int) -> None:
    """The oracle (the reference arithmetic: dequantise, then fp32 fma-chain
    Gemm / direct conv, gemm.cpp:155-162, conv.cpp:143-192) on bounded samples
    of the MLP, transformer-linear and conv workloads, on the same operands
    the GPU ran (E4M3 codes and scales copied back from the device)."""
    import oracle
    if "mlp" in cpu_in:  # the whole forward pass, batch 64
        m = cpu_in["mlp"]
        layers = [(oracle.dequantize(q, sc), b) for q, sc, b in m["layers"]]
        reps, t = 0, time.perf_counter()
        while reps < 200 and time.perf_counter() - t < 2.0:
            h = m["x"]
            for j, (wd, b) in enumerate(layers):
                h = oracle.gemm(h, wd, b, transB=1, act=oracle.ACT_RELU if j < 2 else oracle.ACT_NONE)
            reps += 1
        us = 1e6 * (time.perf_counter() - t) / reps
        cb["mlp_784_256_128_10"] = {"us_per_forward": round(us, 1), "cores": nt,
                                    "gflops": round(2 * 64 * (784 * 256 + 256 * 128 + 128 * 10) / us / 1e3, 2),
                                    "sample": f"{reps} full forward passes (batch 64, W8A32: fp32 activations, "
                                              "dequantised E4M3 weights, bias + ReLU)"}
    if "transformer" in cpu_in:  # 256 rows of each linear
        tr, rows = cpu_in["transformer"], 256
        x = tr["x"]
        flops, t = 0.0, time.perf_counter()
        sx = oracle.dynamic_scale(x)  # amax over the whole activation, as the GPU does
        h_in = {"qkv": x, "o": x, "up": x}
        for name in ("qkv", "o", "up", "down"):
            qw, sw, b = tr["w"][name]
            kk, nn = tr["shapes"][name]
            xin = h_in[name][:rows]
            s = sx if name != "down" else oracle.dynamic_scale(xin)  # down: scale of the sampled GELU rows
            y, _, _ = oracle.qlinear(oracle.quantize(xin, s), s, qw, sw, bias=b,
                                     act=oracle.ACT_GELU_ERF if name == "up" else oracle.ACT_NONE)
            if name == "up":
                h_in["down"] = y.astype(np.float32)
            flops += 2.0 * rows * kk * nn
        dt = time.perf_counter() - t
        cb["transformer_linears_m4096_sample"] = {
            "gflops": round(flops / dt / 1e9, 2), "seconds": round(dt, 2), "cores": nt,
            "sample": f"{rows} of the 4096 rows of each linear (QKV, O, up+GELU, down): dynamic quantise "
                      "(amax over the whole input; for down over the sampled GELU rows), dequantise, "
                      "fma-chain Gemm + bias"}
    if "conv" in cpu_in:  # 4 images of the batch of 32
        c, imgs = cpu_in["conv"], 4
        t = time.perf_counter()
        s = oracle.dynamic_scale(c["x"])
        xi = c["x"][:imgs]
        A = oracle.dequantize(oracle.quantize(xi, s), s)
        W = oracle.dequantize(c["qw"].reshape(c["qw"].shape[0], -1), c["sw"], axis=0).reshape(c["qw"].shape)
        oracle.conv2d(A, W, c["bias"], pads=(1, 1), act=oracle.ACT_RELU)
        dt = time.perf_counter() - t
        f = 2.0 * imgs * 56 * 56 * 256 * 256 * 9
        cb["conv3x3_resnet_sample"] = {
            "gflops": round(f / dt / 1e9, 2), "seconds": round(dt, 2), "cores": nt,
            "sample": f"{imgs} of the 32 images: dynamic quantise (amax over the batch), dequantise, direct conv "
                      "(reference loop order kh, kw, channel) + bias + ReLU"}


if __name__ == "__main__":
    sys.exit(main())
