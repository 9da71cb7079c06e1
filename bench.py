#!/usr/bin/env python3
"""Benchmark of the MI355X hot path for sile's tile kernels, on one GPU.

Measures the BASELINE metric: bf16 GEMM and causal flash-attention forward in
TFLOP/s (fraction of MI355X dense MFMA peak) and fp16 row softmax in GB/s
(fraction of HBM peak).  All inputs are synthetic, drawn from the seeded
recipes of the configurations, and resident in HBM before timing starts.

The JSON line's `value` is the bf16 GEMM M=N=K=8192 throughput (the metric's
first quantity and the workload named in `config.workload`); every other
measured kernel is listed under `components` with its own roofline.  A step is
one launch of the kernel; the K timed steps run back to back between two HIP
events recorded on the launch stream, bracketed by a device synchronisation on
both sides, after an untimed clock-settle period and the W warmup steps.

`cpu_baseline` times the CPU oracle (a restatement of sile's CPU backend loop
nest, compiled like the reference's generated C) on the whole bf16 8192^3 GEMM
on this host's cores; each component carries its own `cpu_baseline` on a
bounded sample of its workload (whole softmax and 4096^3 GEMM, every 8th row
tile of the fp8 GEMM, four whole heads of each attention workload).

Each MFMA workload also carries `same_kernel_on_zero_inputs`: the same launch
timed again after its inputs are zero-filled.  The chip is power-limited under
random data (its engine clock falls from 2.4 GHz to ~1.8 GHz), and all-zero
operands do not toggle the matrix-core datapath, so the ratio of that rate to
`value` is the clock the workload loses to the power limit.  It never replaces
`value`.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME ...]
                       [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from sile_amd import _abi as hip  # noqa: E402

METRIC = ("bf16 GEMM & flash-attn fwd TFLOP/s (% MI355X MFMA peak), softmax GB/s, 1 GPU")

# Published MI355X peaks (dense): bf16/fp16 MFMA 2.5 PFLOP/s, fp8 5.0 PFLOP/s, HBM3E 8 TB/s.
PEAK_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "fp8": 5000.0}
PEAK_HBM_GBS = 8000.0
# fp32 VALU lane rate (the published 157.3 TFLOP/s counts an FMA as 2 flops); an
# exact-order GEMM issues one instruction per flop
PEAK_VALU_F32_TOPS = 78.6
PEAK_F32_PUBLISHED_TFLOPS = 157.3
SETTLE_S = 0.5  # untimed load before each workload's warmup (clock ramp-up)

PROFILE_TRAFFIC = os.path.join(ROOT, "profiles", "traffic.json")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- input recipes

def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits with round-to-nearest-even (numpy, no oracle)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def normal(seed, shape, scale=1.0):
    g = np.random.default_rng(seed)
    out = np.empty(shape, np.float32)
    flat = out.reshape(-1)
    step = 1 << 24
    for i in range(0, flat.size, step):
        flat[i:i + step] = g.standard_normal(min(step, flat.size - i), dtype=np.float32)
    if scale != 1.0:
        out *= np.float32(scale)
    return out


def gemm_inputs(kind, m, n=None, k=None):
    """Host operands of the GEMM configurations at M x N x K (M = N = K = m
    when n and k are not given): (a_bits [M, K], b_bits [N, K] (B
    column-major), scale_a, scale_b, a_type).
    bf16: A, B ~ N(0, 1)/sqrt(K), seeds 4 / 5, rounded to bf16 (RNE).
    fp8: A, B ~ N(0, 1), seeds 9 / 10, quantised per tensor to e4m3fn with
    s = amax / 448, q = rne_sat(x / s)."""
    n = m if n is None else n
    k = m if k is None else k
    if kind == "fp8":
        # the oracle's encoder is the configuration's quantiser (input recipe,
        # not timed work)
        from oracle import cpuref
        a = normal(9, (m, k))
        b = normal(10, (n, k))
        sa = float(np.float32(np.abs(a).max() / 448.0))
        sb = float(np.float32(np.abs(b).max() / 448.0))
        return cpuref.e4m3_encode(a, sa), cpuref.e4m3_encode(b, sb), sa, sb, hip.F8E4M3
    a_bits = bf16_bits(normal(4, (m, k), 1 / np.sqrt(k)))
    b_bits = bf16_bits(normal(5, (n, k), 1 / np.sqrt(k)))
    return a_bits, b_bits, 1.0, 1.0, hip.BF16


ATTN_SHAPE = (4, 32, 128)  # batch, heads, head_dim of the attention configuration


def attention_inputs(s, b=ATTN_SHAPE[0], h=ATTN_SHAPE[1], d=ATTN_SHAPE[2]):
    """Q, K, V [B, H, S, D] fp16 ~ N(0, 1), seeds 6 / 7 / 8."""
    return [normal(seed, (b, h, s, d)).astype(np.float16) for seed in (6, 7, 8)]


def softmax_input(rows=8192, cols=8192):
    """x [rows, cols] fp16 ~ N(0, 4) (sigma 2), seed 3."""
    return normal(3, (rows, cols), 2.0).astype(np.float16)


# ---------------------------------------------------------------- timing

def time_launches(launch, steps, warmup, stream, rotate=1):
    """Runs `launch(i)` warmup + steps times on `stream`; returns the duration
    in ms of the timed region, measured with HIP events recorded on `stream`
    before the first and after the last timed launch.  The launches run
    back to back, so region / steps is the kernel's average launch duration
    (events around every launch would add their own overhead to a 50 us
    kernel).  The timed region is bracketed by a device synchronisation on
    both sides.

    Before the warmup launches the workload runs untimed for SETTLE_S
    seconds: after the seconds of host-side input generation the GPU starts
    at idle clocks and takes a few hundred ms of load to reach its steady
    clock (5 warmup launches of the 8192^3 GEMM under-report it by ~8%)."""
    t0 = time.perf_counter()
    i = 0
    while time.perf_counter() - t0 < SETTLE_S:
        for _ in range(8):
            launch(i % rotate)
            i += 1
        hip.synchronize()
    for i in range(warmup):
        launch(i % rotate)
    hip.synchronize()
    r0, r1 = hip.Event(), hip.Event()
    r0.record(stream)
    for i in range(steps):
        launch(i % rotate)
    r1.record(stream)
    hip.synchronize()
    region_ms = r0.elapsed_ms(r1)
    r0.close()
    r1.close()
    return region_ms


def summarise(name, work, unit_scale, unit, region_ms, steps, bound, peak, traffic):
    """value: work per step over the timed region; roofline.achieved: the
    algorithmic work of one launch over the average launch duration (the same
    quantity here, since a step is one launch)."""
    per_step = region_ms / steps
    value = work / (per_step * 1e-3) / unit_scale
    return {
        "name": name, "value": round(value, 2), "unit": unit, "ms_per_step": round(per_step, 4),
        "roofline": roofline_obj(bound, value, peak, unit, traffic),
    }


def load_traffic():
    if os.path.exists(PROFILE_TRAFFIC):
        with open(PROFILE_TRAFFIC) as f:
            return json.load(f)
    return {}


ZERO_STEPS = 10  # launches timed again on all-zero inputs (MFMA workloads)


def zero_input_rate(launch, inputs, work, peak, steps, stream):
    """The same launch, timed again after its input buffers are filled with
    zeros: with nothing toggling the matrix-core datapath the power-managed
    engine clock stays near its 2.4 GHz peak, so this rate over `value` is
    the clock the chip gives up under the random-data workload.  Reported
    beside `value`, never in its place."""
    for buf in inputs:
        buf.fill_bytes(0)
    n = min(steps, ZERO_STEPS)
    region = time_launches(launch, n, 2, stream)
    v = work / (region / n * 1e-3) / 1e12
    return {"value": round(v, 2), "unit": "TFLOP/s", "frac_of_peak": round(v / peak, 4),
            "ms_per_step": round(region / n, 4),
            "note": "same kernel and launch on all-zero inputs (output not checked); "
                    "the ratio to value is the engine-clock loss under random data"}


def roofline_obj(bound, achieved, peak, unit, traffic):
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


# ---------------------------------------------------------------- workloads

def bench_gemm(name, kind, m, n, k, steps, warmup, stream, traffic, cpu_tile_step=0,
               b_row=False):
    """cpu_tile_step > 0 also times the CPU oracle on every cpu_tile_step-th
    256-row tile of C over the same (de)quantised inputs (the whole GEMM when
    M is below one tile).  The roofline is the matrix cores' unless streaming
    A, B and C once at the HBM peak takes longer (skinny shapes): then it is
    the algorithmic bytes over the step time, in GB/s.  b_row: the same B
    given row-major [K, N] (the canonical matmul's own layout)."""
    log(f"[bench] {name}: generating inputs")
    a_bits, b_bits, sa, sb, t = gemm_inputs(kind, m, n, k)
    if b_row:
        b_bits = np.ascontiguousarray(b_bits.T)
    c_t = hip.BF16
    da, db = hip.DeviceBuffer.from_array(a_bits), hip.DeviceBuffer.from_array(b_bits)
    host = (a_bits, b_bits) if cpu_tile_step else None
    del a_bits, b_bits
    dc = hip.DeviceBuffer(m * n * 2)

    def launch(_):
        hip.gemm(t, t, c_t, m, n, k, da.ptr, k, hip.ROW_MAJOR, db.ptr, n if b_row else k,
                 hip.ROW_MAJOR if b_row else hip.COL_MAJOR, dc.ptr, n, sa, sb, 0, stream)

    log(f"[bench] {name}: timing {steps} steps")
    region = time_launches(launch, steps, warmup, stream)
    flop = 2.0 * m * n * k
    eb = 1 if kind == "fp8" else 2
    nbytes = float(eb * (m * k + n * k) + 2 * m * n)
    res = summarise(name, flop, 1e12, "TFLOP/s", region, steps, "mfma", PEAK_TFLOPS[kind],
                    traffic.get(name))
    res["flop_per_launch"] = flop
    if nbytes / (PEAK_HBM_GBS * 1e9) > flop / (PEAK_TFLOPS[kind] * 1e12):
        gbs = nbytes / (res["ms_per_step"] * 1e-3) / 1e9
        res["roofline"] = roofline_obj("hbm", gbs, PEAK_HBM_GBS, "GB/s", traffic.get(name))
        res["bytes_per_launch"] = nbytes
    else:
        res["same_kernel_on_zero_inputs"] = zero_input_rate(launch, (da, db), flop,
                                                            PEAK_TFLOPS[kind], steps, stream)
    for buf in (da, db, dc):
        buf.close()
    if host is not None:
        from oracle import cpuref
        if b_row:
            host = (host[0], np.ascontiguousarray(host[1].T))
        if kind == "fp8":
            a32, b32 = cpuref.e4m3_decode(host[0], sa), cpuref.e4m3_decode(host[1], sb)
            what = "dequantised fp32 inputs q*s"
        else:
            a32, b32 = cpuref.f32_from_bf16(host[0]), cpuref.f32_from_bf16(host[1])
            what = "up-cast fp32 inputs"
        del host
        c32 = np.zeros((m, n), np.float32)
        if m < 256:
            cpu_tile_step = 1
        rows = m if m < 256 else ((m // 256 + cpu_tile_step - 1) // cpu_tile_step) * 256
        log(f"[bench] {name}: cpu oracle on {rows} of {m} rows")
        res["cpu_baseline"] = cpu_timed(
            lambda: cpuref.gemm_nt(a32, b32, bm=min(256, m), row_tile_step=cpu_tile_step, out=c32),
            2.0 * rows * n * k, 1e12, "TFLOP/s",
            (f"every {cpu_tile_step}th 256-row tile of C ({rows} of {m} rows, all columns, full K)"
             if cpu_tile_step > 1 else "the whole GEMM")
            + f" on {what}; canonical-matmul loop nest, gcc -O2 -fopenmp",
            full_work=2.0 * m * n * k)
    return res


def bench_attention(name, s, steps, warmup, stream, traffic, cpu_heads=0, d=ATTN_SHAPE[2],
                    dt="f16", causal=True):
    """cpu_heads > 0 also times the CPU oracle on the first cpu_heads (b, h)
    slices, every query row, causal (fp16 causal lines only).  dt "bf16"
    rounds the same N(0, 1) inputs to bf16; causal False attends to every
    key."""
    b, h = ATTN_SHAPE[:2]
    if dt != "f16" or not causal:
        cpu_heads = 0
    log(f"[bench] {name}: generating inputs")
    bufs, host = [], []
    if dt == "bf16":
        xs = [bf16_bits(normal(seed, (b, h, s, d))) for seed in (6, 7, 8)]
    else:
        xs = attention_inputs(s, d=d)
    for x in xs:
        bufs.append(hip.DeviceBuffer.from_array(x.view(np.uint16)))
        if cpu_heads:
            host.append(x.reshape(b * h, s, d)[:cpu_heads].astype(np.float32))
        del x
    del xs
    do = hip.DeviceBuffer(b * h * s * d * 2)
    scale = 1.0 / np.sqrt(d)

    t = hip.BF16 if dt == "bf16" else hip.F16

    def launch(_):
        hip.flash_attn_fwd(t, b, h, s, d, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, do.ptr,
                           scale, causal, stream)

    log(f"[bench] {name}: timing {steps} steps")
    region = time_launches(launch, steps, warmup, stream)
    # unmasked (query, key) pairs only: 2 products x 2 flop x D per pair
    flop = 4.0 * d * b * h * (s * (s + 1) / 2 if causal else s * s)
    res = summarise(name, flop, 1e12, "TFLOP/s", region, steps, "mfma", PEAK_TFLOPS["f16"],
                    traffic.get(name))
    res["flop_per_launch"] = flop
    res["flop_convention"] = ("4*D*B*H*S*(S+1)/2 (causal pairs only)" if causal
                              else "4*D*B*H*S*S (every pair)")
    res["same_kernel_on_zero_inputs"] = zero_input_rate(launch, bufs, flop, PEAK_TFLOPS["f16"],
                                                        steps, stream)
    for buf in bufs + [do]:
        buf.close()
    if cpu_heads:
        from oracle import cpuref
        o32 = np.zeros((s, d), np.float32)

        def run():
            for i in range(cpu_heads):
                cpuref.attention_fwd(host[0][i], host[1][i], host[2][i], scale, causal=True,
                                     out=o32)

        log(f"[bench] {name}: cpu oracle on {cpu_heads} of {b * h} heads")
        res["cpu_baseline"] = cpu_timed(
            run, flop * cpu_heads / (b * h), 1e12, "TFLOP/s",
            f"{cpu_heads} of {b * h} (batch, head) slices, every query row, causal, on up-cast "
            "fp32 Q/K/V; naive fp32 restatement (scores, max, expf, sum, P.V), gcc -O2 -fopenmp",
            full_work=flop)
    return res


def bench_softmax(name, steps, warmup, stream, traffic, cpu=False):
    rows = cols = 8192
    log(f"[bench] {name}: generating inputs")
    x = softmax_input(rows, cols)
    # 4 input/output pairs = 1 GiB, four times the 256 MiB Infinity Cache, so
    # every timed launch reads its input from HBM
    rotate = 4
    xs = [hip.DeviceBuffer.from_array(x.view(np.uint16)) for _ in range(rotate)]
    ys = [hip.DeviceBuffer(rows * cols * 2) for _ in range(rotate)]
    x32 = x.astype(np.float32) if cpu else None
    del x

    def launch(i):
        hip.softmax_rows(hip.F16, hip.F16, rows, cols, xs[i].ptr, cols, ys[i].ptr, cols, stream)

    def copy(i):
        hip.copy_rows(rows, cols * 2, xs[i].ptr, cols * 2, ys[i].ptr, cols * 2, stream)

    log(f"[bench] {name}: timing {steps} steps")
    region = time_launches(launch, steps, warmup, stream, rotate=rotate)
    nbytes = 4.0 * rows * cols  # read 2 B + write 2 B per element
    res = summarise(name, nbytes, 1e9, "GB/s", region, steps, "hbm", PEAK_HBM_GBS,
                    traffic.get(name))
    res["bytes_per_launch"] = nbytes
    # the ceiling of this traffic on this box: the same bytes copied by
    # sile_hip_copy_rows (contiguous rows: sile_copy_flat_b128, the fastest
    # copy shape measured on the device, 16-byte non-temporal accesses and no
    # arithmetic) over the same rotating buffers
    log(f"[bench] {name}: timing the copy ceiling ({steps} steps)")
    copy_ms = time_launches(copy, steps, warmup, stream, rotate=rotate) / steps
    ceiling = nbytes / (copy_ms * 1e-3) / 1e9
    res["copy_ceiling"] = {"kernel": "sile_copy_flat_b128", "value": round(ceiling, 2),
                           "unit": "GB/s", "ms_per_step": round(copy_ms, 4),
                           "frac_of_peak": round(ceiling / PEAK_HBM_GBS, 4)}
    res["frac_of_copy_ceiling"] = round(res["value"] / ceiling, 4)
    # each direction of that traffic alone, at the same bytes per launch
    # (256 MiB, over four rotating buffers of their own): the write-only
    # stream (a splat stored to [2 rows, cols] f16, sile_hip_fill_rows) and
    # the read-only stream (the row max of what it wrote, sile_hip_reduce_rows,
    # on the softmax's row shape: one 8192-element row per 512-thread
    # workgroup)
    zs = [hip.DeviceBuffer(int(nbytes)) for _ in range(rotate)]
    outs = [hip.DeviceBuffer(2 * rows * 4) for _ in range(rotate)]
    streams = {}
    for kind, fn, kernel in (
            ("write_stream", lambda i: hip.fill_rows(hip.F16, 2 * rows, cols, 0.5, zs[i].ptr,
                                                     cols, stream),
             "sile_fill_flat_b128"),
            ("read_stream", lambda i: hip.reduce_rows(hip.REDUCE_MAX, hip.F16, 2 * rows, cols,
                                                      zs[i].ptr, cols, outs[i].ptr, stream),
             "sile_reduce_rows_f16_b512")):
        log(f"[bench] {name}: timing the {kind.replace('_', ' ')} ({steps} steps)")
        ms = time_launches(fn, steps, warmup, stream, rotate=rotate) / steps
        rate = nbytes / (ms * 1e-3) / 1e9
        streams[kind] = rate
        res[kind] = {"kernel": kernel, "value": round(rate, 2), "unit": "GB/s",
                     "bytes_per_launch": nbytes, "ms_per_step": round(ms, 4),
                     "frac_of_peak": round(rate / PEAK_HBM_GBS, 4)}
    res["frac_of_best_stream"] = round(res["value"] / max(ceiling, *streams.values()), 4)
    for buf in xs + ys + zs + outs:
        buf.close()
    if x32 is not None:
        from oracle import cpuref
        log(f"[bench] {name}: cpu oracle on the whole matrix")
        res["cpu_baseline"] = cpu_timed(
            lambda: cpuref.softmax_rows(x32), nbytes, 1e9, "GB/s",
            "the whole [8192, 8192] softmax on up-cast fp32 input, rated by the fp16 "
            "workload's algorithmic bytes (4 per element); sequential max / expf / sum / "
            "divide per row, gcc -O2 -fopenmp")
    return res


# vec_add<TILE=4> (crates/sile/tests/backend_vec_add.rs:3-9) in the printed
# LLIR form (crates/sile-llvm-ir/src/print.rs:6-57)
LLIR_VEC_ADD4 = """\
; vec_add<TILE=4> (crates/sile/examples/vec_add.rs:3-13) written by hand in the
; printed LLIR form of crates/sile-llvm-ir/src/print.rs: c[4 pid + i] = a[..] + b[..]
define void @vec_add(ptr addrspace(1) %a, ptr addrspace(1) %b, ptr addrspace(1) %c, ptr addrspace(4) %__sile_shapes) {
  ; sile.param %a [rank=1, shape_offset=0, elem=f32]
  ; sile.param %b [rank=1, shape_offset=1, elem=f32]
  ; sile.param %c [rank=1, shape_offset=2, elem=f32]
  ; sile.param %__sile_shapes [elem=i64]
bb0:
  %pid = call i32 @llvm.nvvm.ctaid.x()
  %base = mul %pid, 4
  br label %vec_add_header ; args(0)
vec_add_header:
  ; args(%i: i64)
  %cond = icmp slt %i, 4
  br i1 %cond, label %vec_add_body, label %vec_add_exit
vec_add_body:
  %idx = add %base, %i
  %pa = getelementptr f32, ptr addrspace(1) %a, i64 %idx
  %va = load f32, ptr addrspace(1) %pa
  %pb = getelementptr f32, ptr addrspace(1) %b, i64 %idx
  %vb = load f32, ptr addrspace(1) %pb
  %sum = fadd %va, %vb
  %pc = getelementptr f32, ptr addrspace(1) %c, i64 %idx
  store f32 %sum, ptr addrspace(1) %pc
  %next = add %i, 1
  br label %vec_add_header ; args(%next)
vec_add_exit:
  ret void
}
"""


def bench_llir_vec_add(name, steps, warmup):
    """vec_add<TILE=4> generated from LLIR (LLIR_VEC_ADD4) by
    sile_hip_llir_compile and run through sile_hip_launch_llir, which is
    synchronous like the reference's apply(): each step is one whole call
    (table upload, launch, wait).  c = a + b over 64M fp32 elements, 12 bytes
    of HBM traffic per element."""
    n = 64 << 20
    kern = hip.LlirKernel(LLIR_VEC_ADD4, (2, 1, 4))
    a = hip.DeviceBuffer(n * 4)
    b = hip.DeviceBuffer(n * 4)
    c = hip.DeviceBuffer(n * 4)
    a.fill_bytes(0)
    b.fill_bytes(0)
    ptrs, shapes, grid = [a.ptr, b.ptr, c.ptr], [n, n, n], (n // 4, 1, 1)
    for _ in range(warmup):
        kern(ptrs, shapes, grid)
    t0 = time.perf_counter()
    for _ in range(steps):
        kern(ptrs, shapes, grid)
    dt = (time.perf_counter() - t0) / steps
    nbytes = 12.0 * n
    res = summarise(name, nbytes, 1e9, "GB/s", dt * 1e3 * steps, steps, "hbm", PEAK_HBM_GBS, None)
    res["bytes_per_launch"] = nbytes
    for buf in (a, b, c):
        buf.close()
    kern.close()
    return res


# softmax<BM=4, BN=8192> (crates/sile/examples/softmax.rs:3-16) in the printed
# LLIR form (crates/sile-llvm-ir/src/print.rs:6-57), as the generic code
# generation gets it when the pattern router is not used: its three column
# loops (8192 iterations) are spread over a 1024-lane workgroup per program
LLIR_SOFTMAX_4x8192 = """\
define void @softmax(ptr addrspace(1) %x, ptr addrspace(1) %y, ptr addrspace(4) %__sile_shapes) {
  ; sile.param %x [rank=2, shape_offset=0, elem=f32]
  ; sile.param %y [rank=2, shape_offset=2, elem=f32]
  ; sile.param %__sile_shapes [elem=i64]
bb0:
  %__shape_x = getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 0
  %ldx_p = getelementptr i64, ptr addrspace(4) %__shape_x, i64 1
  %ldx = load i64, ptr addrspace(4) %ldx_p
  %__shape_y = getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 2
  %ldy_p = getelementptr i64, ptr addrspace(4) %__shape_y, i64 1
  %ldy = load i64, ptr addrspace(4) %ldy_p
  %m = call i32 @llvm.nvvm.ctaid.x()
  %row0 = mul %m, 4
  %tile = alloca [4 x [8192 x f32]], addrspace(5)
  br label %sm_row_header ; args(0)
sm_row_header:
  ; args(%r: i64)
  %rc = icmp slt %r, 4
  br i1 %rc, label %sm_row_body, label %sm_exit
sm_row_body:
  %row = add %row0, %r
  %xrow = mul %row, %ldx
  %x0p = getelementptr f32, ptr addrspace(1) %x, i64 %xrow
  %x0 = load f32, ptr addrspace(1) %x0p
  br label %sm_max_header ; args(1, %x0)
sm_max_header:
  ; args(%c: i64, %mx: f32)
  %mc = icmp slt %c, 8192
  br i1 %mc, label %sm_max_body, label %sm_exp_header ; false_args(0, 0.0)
sm_max_body:
  %xi = add %xrow, %c
  %xp = getelementptr f32, ptr addrspace(1) %x, i64 %xi
  %xv = load f32, ptr addrspace(1) %xp
  %gt = fcmp ogt %xv, %mx
  %mx_next = select i1 %gt, f32 %xv, f32 %mx
  %c_next = add %c, 1
  br label %sm_max_header ; args(%c_next, %mx_next)
sm_exp_header:
  ; args(%e: i64, %sum: f32)
  %ec = icmp slt %e, 8192
  br i1 %ec, label %sm_exp_body, label %sm_div_header ; false_args(0)
sm_exp_body:
  %xe = add %xrow, %e
  %xep = getelementptr f32, ptr addrspace(1) %x, i64 %xe
  %xev = load f32, ptr addrspace(1) %xep
  %d = fsub %xev, %mx
  %ex = call f32 @llvm.exp.f32(f32 %d)
  %tp = getelementptr [4 x [8192 x f32]], ptr addrspace(5) %tile, i64 %r, i64 %e
  store f32 %ex, ptr addrspace(5) %tp
  %sum_next = fadd %sum, %ex
  %e_next = add %e, 1
  br label %sm_exp_header ; args(%e_next, %sum_next)
sm_div_header:
  ; args(%q: i64)
  %qc = icmp slt %q, 8192
  br i1 %qc, label %sm_div_body, label %sm_row_latch
sm_div_body:
  %tq = getelementptr [4 x [8192 x f32]], ptr addrspace(5) %tile, i64 %r, i64 %q
  %tv = load f32, ptr addrspace(5) %tq
  %yv = fdiv %tv, %sum
  %yrow = mul %row, %ldy
  %yi = add %yrow, %q
  %yp = getelementptr f32, ptr addrspace(1) %y, i64 %yi
  store f32 %yv, ptr addrspace(1) %yp [writeonly]
  %q_next = add %q, 1
  br label %sm_div_header ; args(%q_next)
sm_row_latch:
  %r_next = add %r, 1
  br label %sm_row_header ; args(%r_next)
sm_exit:
  ret void
}
"""


def bench_llir_softmax(name, steps, warmup, text=None):
    """softmax<BM=4, BN=8192> over f32 [8192, 8192] generated from LLIR
    (LLIR_SOFTMAX_4x8192, or `text`), one workgroup per program, through the
    synchronous sile_hip_launch_llir (table upload, launch, wait per call),
    rated by the routed softmax's algorithmic bytes (8 per element: read x,
    write y)."""
    rows = cols = 8192
    kern = hip.LlirKernel(text or LLIR_SOFTMAX_4x8192, (1, 4, cols))
    x = hip.DeviceBuffer.from_array(normal(3, (rows, cols), 2.0))
    y = hip.DeviceBuffer(rows * cols * 4)
    ptrs, shapes, grid = [x.ptr, y.ptr], [rows, cols, rows, cols], (rows // 4, 1, 1)
    for _ in range(warmup):
        kern(ptrs, shapes, grid)
    t0 = time.perf_counter()
    for _ in range(steps):
        kern(ptrs, shapes, grid)
    dt = (time.perf_counter() - t0) / steps
    nbytes = 8.0 * rows * cols
    res = summarise(name, nbytes, 1e9, "GB/s", dt * 1e3 * steps, steps, "hbm", PEAK_HBM_GBS, None)
    res["bytes_per_launch"] = nbytes
    x.close()
    y.close()
    kern.close()
    return res


def llir_matmul_inputs(size):
    """The generated matmul lines' A and B: seeded N(0, 1) f32 [size, size]."""
    return normal(4, (size, size), 1.0), normal(5, (size, size), 1.0)


def bench_llir_matmul(name, steps, warmup, size=2048, tile=64, bk=8, gen="matmul"):
    """A matmul program's LLIR (tests/llir_shapes.py) at M = N = K = size
    with tile x tile cells a program: `matmul` is the canonical matmul
    (canonical_matmul.rs:24-444), the row x column nest with each cell's k
    loop; `mma_k_loop` the K-tile loop of tile loads and the tile MMA nest
    (mma.rs:25-260) carrying its accumulator tile.  The nests spread over a
    1024-lane workgroup, each cell's sum serial on its lane (the reference's
    order, bit-exact), through the synchronous sile_hip_launch_llir; 2 M N K
    flops per call, against the VALU rate without FMA (the order forbids
    contraction)."""
    from tests import llir_shapes
    kern = hip.LlirKernel(getattr(llir_shapes, gen)(tile, tile, bk), (2, tile, tile))
    ha, hb = llir_matmul_inputs(size)
    a = hip.DeviceBuffer.from_array(ha)
    b = hip.DeviceBuffer.from_array(hb)
    c = hip.DeviceBuffer(size * size * 4)
    ptrs, shapes = [a.ptr, b.ptr, c.ptr], [size] * 6
    grid = ((size // tile) ** 2, 1, 1)
    for _ in range(warmup):
        kern(ptrs, shapes, grid)
    t0 = time.perf_counter()
    for _ in range(steps):
        kern(ptrs, shapes, grid)
    dt = (time.perf_counter() - t0) / steps
    res = summarise(name, 2.0 * size ** 3, 1e12, "TFLOP/s", dt * 1e3 * steps, steps, "valu",
                    PEAK_VALU_F32_TOPS, None)
    form = "canonical matmul" if gen == "matmul" else "K-tile MMA loop"
    res["note"] = (f"{form}<{tile}, {tile}, {bk}> LLIR, f32, one 1024-lane workgroup "
                   "a program, bit-identical to the reference's order")
    for buf in (a, b, c):
        buf.close()
    kern.close()
    return res


# softmax<BM=4, BN=8192> (crates/sile/examples/softmax.rs:3-16) in the
# printed Tile IR form (crates/sile-tile-ir/src/print.rs:5-354) after the
# default passes, the text a Rust HipBackend hands to sile_hip_tile_ir_route
TILE_IR_SOFTMAX_4x8192 = """\
module {
  entry @softmax(
    %0 {sym_name = "x", rank = 2} : tile<ptr<f32>>,
    %1 {sym_name = "y", rank = 2} : tile<ptr<f32>>,
    %2 {sym_name = "__shape_x", kind = "shape.desc", source = %0} : shape_desc<2>,
    %3 {sym_name = "__launch_idx0", kind = "launch.index", dim = 0} : tile<i64>,
    %4 {sym_name = "__launch_idx1", kind = "launch.index", dim = 1} : tile<i64>,
    %12 {sym_name = "__shape_y", kind = "shape.desc", source = %1} : shape_desc<2>
  ) {
    ^bb0:  // entry
      %5 = load_ptr_tko %0, [%3, %4] {shape = [4, 8192], stride_dim = 1} : tile<4x8192xf32>
      %6 = reduce %5 {axis = 1, combiner = "max", input_shape = [4, 8192]} : tile<4x1xf32>
      %9 = map exp(subf(%5, broadcast(%6, src_shape=[4, 1]))) {shape = [4, 8192]} : tile<4x8192xf32>
      %10 = reduce %9 {axis = 1, combiner = "sum", input_shape = [4, 8192]} : tile<4x1xf32>
      %13 = map divf(%9, broadcast(%10, src_shape=[4, 1])) {shape = [4, 8192]} : tile<4x8192xf32>
      %14 = store_ptr_tko %1, %13, [%3, %4] {shape = [4, 8192], stride_dim = 1} : none
      return
  }
}
"""


def bench_tile_ir_softmax(name, steps, warmup):
    """softmax<BM=4, BN=8192> over f32 [8192, 8192] given as printed Tile IR:
    routed once by sile_hip_tile_ir_route (to the row softmax kernel), then
    each step is one synchronous sile_hip_tile_ir_launch, like the reference's
    apply().  8 bytes of HBM traffic per element (read 4, write 4); two
    input/output pairs (1 GiB) rotate so every call reads from HBM."""
    rows = cols = 8192
    bm = 4
    text = TILE_IR_SOFTMAX_4x8192
    shapes, programs = [rows, cols, rows, cols], rows // bm
    route = hip.tile_ir_route(text, shapes, programs)
    if route.kind != hip.ROUTE_SOFTMAX_ROWS:
        raise RuntimeError(f"softmax routed to {route.name}: {route.reason}")
    log(f"[bench] {name}: generating inputs")
    x = normal(3, (rows, cols), 2.0)
    rotate = 2
    xs = [hip.DeviceBuffer.from_array(x) for _ in range(rotate)]
    ys = [hip.DeviceBuffer(rows * cols * 4) for _ in range(rotate)]
    del x

    def call(i):
        hip.tile_ir_launch(route, [xs[i].ptr, ys[i].ptr], shapes, programs)

    for i in range(warmup):
        call(i % rotate)
    t0 = time.perf_counter()
    for i in range(steps):
        call(i % rotate)
    dt = (time.perf_counter() - t0) / steps
    nbytes = 8.0 * rows * cols
    res = summarise(name, nbytes, 1e9, "GB/s", dt * 1e3 * steps, steps, "hbm", PEAK_HBM_GBS, None)
    res["bytes_per_launch"] = nbytes
    res["route"] = route.name
    for buf in xs + ys:
        buf.close()
    return res


def bench_reduce_rows(name, steps, warmup, stream):
    """Row max and row sum over fp32 [8192, 8192] (the reference's reduce and
    its fused load + vec4 sum, bit-identical): sile_hip_reduce_rows (max) and
    sile_hip_reduce_rows_fused_sum, each launch reading 256 MiB from HBM (two
    inputs rotate, 512 MiB, past the 256 MiB Infinity Cache).  `value` is the
    row sum's rate; the max is listed beside it."""
    rows = cols = 8192
    log(f"[bench] {name}: generating inputs")
    x = normal(3, (rows, cols), 2.0)
    rotate = 2
    xs = [hip.DeviceBuffer.from_array(x) for _ in range(rotate)]
    del x
    out = hip.DeviceBuffer(rows * 4)
    nbytes = 4.0 * rows * cols + 4.0 * rows

    def row_sum(i):
        hip.reduce_rows_fused_sum(rows, cols, xs[i].ptr, cols, rows * cols, out.ptr, stream)

    def row_max(i):
        hip.reduce_rows(hip.REDUCE_MAX, hip.F32, rows, cols, xs[i].ptr, cols, out.ptr, stream)

    log(f"[bench] {name}: timing {steps} steps")
    region = time_launches(row_sum, steps, warmup, stream, rotate=rotate)
    res = summarise(name, nbytes, 1e9, "GB/s", region, steps, "hbm", PEAK_HBM_GBS, None)
    res["bytes_per_launch"] = nbytes
    mx = time_launches(row_max, steps, warmup, stream, rotate=rotate) / steps
    res["row_max"] = {"value": round(nbytes / (mx * 1e-3) / 1e9, 2), "unit": "GB/s",
                      "ms_per_step": round(mx, 4),
                      "frac_of_peak": round(nbytes / (mx * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    for buf in xs + [out]:
        buf.close()
    return res


def bench_matvec(name, steps, warmup, stream, traffic, bk=32):
    """The matvec program of crates/sile/examples/mlp.rs:26-44 over fp32
    x [8192, 8192], y [8192] (BK = 32, bit-identical to the CPU backend):
    sile_hip_matvec_f32, each launch reading x's 256 MiB from HBM (two inputs
    rotate, 512 MiB, past the 256 MiB Infinity Cache).  Bytes per launch:
    x, y and the output."""
    rows = cols = 8192
    log(f"[bench] {name}: generating inputs")
    x = normal(11, (rows, cols), 1.0)
    y = normal(12, (cols,), 1.0)
    rotate = 2
    xs = [hip.DeviceBuffer.from_array(x) for _ in range(rotate)]
    del x
    dy = hip.DeviceBuffer.from_array(y)
    out = hip.DeviceBuffer(rows * 4)
    nbytes = 4.0 * rows * cols + 4.0 * cols + 4.0 * rows

    def launch(i):
        hip.matvec_f32(rows, cols, bk, xs[i].ptr, cols, dy.ptr, out.ptr, 0.0, stream)

    log(f"[bench] {name}: timing {steps} steps")
    region = time_launches(launch, steps, warmup, stream, rotate=rotate)
    res = summarise(name, nbytes, 1e9, "GB/s", region, steps, "hbm", PEAK_HBM_GBS,
                    traffic.get(name))
    res["bytes_per_launch"] = nbytes
    res["note"] = (f"matvec<BM, BK={bk}> (mlp.rs) over f32 x [{rows}, {cols}], y [{cols}], "
                   "in the reference's order (bit-identical)")
    for buf in xs + [dy, out]:
        buf.close()
    return res


def bench_parallel_reduce(name, steps, warmup):
    """The reference's parallel_reduce (crates/sile/examples/parallel_reduce.rs: one atomic add of
    each program's fused vec4 tile sum into out[0]) over 64M fp32 elements,
    TILE = 4096 (16384 programs), through the synchronous DSL entry point
    sile_hip_kernel_parallel_reduce, like apply(); 256 MiB read per call."""
    n, tile = 1 << 26, 4096
    programs = n // tile
    log(f"[bench] {name}: generating inputs")
    a = normal(1, (n,), 1.0)
    da = hip.DeviceBuffer.from_array(a)
    del a
    dout = hip.DeviceBuffer.from_array(np.zeros(1, np.float32))

    def call():
        hip.kernel_parallel_reduce([da.ptr, dout.ptr], programs, [n, 1], tile)

    for _ in range(warmup):
        call()
    t0 = time.perf_counter()
    for _ in range(steps):
        call()
    dt = (time.perf_counter() - t0) / steps
    nbytes = 4.0 * n
    res = summarise(name, nbytes, 1e9, "GB/s", dt * 1e3 * steps, steps, "hbm", PEAK_HBM_GBS, None)
    res["bytes_per_launch"] = nbytes
    res["note"] = "synchronous calls timed on the host clock (launch and wait per call)"
    for buf in (da, dout):
        buf.close()
    return res


def bench_gemm_f32_exact(name, size, steps, warmup, stream, traffic, cpu=False):
    """fp32 GEMM M=N=K=size in the reference's canonical per-cell order
    (bit-identical to its CPU backend), A and B row-major U(-1,1) (seeds 1/2,
    the recipe of BASELINE config 1).  Every flop is its own instruction (the
    product and the sum are rounded separately), so the bound is the VALU's
    lane rate: 256 CUs x 128 lanes x 2.4 GHz = 78.6 T instructions/s."""
    n = size
    a = np.random.default_rng(1).uniform(-1, 1, size=(n, n)).astype(np.float32)
    b = np.random.default_rng(2).uniform(-1, 1, size=(n, n)).astype(np.float32)
    da, db = hip.DeviceBuffer.from_array(a), hip.DeviceBuffer.from_array(b)
    dc = hip.DeviceBuffer(n * n * 4)
    host = (a, b) if cpu else None
    del a, b

    def launch(i):
        hip.gemm(hip.F32, hip.F32, hip.F32, n, n, n, da.ptr, n, hip.ROW_MAJOR, db.ptr, n,
                 hip.ROW_MAJOR, dc.ptr, n, 1.0, 1.0, 0, stream)

    log(f"[bench] {name}: timing {steps} steps")
    region = time_launches(launch, steps, warmup, stream)
    flop = 2.0 * n ** 3
    res = summarise(name, flop, 1e12, "TFLOP/s", region, steps, "valu", PEAK_VALU_F32_TOPS,
                    traffic.get(name))
    # the same rate against the published fp32 peak (which counts an FMA as 2
    # flops; the reference's order forbids FMA, so 0.5 is this path's ceiling)
    res["frac_of_published_fp32_peak"] = round(res["value"] / PEAK_F32_PUBLISHED_TFLOPS, 4)
    res["flop_per_launch"] = flop
    for buf in (da, db, dc):
        buf.close()
    if host is not None:
        from oracle import cpuref
        c32 = np.zeros((n, n), np.float32)
        grid = (n // 32 * (n // 32), 1, 1)
        log(f"[bench] {name}: cpu oracle, sile_kernel_matmul<32, 32, 32>")
        res["cpu_baseline"] = cpu_timed(
            lambda: cpuref.kernel_matmul(host[0], host[1], c32, grid, 32, 32, 32), flop, 1e12,
            "TFLOP/s", f"the whole {n}^3 GEMM as sile_kernel_matmul with 32x32x32 tiles "
            "(the reference's program loop and per-cell order), gcc -O2 -fopenmp")
    return res


def bench_copy_calibration(name, steps, warmup):
    """A plain device-to-device copy of COPY_BYTES (the HIP runtime's blit
    kernel behind sile_hip_memcpy_dtod).  Run under rocprofv3 --pmc it gives
    the FETCH_SIZE / WRITE_SIZE that a kernel moving exactly COPY_BYTES each
    way reports, the scale used to turn the other kernels' counters into
    bytes."""
    src, dst = hip.DeviceBuffer(COPY_BYTES), hip.DeviceBuffer(COPY_BYTES)
    src.fill_bytes(1)
    for _ in range(warmup):
        hip.call("sile_hip_memcpy_dtod", dst.ptr, src.ptr, COPY_BYTES)
    hip.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        hip.call("sile_hip_memcpy_dtod", dst.ptr, src.ptr, COPY_BYTES)
    hip.synchronize()
    dt = (time.perf_counter() - t0) / steps
    src.close()
    dst.close()
    return {"name": name, "value": round(2 * COPY_BYTES / dt / 1e9, 1), "unit": "GB/s",
            "ms_per_step": round(dt * 1e3, 4), "bytes_each_way": COPY_BYTES}


COPY_BYTES = 512 << 20
# (batch, head) slices of the attention workloads the CPU oracle runs in full
CPU_ATTN_HEADS = 4


def cpu_baseline(row_tile_step=1):
    """CPU oracle on a deterministic sample of the bf16 GEMM 8192^3 workload:
    every `row_tile_step`-th 256-row tile of C (all 8192 columns, full K),
    inputs up-cast from the same bf16 data."""
    from oracle import cpuref

    m = n = k = 8192
    log("[bench] cpu baseline: generating inputs")
    a = cpuref.f32_from_bf16(bf16_bits(normal(4, (m, k), 1 / np.sqrt(k))))
    b = cpuref.f32_from_bf16(bf16_bits(normal(5, (n, k), 1 / np.sqrt(k))))
    c = np.zeros((m, n), np.float32)
    tiles = (m // 256 + row_tile_step - 1) // row_tile_step
    rows = tiles * 256
    log(f"[bench] cpu baseline: {rows} rows x {n} cols x {k} k on {cpuref.num_threads()} threads")
    t0 = time.perf_counter()
    cpuref.gemm_nt(a, b, bm=256, row_tile_step=row_tile_step, out=c)
    dt = time.perf_counter() - t0
    flop = 2.0 * rows * n * k
    return {
        "value": round(flop / dt / 1e12, 6), "unit": "TFLOP/s", "cores": cpuref.num_threads(),
        "kind": "port",
        "sample": ((f"every {row_tile_step}th 256-row tile of C ({rows} of {m} rows, all "
                    "columns, full K)" if row_tile_step > 1 else "the whole GEMM")
                   + f" of bf16 GEMM 8192^3 on up-cast fp32 inputs: {flop:.3e} flop in {dt:.2f} s;"
                   " oracle = canonical-matmul loop nest (sequential fp32 mul-then-add per cell),"
                   " gcc -O2 -fopenmp"),
        "seconds": round(dt, 3),
        **({"extrapolated_full_seconds": round(dt * m / rows, 3),
            "extrapolated_note": "extrapolated, not measured: the sample's time scaled by "
                                 "the whole GEMM's rows over the sample's"}
           if rows < m else {}),
    }


def cpu_timed(run, work, unit_scale, unit, sample, min_s=1.0, full_work=None):
    """Times `run()` (a CPU oracle call on this host's cores), repeated until
    at least `min_s` seconds have passed; returns a cpu_baseline object whose
    value is `work` (the algorithmic work of one run, in the GPU workload's
    own unit) per second of one run.  For a sample of the workload,
    `full_work` (the whole workload's work) adds the time the whole workload
    would take at the sample's rate, labelled as extrapolated."""
    from oracle import cpuref

    reps, t0 = 0, time.perf_counter()
    while True:
        run()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_s:
            break
    per = dt / reps
    out = {"value": round(work / per / unit_scale, 6), "unit": unit,
           "cores": cpuref.num_threads(), "kind": "port",
           "sample": f"{sample}; {reps} run(s), {per:.3f} s each", "seconds": round(dt, 3)}
    if full_work is not None and full_work > work:
        out["extrapolated_full_seconds"] = round(per * full_work / work, 3)
        out["extrapolated_note"] = ("extrapolated, not measured: one run's time scaled by the "
                                    "whole workload's work over the sample's")
    return out


# ---------------------------------------------------------------- PMC traffic

def traffic_from_pmc(root):
    """Builds profiles/traffic.json from rocprofv3 --pmc runs of this script,
    one per workload and counter: ROOT/pmc_fetch_<name>/ (FETCH_SIZE) and
    ROOT/pmc_write_<name>/ (WRITE_SIZE), <name> being a workload of ALL or
    EXTRA (those without both runs are left out).  The mean per-dispatch KiB of the workload's kernel is
    scaled by what the same counter reads for the copy calibration (COPY_BYTES
    each way): bytes = KiB * COPY_BYTES / copy_KiB.  Only the dispatches of
    the random-data run count: those after the inputs are zero-filled for
    `same_kernel_on_zero_inputs` (a runtime fill dispatch after the workload's
    first) run at another clock and fetch differently through the L2."""
    import csv
    import glob

    def mean_kib(d, counter, want):
        vals = []
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(path) as f:
                rows = [r for r in csv.DictReader(f) if r.get("Counter_Name") == counter]
            first = min((int(r["Dispatch_Id"]) for r in rows if want(r["Kernel_Name"])), default=0)
            cut = min((int(r["Dispatch_Id"]) for r in rows
                       if "fillBuffer" in r["Kernel_Name"] and int(r["Dispatch_Id"]) > first),
                      default=None)
            vals += [float(r["Counter_Value"]) for r in rows
                     if want(r["Kernel_Name"]) and (cut is None or int(r["Dispatch_Id"]) < cut)]
        return sum(vals) / len(vals) if vals else None

    def is_copy(k):
        return "copyBuffer" in k

    cf = mean_kib(os.path.join(root, "pmc_fetch_copy_calibration"), "FETCH_SIZE", is_copy)
    cw = mean_kib(os.path.join(root, "pmc_write_copy_calibration"), "WRITE_SIZE", is_copy)
    if not cf or not cw:
        raise SystemExit("no copy-calibration dispatches found under " + root)
    sf, sw = COPY_BYTES / (cf * 1024), COPY_BYTES / (cw * 1024)
    out = {"_scale": {"fetch": round(sf, 4), "write": round(sw, 4), "copy_bytes": COPY_BYTES,
                      "copy_fetch_kib": round(cf, 1), "copy_write_kib": round(cw, 1)}}
    for name in ALL + EXTRA:
        prefix = WORKLOAD_KERNEL.get(name, "sile_")

        def is_sile(k):
            return k.startswith(prefix)
        f = mean_kib(os.path.join(root, "pmc_fetch_" + name), "FETCH_SIZE", is_sile)
        w = mean_kib(os.path.join(root, "pmc_write_" + name), "WRITE_SIZE", is_sile)
        if f is not None and w is not None:
            out[name] = round(f * 1024 * sf + w * 1024 * sw)
    return out


# the kernel a workload's line is about (the softmax workload also runs the copy
# that measures its ceiling)
WORKLOAD_KERNEL = {"softmax_f16_8192": "sile_softmax_rows", "gemm_bf16_8192": "sile_gemm_nt",
                   "gemm_bf16_8192_brow": "sile_gemm_nn", "gemm_fp8_8192_brow": "sile_gemm_nt",
                   "gemm_bf16_4096": "sile_gemm_nt", "gemm_fp8_8192": "sile_gemm_nt",
                   "flash_attn_fwd_f16_s8192": "sile_flash_attn", "flash_attn_fwd_f16_s4096":
                   "sile_flash_attn", "gemm_f32_exact_4096": "sile_gemm_f32_exact",
                   "gemm_f32_exact_512": "sile_gemm_f32_exact",
                   "flash_attn_fwd_f16_s8000": "sile_flash_attn",
                   "flash_attn_fwd_f16_s8192_d64": "sile_flash_attn",
                   "matvec_f32_8192": "sile_dsl_matvec", "matvec_f32_8192_bk8": "sile_dsl_matvec",
                   "llir_softmax_f32_8192": "sile_kernel_softmax",
                   "llir_softmax_ref_shapes_f32_8192": "sile_kernel_softmax",
                   "llir_matmul_f32_2048": "sile_kernel_matmul",
                   "llir_mma_k_loop_f32_2048": "sile_kernel_mma_k_loop",
                   "tile_ir_softmax_f32_8192": "sile_softmax_rows"}

ALL = ["gemm_bf16_8192", "gemm_bf16_4096", "gemm_fp8_8192", "flash_attn_fwd_f16_s8192",
       "flash_attn_fwd_f16_s4096", "softmax_f16_8192"]
EXTRA = ["copy_calibration", "llir_vec_add", "llir_softmax_f32_8192", "llir_softmax_ref_shapes_f32_8192",
         "llir_matmul_f32_2048", "llir_mma_k_loop_f32_2048",
         "tile_ir_softmax_f32_8192",
         "gemm_f32_exact_4096",
         "gemm_f32_exact_512", "reduce_rows_f32_8192", "parallel_reduce_f32",
         # the mlp example's matvec program (BK 32; _bk8: the example's BK)
         "matvec_f32_8192", "matvec_f32_8192_bk8",
         # shapes off the headline configurations: 128 x 128 tiles, split K', the
         # transposed form (M x N x K)
         "gemm_bf16_2048x2048x2048", "gemm_bf16_128x8192x8192", "gemm_bf16_8192x64x8192",
         "gemm_fp8_256x8192x8192",
         # causal attention at an S that is not a multiple of the query block,
         # and at head_dim 64
         "flash_attn_fwd_f16_s8000", "flash_attn_fwd_f16_s8192_d64",
         # bf16 inputs, and every (query, key) pair (not causal)
         "flash_attn_fwd_bf16_s8192", "flash_attn_fwd_f16_s8192_nc",
         # B row-major [K, N], the canonical matmul's own layout
         "gemm_bf16_8192_brow", "gemm_fp8_8192_brow"]


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", nargs="*", default=None, choices=ALL + EXTRA)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--traffic-from", metavar="PMC_ROOT",
                    help="write profiles/traffic.json from rocprofv3 --pmc runs and exit")
    args = ap.parse_args()
    if args.traffic_from:
        t = traffic_from_pmc(args.traffic_from)
        os.makedirs(os.path.dirname(PROFILE_TRAFFIC), exist_ok=True)
        with open(PROFILE_TRAFFIC, "w") as f:
            json.dump(t, f, indent=1, sort_keys=True)
        print(json.dumps(t))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path, so --gpus N "
              "with N > 1 is not supported (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    hip.init(0)
    info = hip.device_info(0)
    log(f"[bench] device {info['name']} {info['gcn_arch']} CUs={info['compute_units']} "
        f"clock={info['clock_khz'] / 1e3:.0f} MHz")
    stream = hip.Stream()
    traffic = load_traffic()
    names = args.only or ALL
    cpu = not args.no_cpu_baseline
    results = {}
    for name in names:
        if name == "copy_calibration":
            results[name] = bench_copy_calibration(name, args.steps, args.warmup)
        elif name == "llir_vec_add":
            results[name] = bench_llir_vec_add(name, args.steps, args.warmup)
        elif name == "llir_softmax_f32_8192":
            results[name] = bench_llir_softmax(name, args.steps, args.warmup)
        elif name == "llir_matmul_f32_2048":
            results[name] = bench_llir_matmul(name, args.steps, args.warmup)
        elif name == "llir_mma_k_loop_f32_2048":
            results[name] = bench_llir_matmul(name, args.steps, args.warmup, bk=16, gen="mma_k_loop")
        elif name == "llir_softmax_ref_shapes_f32_8192":
            # the same program in the reference's loop shapes: a loop nest and
            # a private tile per op (tests/llir_shapes.py)
            from tests import llir_shapes
            results[name] = bench_llir_softmax(name, args.steps, args.warmup,
                                               llir_shapes.softmax(4, 8192))
        elif name == "tile_ir_softmax_f32_8192":
            results[name] = bench_tile_ir_softmax(name, args.steps, args.warmup)
        elif name == "reduce_rows_f32_8192":
            results[name] = bench_reduce_rows(name, args.steps, args.warmup, stream)
        elif name == "parallel_reduce_f32":
            results[name] = bench_parallel_reduce(name, args.steps, args.warmup)
        elif name.startswith("matvec_f32_8192"):
            bk = int(name.split("_bk")[-1]) if "_bk" in name else 32
            results[name] = bench_matvec(name, args.steps, args.warmup, stream, traffic, bk=bk)
        elif name.startswith("gemm_f32_exact_"):
            size = int(name.split("_")[-1])
            results[name] = bench_gemm_f32_exact(name, size, args.steps, args.warmup, stream,
                                                 traffic, cpu=cpu and size <= 1024)
        elif name.startswith("gemm_"):
            kind = "fp8" if "fp8" in name else "bf16"
            b_row = name.endswith("_brow")
            dims = name.removesuffix("_brow").split("_")[-1]
            m, n, k = map(int, dims.split("x")) if "x" in dims else (int(dims),) * 3
            # the bf16 8192^3 GEMM's CPU time is the headline cpu_baseline below
            step = (0 if not cpu or name == "gemm_bf16_8192"
                    else 8 if 2.0 * m * n * k > 2e11 else 1)
            results[name] = bench_gemm(name, kind, m, n, k, args.steps, args.warmup, stream,
                                       traffic, cpu_tile_step=step, b_row=b_row)
        elif name.startswith("flash_attn"):
            # flash_attn_fwd_<f16|bf16>_s<S>[_d<D>][_nc] (_nc: not causal)
            causal = not name.endswith("_nc")
            tail = name.removesuffix("_nc").split("_s")[-1]
            s_len, d = (map(int, tail.split("_d")) if "_d" in tail else (int(tail), ATTN_SHAPE[2]))
            results[name] = bench_attention(name, s_len, args.steps, args.warmup, stream, traffic,
                                            cpu_heads=CPU_ATTN_HEADS if cpu else 0, d=d,
                                            dt="bf16" if "_bf16_" in name else "f16",
                                            causal=causal)
        else:
            results[name] = bench_softmax(name, args.steps, args.warmup, stream, traffic,
                                          cpu=cpu)
        r = results[name]
        frac = r.get("roofline", {}).get("frac")
        log(f"[bench] {name}: {r['value']} {r['unit']} ({r['ms_per_step']} ms/step"
            + (f", {100 * frac:.1f}% of peak)" if frac is not None else ")"))
        z = r.get("same_kernel_on_zero_inputs")
        if z:
            log(f"[bench] {name}: same kernel on all-zero inputs {z['value']} {z['unit']} "
                f"({100 * z['frac_of_peak']:.1f}% of peak; the rest is the power-managed clock)")

    head = results.get("gemm_bf16_8192") or next(iter(results.values()))
    head_cpu = None
    if cpu and head["name"] == "gemm_bf16_8192":
        head_cpu = cpu_baseline()
        head["cpu_baseline"] = head_cpu
        log(f"[bench] cpu baseline: {head_cpu['value']} TFLOP/s on {head_cpu['cores']} threads")
    workloads = {
        "gemm_bf16_8192": "bf16 GEMM M=N=K=8192, A row-major, B column-major, fp32 acc, bf16 out",
    }
    line = {
        "metric": METRIC,
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if "bf16" in head["name"] else ("fp8" if "fp8" in head["name"] else "f16"),
        "data": "synthetic (seeded recipes of the BASELINE configs; inputs resident in HBM)",
        "config": {"workload": workloads.get(head["name"], head["name"]),
                   "parallelism": "single GPU"},
        "roofline": head.get("roofline"),
        "cpu_baseline": head_cpu,
        "components": results,
        "device": {"name": info["name"], "arch": info["gcn_arch"], "cus": info["compute_units"]},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
