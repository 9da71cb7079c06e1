"""GPU parity at the benchmarked shapes, on the benchmark's own inputs.

Every workload bench.py times is run here once with the inputs bench.py
generates (its gemm_inputs / attention_inputs / softmax_input recipes, the
seeded configurations), and a deterministic sample of the output is compared
with the CPU oracle:
  * GEMM M = N = K = 8192 (bf16 and fp8, B column-major and row-major) and
    4096 (bf16): every 16th (8192) or 4th (4096) 256-row tile of C, all
    columns, full K, against the canonical matmul on the (de)quantised fp32
    inputs;
  * causal flash attention B=4 H=32 D=128 at S = 4096 and 8192: three
    (batch, head) pairs, the first, the last and every 16th 128-query block;
  * row softmax [8192, 8192] fp16: every 64th row;
  * the matmuls generated from LLIR, f32 2048^3 (canonical and K-tile MMA
    forms): three rows of programs, bit for bit.
Bound for 16-bit and fp8 outputs: |g - r| <= 2e-2 + 1e-2 |r| (the north
star's 2e-2 absolute / 1e-2 relative), and every output element finite.
"""
import numpy as np
import pytest

import bench
from oracle import cpuref
from tests.helpers import assert_close, assert_same_bits, say

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


@pytest.mark.parametrize("kind,size,step,b_row", [("bf16", 8192, 16, False),
                                                  ("fp8", 8192, 16, False),
                                                  ("bf16", 4096, 4, False),
                                                  ("bf16", 8192, 16, True),
                                                  ("fp8", 8192, 16, True)])
def test_gemm_at_bench_shape(hip, kind, size, step, b_row):
    """b_row: the same B given row-major [K, N] (bench.py's *_brow lines)."""
    m = n = k = size
    say(f"bench-shape gemm {kind} {size}^3 B {'row' if b_row else 'column'}-major "
        f"(every {step}th 256-row tile checked)")
    a_bits, b_bits, sa, sb, t = bench.gemm_inputs(kind, size)
    da = hip.DeviceBuffer.from_array(a_bits)
    db = hip.DeviceBuffer.from_array(np.ascontiguousarray(b_bits.T) if b_row else b_bits)
    dc = hip.DeviceBuffer(m * n * 2)
    dc.fill_bytes(0xFF)  # NaN: a cell the kernel skips is caught
    hip.gemm(t, t, hip.BF16, m, n, k, da.ptr, k, hip.ROW_MAJOR, db.ptr, n if b_row else k,
             hip.ROW_MAJOR if b_row else hip.COL_MAJOR, dc.ptr, n, sa, sb)
    hip.synchronize()
    got = cpuref.f32_from_bf16(dc.download(np.uint16, (m, n)))
    for buf in (da, db, dc):
        buf.close()
    assert np.isfinite(got).all()
    if kind == "fp8":
        a32, b32 = cpuref.e4m3_decode(a_bits, sa), cpuref.e4m3_decode(b_bits, sb)
    else:
        a32, b32 = cpuref.f32_from_bf16(a_bits), cpuref.f32_from_bf16(b_bits)
    del a_bits, b_bits
    ref = np.full((m, n), np.nan, np.float32)
    cpuref.gemm_nt(a32, b32, bm=256, row_tile_step=step, out=ref)
    rows = ~np.isnan(ref[:, 0])
    assert rows.sum() == (m // 256 // step) * 256
    assert_close(got[rows], ref[rows], atol=ATOL, rtol=RTOL, what=f"{kind} {size}^3 sampled")


@pytest.mark.parametrize("s", [4096, 8192])
def test_flash_attention_at_bench_shape(hip, s):
    b, h, d = bench.ATTN_SHAPE
    say(f"bench-shape causal flash attention f16 B={b} H={h} S={s} D={d}")
    qkv = bench.attention_inputs(s)
    bufs = [hip.DeviceBuffer.from_array(x.view(np.uint16)) for x in qkv]
    do = hip.DeviceBuffer(b * h * s * d * 2)
    do.fill_bytes(0xFF)
    scale = 1.0 / np.sqrt(d)
    hip.flash_attn_fwd(hip.F16, b, h, s, d, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, do.ptr, scale,
                       True)
    hip.synchronize()
    got = do.download(np.uint16, (b, h, s, d)).view(np.float16)
    for buf in bufs + [do]:
        buf.close()
    assert np.isfinite(got).all()
    blocks = sorted(set(list(range(0, s // 128, 16)) + [s // 128 - 1]))
    for bi, hi in ((0, 0), (1, 17), (b - 1, h - 1)):
        q, k, v = (x[bi, hi].astype(np.float32) for x in qkv)
        ref = np.zeros((s, d), np.float32)
        for blk in blocks:
            sl = slice(blk * 128, blk * 128 + 128)
            cpuref.attention_fwd(q, k, v, scale, True, sl.start, sl.stop, out=ref)
            assert_close(got[bi, hi, sl].astype(np.float32), ref[sl], atol=ATOL, rtol=RTOL,
                         what=f"S={s} b{bi} h{hi} block {blk}")


def test_softmax_at_bench_shape(hip):
    rows = cols = 8192
    say(f"bench-shape softmax f16 [{rows}, {cols}]")
    x = bench.softmax_input(rows, cols)
    dx = hip.DeviceBuffer.from_array(x.view(np.uint16))
    dy = hip.DeviceBuffer(rows * cols * 2)
    dy.fill_bytes(0xFF)
    hip.softmax_rows(hip.F16, hip.F16, rows, cols, dx.ptr, cols, dy.ptr, cols)
    hip.synchronize()
    got = dy.download(np.uint16, (rows, cols)).view(np.float16)
    dx.close()
    dy.close()
    assert np.isfinite(got).all()
    sample = slice(0, rows, 64)
    ref = cpuref.softmax_rows(x[sample].astype(np.float32))
    # every softmax output here is far below 2e-2: the bound is relative
    assert_close(got[sample].astype(np.float32), ref, atol=1e-6, rtol=RTOL, what="softmax")


@pytest.mark.parametrize("gen,bk", [("matmul", 8), ("mma_k_loop", 16)])
def test_generated_matmul_at_bench_shape(hip, gen, bk):
    """The generated LLIR matmul lines (bench.py llir_matmul_f32_2048 and
    llir_mma_k_loop_f32_2048): f32 2048^3 on the bench's inputs, 64 x 64
    cells a program; the first, a middle and the last row of programs are
    bit for bit the oracle's canonical order (each cell one sequential sum
    over k of rounded products)."""
    from tests import llir_shapes
    size, tile = 2048, 64
    say(f"bench-shape generated {gen}<{tile}, {tile}, {bk}> {size}^3")
    a, b = bench.llir_matmul_inputs(size)
    kern = hip.LlirKernel(getattr(llir_shapes, gen)(tile, tile, bk), (2, tile, tile))
    da, db = hip.DeviceBuffer.from_array(a), hip.DeviceBuffer.from_array(b)
    dc = hip.DeviceBuffer(size * size * 4)
    dc.fill_bytes(0xFF)
    kern([da.ptr, db.ptr, dc.ptr], [size] * 6, ((size // tile) ** 2, 1, 1))
    got = dc.download(np.float32, (size, size))
    for buf in (da, db, dc):
        buf.close()
    kern.close()
    for tr in (0, 15, size // tile - 1):
        rows = slice(tr * tile, (tr + 1) * tile)
        want = np.zeros((tile, size), np.float32)
        cpuref.kernel_matmul(np.ascontiguousarray(a[rows]), b, want, (1, size // tile, 1), tile, tile, bk)
        assert_same_bits(got[rows], want, what=f"generated {gen}, row tile {tr}")
