"""GPU parity of sile_hip_gemm against the CPU oracle's canonical matmul on the
(de)quantised fp32 inputs.

Tolerances: the north star's 2e-2 absolute / 1e-2 relative bound for bf16,
fp16 and fp8 outputs, applied per element as |g - r| <= 2e-2 + 1e-2 |r|;
the f32 path is bit-exact (canonical order).
"""
import numpy as np
import pytest

from oracle import cpuref
from tests.helpers import assert_close, bf16_round, f16_round, fp8_quantise, rng, say

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def _to_f32(hip, buf, c_type, m, n):
    if c_type == 0:
        return buf.download(np.float32, (m, n))
    bits = buf.download(np.uint16, (m, n))
    if c_type == hip.BF16:
        return cpuref.f32_from_bf16(bits)
    return bits.view(np.float16).astype(np.float32)


def _run(hip, a_t, c_t, a_bits, b_bits, m, n, k, scale_a=1.0, scale_b=1.0, bk=0, tile=0,
         splits=0):
    da = hip.DeviceBuffer.from_array(a_bits)
    db = hip.DeviceBuffer.from_array(b_bits)
    cbytes = 4 if c_t == hip.F32 else 2
    dc = hip.DeviceBuffer(m * n * cbytes)
    dc.fill_bytes(0xFF)  # NaN pattern: any cell the kernel skips is caught
    hip.gemm(a_t, a_t, c_t, m, n, k, da.ptr, k, hip.ROW_MAJOR, db.ptr, k, hip.COL_MAJOR,
             dc.ptr, n, scale_a, scale_b, bk, tile=tile, splits=splits)
    hip.synchronize()
    return _to_f32(hip, dc, c_t, m, n)


# tile sizes of the LDS kernels: 0 lets the shape choose, 256 / 128 force one
# (sile_hip_gemm_tiled), so every case reaches both kernels
TILES = [0, 256, 128]


SHAPES = [(256, 256, 64), (512, 256, 128), (768, 1024, 320), (2048, 2048, 1024), (256, 512, 32),
          (512, 512, 96)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("out", ["bf16", "f32"])
@pytest.mark.parametrize("tile", TILES)
def test_bf16_gemm(hip, m, n, k, out, tile):
    say(f"gemm bf16 {m}x{n}x{k} -> {out} tile={tile}")
    a = (rng(4).normal(size=(m, k)) / np.sqrt(k)).astype(np.float32)
    bt = (rng(5).normal(size=(n, k)) / np.sqrt(k)).astype(np.float32)
    a_bits, a_f = bf16_round(a)
    b_bits, b_f = bf16_round(bt)
    c_t = hip.BF16 if out == "bf16" else hip.F32
    got = _run(hip, hip.BF16, c_t, a_bits, b_bits, m, n, k, tile=tile)
    ref = cpuref.gemm_nt(a_f, b_f)
    if out == "f32":
        assert_close(got, ref, atol=1e-4, rtol=1e-4, what="bf16 gemm f32 out")
    else:
        assert_close(got, ref, atol=ATOL, rtol=RTOL, what="bf16 gemm")
        # and the bf16 output is the rounding of an fp32 value close to ref
        assert np.mean(np.abs(got - ref)) < 4e-3


@pytest.mark.parametrize("m,n,k", SHAPES[:3])
@pytest.mark.parametrize("tile", TILES)
def test_f16_gemm(hip, m, n, k, tile):
    say(f"gemm f16 {m}x{n}x{k} tile={tile}")
    a = (rng(14).normal(size=(m, k)) / np.sqrt(k)).astype(np.float32)
    bt = (rng(15).normal(size=(n, k)) / np.sqrt(k)).astype(np.float32)
    a_bits, a_f = f16_round(a)
    b_bits, b_f = f16_round(bt)
    got = _run(hip, hip.F16, hip.F16, a_bits, b_bits, m, n, k, tile=tile)
    assert_close(got, cpuref.gemm_nt(a_f, b_f), atol=ATOL, rtol=RTOL, what="f16 gemm")


def test_gemm_k_truncation(hip):
    """The reference's K truncation K' = (K // bk) * bk on K = 320: bk = 128 ->
    K' = 256, bk = 96 -> K' = 288 (both multiples of the 32-element k-step of
    the 16-bit kernels), bk = 70 -> K' = 280, which ends inside a half k-step."""
    say("gemm bf16 K truncation")
    m = n = 256
    k = 320
    a = (rng(6).normal(size=(m, k)) / np.sqrt(k)).astype(np.float32)
    bt = (rng(7).normal(size=(n, k)) / np.sqrt(k)).astype(np.float32)
    a_bits, a_f = bf16_round(a)
    b_bits, b_f = bf16_round(bt)
    for bk in (128, 96):
        got = _run(hip, hip.BF16, hip.F32, a_bits, b_bits, m, n, k, bk=bk)
        assert_close(got, cpuref.gemm_nt(a_f, b_f, bk=bk), atol=1e-4, rtol=1e-4,
                     what=f"K'={(k // bk) * bk}")
    got = _run(hip, hip.BF16, hip.F32, a_bits, b_bits, m, n, k, bk=70)
    assert_close(got, cpuref.gemm_nt(a_f, b_f, bk=70), atol=1e-4, rtol=1e-4, what="K'=280")


@pytest.mark.parametrize("m,n,k,out", [(256, 256, 128, "bf16"), (512, 768, 512, "bf16"),
                                       (2048, 2048, 2048, "bf16"), (256, 512, 320, "bf16"),
                                       (512, 256, 64, "f32"), (768, 512, 448, "f32")])
def test_fp8_gemm(hip, m, n, k, out):
    """K' = 320, 64 and 448 end in a half k-step (64 of 128 fp8 elements)."""
    say(f"gemm fp8 {m}x{n}x{k} -> {out}")
    a = rng(9).normal(size=(m, k)).astype(np.float32)
    bt = rng(10).normal(size=(n, k)).astype(np.float32)
    qa, sa, a_deq = fp8_quantise(a)
    qb, sb, b_deq = fp8_quantise(bt)
    c_t = hip.BF16 if out == "bf16" else hip.F32
    got = _run(hip, hip.F8E4M3, c_t, qa, qb, m, n, k, sa, sb)
    ref = cpuref.gemm_nt(a_deq, b_deq)
    # fp8 GEMM outputs grow like sqrt(K) here (unit-variance inputs): the
    # relative part of the bound dominates.  The fp8 MFMAs do not sum their
    # products in full fp32 precision (about 2e-3 absolute from the exact sum
    # at K = 256, with either instruction shape), so an fp32 output gets the
    # same north-star bound as a bf16 one.
    assert_close(got, ref, atol=ATOL, rtol=RTOL, what=f"fp8 gemm {out} out")


@pytest.mark.parametrize("kind,tile", [("bf16", 256), ("bf16", 128), ("fp8", 0)])
@pytest.mark.parametrize("k,bk", [(192, 96), (192, 64), (192, 50), (192, 7), (192, 100),
                                  (192, 190), (48, 33), (48, 9)])
def test_truncated_k_ignores_nonfinite_tail(hip, kind, tile, k, bk):
    """K' = (K / bk) * bk stops anywhere inside a k-step (K' = 192, 150, 189,
    100, 190, 33, 45: inside the first or the second half k-step, or at its
    end): the columns past K' (here NaN and Inf) reach LDS with the last
    k-step and must be masked out of the result."""
    m, n = 256, 512
    kp = (k // bk) * bk
    say(f"gemm {kind} K={k} bk={bk} (K'={kp}) with a non-finite tail, tile={tile}")
    a = rng(11).normal(size=(m, k)).astype(np.float32)
    bt = rng(12).normal(size=(n, k)).astype(np.float32)
    if kind == "bf16":
        a /= np.sqrt(kp)
        bt /= np.sqrt(kp)
        a_bits, a_f = bf16_round(a)
        b_bits, b_f = bf16_round(bt)
        a_bits[:, kp:] = 0x7FC0          # NaN
        b_bits[:, kp:] = 0x7F80          # +Inf
        got = _run(hip, hip.BF16, hip.F32, a_bits, b_bits, m, n, k, bk=bk, tile=tile)
        ref = cpuref.gemm_nt(a_f[:, :kp], b_f[:, :kp])
        assert_close(got, ref, atol=1e-4, rtol=1e-4, what="bf16 truncated K")
    else:
        qa, sa, a_deq = fp8_quantise(a)
        qb, sb, b_deq = fp8_quantise(bt)
        qa[:, kp:] = 0x7F                # e4m3fn NaN
        qb[:, kp:] = 0xFF
        got = _run(hip, hip.F8E4M3, hip.F32, qa, qb, m, n, k, sa, sb, bk=bk)
        ref = cpuref.gemm_nt(a_deq[:, :kp], b_deq[:, :kp])
        assert_close(got, ref, atol=ATOL, rtol=RTOL, what="fp8 truncated K")
    assert np.isfinite(got).all()


@pytest.mark.parametrize("kind", ["bf16", "fp8"])
def test_padded_leading_dimensions(hip, kind):
    """A, B and C inside larger row pitches (lda > K, ldb > K, ldc > N): the
    padding is never read into the result and never written."""
    m, n, k = 512, 256, 320
    lda, ldb, ldc = k + 64, k + 128, n + 64
    say(f"gemm {kind} {m}x{n}x{k} lda={lda} ldb={ldb} ldc={ldc}")
    a = rng(13).normal(size=(m, k)).astype(np.float32)
    bt = rng(14).normal(size=(n, k)).astype(np.float32)
    if kind == "bf16":
        a /= np.sqrt(k)
        bt /= np.sqrt(k)
        qa, a_f = bf16_round(a)
        qb, b_f = bf16_round(bt)
        t, sa, sb, pad = hip.BF16, 1.0, 1.0, 0x7FC0   # NaN in the padding
        ref = cpuref.gemm_nt(a_f, b_f)
    else:
        qa, sa, a_f = fp8_quantise(a)
        qb, sb, b_f = fp8_quantise(bt)
        t, pad = hip.F8E4M3, 0x7F
        ref = cpuref.gemm_nt(a_f, b_f)
    ap = np.full((m, lda), pad, qa.dtype)
    ap[:, :k] = qa
    bp = np.full((n, ldb), pad, qb.dtype)
    bp[:, :k] = qb
    da, db = hip.DeviceBuffer.from_array(ap), hip.DeviceBuffer.from_array(bp)
    dc = hip.DeviceBuffer(m * ldc * 4)
    dc.fill_bytes(0xFF)
    hip.gemm(t, t, hip.F32, m, n, k, da.ptr, lda, hip.ROW_MAJOR, db.ptr, ldb, hip.COL_MAJOR,
             dc.ptr, ldc, sa, sb)
    hip.synchronize()
    got = dc.download(np.float32, (m, ldc))
    tol = (1e-4, 1e-4) if kind == "bf16" else (ATOL, RTOL)
    assert_close(got[:, :n], ref, atol=tol[0], rtol=tol[1], what=f"{kind} padded")
    # the columns past N keep the 0xFF fill
    assert (got[:, n:].view(np.uint32) == 0xFFFFFFFF).all()


@pytest.mark.parametrize("kind,out,tile", [("bf16", "bf16", 256), ("bf16", "bf16", 128),
                                           ("bf16", "f32", 256), ("bf16", "f32", 128),
                                           ("f16", "f16", 256), ("f16", "f16", 128),
                                           ("fp8", "bf16", 256)])
@pytest.mark.parametrize("m,n,k", [(300, 260, 256), (257, 1028, 320), (768, 300, 448)])
def test_ragged_m_n(hip, kind, out, tile, m, n, k):
    """M and N that are not multiples of the tile (256 or 128, forced): the
    last tile row / column is computed from rows / columns M - tile / N - tile
    on.  Every
    element is checked; C sits in a wider pitch whose columns past N must keep
    their fill.  With N % 8 == 4 (all three N here) the last column tile's rows
    start 8 bytes off a 16-byte boundary, so its 16-bit C is written back with
    the 8-byte stores, the other tiles' with 16-byte stores."""
    if kind == "fp8" and k % 64:
        pytest.skip("fp8 K' is a multiple of 64")
    ldc = n + 12
    say(f"gemm {kind} ragged {m}x{n}x{k} -> {out} tile={tile}")
    a = rng(21).normal(size=(m, k)).astype(np.float32)
    bt = rng(22).normal(size=(n, k)).astype(np.float32)
    if kind == "fp8":
        qa, sa, a_f = fp8_quantise(a)
        qb, sb, b_f = fp8_quantise(bt)
        t = hip.F8E4M3
    else:
        a /= np.sqrt(k)
        bt /= np.sqrt(k)
        rnd = bf16_round if kind == "bf16" else f16_round
        (qa, a_f), (qb, b_f) = rnd(a), rnd(bt)
        sa = sb = 1.0
        t = hip.BF16 if kind == "bf16" else hip.F16
    c_t = {"bf16": hip.BF16, "f16": hip.F16, "f32": hip.F32}[out]
    cb = 4 if out == "f32" else 2
    da, db = hip.DeviceBuffer.from_array(qa), hip.DeviceBuffer.from_array(qb)
    dc = hip.DeviceBuffer(m * ldc * cb)
    dc.fill_bytes(0xFF)
    hip.gemm(t, t, c_t, m, n, k, da.ptr, k, hip.ROW_MAJOR, db.ptr, k, hip.COL_MAJOR,
             dc.ptr, ldc, sa, sb, tile=tile)
    hip.synchronize()
    got = _to_f32(hip, dc, c_t, m, ldc)
    ref = cpuref.gemm_nt(a_f, b_f)
    tol = (1e-4, 1e-4) if (out == "f32" and kind != "fp8") else (ATOL, RTOL)
    assert_close(got[:, :n], ref, atol=tol[0], rtol=tol[1], what=f"{kind} ragged")
    raw = dc.download(np.uint32 if cb == 4 else np.uint16, (m, ldc))
    assert (raw[:, n:] == (0xFFFFFFFF if cb == 4 else 0xFFFF)).all()


@pytest.mark.parametrize("m,n,k", [(200, 300, 150),      # 32-wide tiles, ragged edges
                                   (2048, 2000, 40),      # 64-wide tiles, K' not a multiple of 16
                                   (4096, 4096, 33)])     # 128-wide tiles
def test_f32_gemm_exact(hip, m, n, k):
    """The fp32 path keeps the canonical per-cell order whatever its tiling:
    bit-identical to the oracle for both B layouts."""
    say(f"gemm f32 exact {m}x{n}x{k} (both B layouts)")
    a = rng(1).uniform(-1, 1, size=(m, k)).astype(np.float32)
    b = rng(2).uniform(-1, 1, size=(k, n)).astype(np.float32)
    da, dbr = hip.DeviceBuffer.from_array(a), hip.DeviceBuffer.from_array(b)
    dbc = hip.DeviceBuffer.from_array(np.ascontiguousarray(b.T))
    dc = hip.DeviceBuffer(m * n * 4)
    ref = cpuref.gemm_nt(a, np.ascontiguousarray(b.T), bk=0)
    hip.gemm(hip.F32, hip.F32, hip.F32, m, n, k, da.ptr, k, hip.ROW_MAJOR, dbr.ptr, n,
             hip.ROW_MAJOR, dc.ptr, n)
    hip.synchronize()
    np.testing.assert_array_equal(dc.download(np.float32, (m, n)), ref)
    hip.gemm(hip.F32, hip.F32, hip.F32, m, n, k, da.ptr, k, hip.ROW_MAJOR, dbc.ptr, k,
             hip.COL_MAJOR, dc.ptr, n)
    hip.synchronize()
    np.testing.assert_array_equal(dc.download(np.float32, (m, n)), ref)


@pytest.mark.parametrize("size", [4096])
def test_bf16_gemm_config3_sampled(hip, size):
    """BASELINE config 3 at 4096^3: every 4th 256-row tile checked against the
    oracle, every element of those tiles."""
    say(f"gemm bf16 {size}^3 sampled")
    m = n = k = size
    a = (rng(4).normal(size=(m, k)) / np.sqrt(k)).astype(np.float32)
    bt = (rng(5).normal(size=(n, k)) / np.sqrt(k)).astype(np.float32)
    a_bits, a_f = bf16_round(a)
    b_bits, b_f = bf16_round(bt)
    got = _run(hip, hip.BF16, hip.BF16, a_bits, b_bits, m, n, k)
    ref = np.full((m, n), np.nan, np.float32)
    cpuref.gemm_nt(a_f, b_f, bm=256, row_tile_step=4, out=ref)
    rows = ~np.isnan(ref[:, 0])
    assert rows.sum() == 4 * 256
    assert_close(got[rows], ref[rows], atol=ATOL, rtol=RTOL, what="bf16 4096 sampled")
    assert np.isfinite(got).all()



@pytest.mark.parametrize("kind,out", [("bf16", "bf16"), ("bf16", "f32"), ("f16", "f16"),
                                      ("f16", "f32"), ("fp8", "bf16"), ("fp8", "f32")])
@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (100, 256, 64), (16, 300, 130), (255, 255, 255),
                                   (300, 100, 64), (2, 1000, 37), (257, 258, 96), (64, 64, 64)])
def test_small_shapes_mfma(hip, kind, out, m, n, k):
    """Shapes below one LDS tile, N not a multiple of 4, or (here, always)
    C's rows not 16-byte aligned run the any-shape MFMA kernel (300 x 100,
    16-bit: the transposed LDS form): every element against the oracle, C in
    a wider pitch whose columns past N keep their fill."""
    ldc = n + 3
    say(f"gemm small {kind} {m}x{n}x{k} -> {out}")
    a = rng(41).normal(size=(m, k)).astype(np.float32)
    bt = rng(42).normal(size=(n, k)).astype(np.float32)
    # leading dimensions: 16-byte multiples of the element size
    ea = 1 if kind == "fp8" else 2
    lda = ldb = -(-k * ea // 16) * 16 // ea
    if kind == "fp8":
        qa, sa, a_f = fp8_quantise(a)
        qb, sb, b_f = fp8_quantise(bt)
        t = hip.F8E4M3
    else:
        a /= np.sqrt(k)
        bt /= np.sqrt(k)
        rnd = bf16_round if kind == "bf16" else f16_round
        (qa, a_f), (qb, b_f) = rnd(a), rnd(bt)
        sa = sb = 1.0
        t = hip.BF16 if kind == "bf16" else hip.F16
    pad = 0x7F if kind == "fp8" else 0x7FC0 if kind == "bf16" else 0x7E00   # NaN
    ap = np.full((m, lda), pad, qa.dtype)
    ap[:, :k] = qa
    bp = np.full((n, ldb), pad, qb.dtype)
    bp[:, :k] = qb
    c_t = {"bf16": hip.BF16, "f16": hip.F16, "f32": hip.F32}[out]
    cb = 4 if out == "f32" else 2
    da, db = hip.DeviceBuffer.from_array(ap), hip.DeviceBuffer.from_array(bp)
    dc = hip.DeviceBuffer(m * ldc * cb)
    dc.fill_bytes(0xFF)
    hip.gemm(t, t, c_t, m, n, k, da.ptr, lda, hip.ROW_MAJOR, db.ptr, ldb, hip.COL_MAJOR,
             dc.ptr, ldc, sa, sb)
    hip.synchronize()
    got = _to_f32(hip, dc, c_t, m, ldc)
    ref = cpuref.gemm_nt(a_f, b_f)
    tol = (1e-4, 1e-4) if (out == "f32" and kind != "fp8") else (ATOL, RTOL)
    assert_close(got[:, :n], ref, atol=tol[0], rtol=tol[1], what=f"{kind} small {m}x{n}x{k}")
    raw = dc.download(np.uint32 if cb == 4 else np.uint16, (m, ldc))
    assert (raw[:, n:] == (0xFFFFFFFF if cb == 4 else 0xFFFF)).all()


@pytest.mark.parametrize("kind", ["bf16", "fp8"])
@pytest.mark.parametrize("k,bk", [(192, 50), (192, 7), (48, 33), (130, 64)])
def test_small_shapes_truncated_k(hip, kind, k, bk):
    """K' = (K / bk) * bk inside a k-step of the any-shape kernel, with NaN /
    Inf past K' in the operands: masked out."""
    m, n = 100, 72
    kp = (k // bk) * bk
    say(f"gemm small {kind} {m}x{n} K={k} bk={bk}")
    a = rng(43).normal(size=(m, k)).astype(np.float32)
    bt = rng(44).normal(size=(n, k)).astype(np.float32)
    if kind == "bf16":
        a /= np.sqrt(kp)
        bt /= np.sqrt(kp)
        qa, a_f = bf16_round(a)
        qb, b_f = bf16_round(bt)
        qa[:, kp:] = 0x7FC0
        qb[:, kp:] = 0x7F80
        t, sa, sb = hip.BF16, 1.0, 1.0
    else:
        qa, sa, a_f = fp8_quantise(a)
        qb, sb, b_f = fp8_quantise(bt)
        qa[:, kp:] = 0x7F
        qb[:, kp:] = 0xFF
        t = hip.F8E4M3
    ea = 1 if kind == "fp8" else 2
    ld = -(-k * ea // 16) * 16 // ea
    ap = np.zeros((m, ld), qa.dtype)
    ap[:, :k] = qa
    bp = np.zeros((n, ld), qb.dtype)
    bp[:, :k] = qb
    da, db = hip.DeviceBuffer.from_array(ap), hip.DeviceBuffer.from_array(bp)
    dc = hip.DeviceBuffer(m * n * 4)
    hip.gemm(t, t, hip.F32, m, n, k, da.ptr, ld, hip.ROW_MAJOR, db.ptr, ld, hip.COL_MAJOR,
             dc.ptr, n, sa, sb, bk)
    hip.synchronize()
    got = dc.download(np.float32, (m, n))
    ref = cpuref.gemm_nt(a_f[:, :kp], b_f[:, :kp])
    tol = (1e-4, 1e-4) if kind == "bf16" else (ATOL, RTOL)
    assert_close(got, ref, atol=tol[0], rtol=tol[1], what=f"{kind} small truncated K")
    assert np.isfinite(got).all()


@pytest.mark.parametrize("kind,out,tile", [("bf16", "bf16", 256), ("bf16", "bf16", 128),
                                           ("f16", "f16", 256), ("f16", "f16", 128),
                                           ("fp8", "bf16", 256), ("bf16", "f32", 256),
                                           ("bf16", "f32", 128)])
@pytest.mark.parametrize("k,bk", [(192, 50), (192, 100), (320, 70)])
def test_truncated_k_ragged_tiles_padded_rows(hip, kind, out, tile, k, bk):
    """The any-K' masking of the LDS kernels (256 and 128 tiles, forced) on a
    ragged shape (300 x 260: the last tile row and column moved back) with
    lda = ldb = K + 64: the
    elements past K' inside each row (up to K, then the row padding) are
    NaN / Inf and must be masked, for 16-bit and fp8 -> bf16 outputs too."""
    m, n = 300, 260
    kp = (k // bk) * bk
    ea = 1 if kind == "fp8" else 2
    ld = k + 64
    say(f"gemm {kind} {m}x{n} K={k} bk={bk} (K'={kp}) lda=ldb={ld} -> {out} tile={tile}")
    a = rng(45).normal(size=(m, k)).astype(np.float32)
    bt = rng(46).normal(size=(n, k)).astype(np.float32)
    if kind == "fp8":
        qa, sa, a_f = fp8_quantise(a)
        qb, sb, b_f = fp8_quantise(bt)
        nan_a, inf_b = 0x7F, 0xFF
        t = hip.F8E4M3
    else:
        a /= np.sqrt(kp)
        bt /= np.sqrt(kp)
        rnd = bf16_round if kind == "bf16" else f16_round
        (qa, a_f), (qb, b_f) = rnd(a), rnd(bt)
        nan_a = 0x7FC0 if kind == "bf16" else 0x7E00
        inf_b = 0x7F80 if kind == "bf16" else 0x7C00
        sa = sb = 1.0
        t = hip.BF16 if kind == "bf16" else hip.F16
    ap = np.full((m, ld), nan_a, qa.dtype)
    ap[:, :kp] = qa[:, :kp]
    bp = np.full((n, ld), inf_b, qb.dtype)
    bp[:, :kp] = qb[:, :kp]
    c_t = {"bf16": hip.BF16, "f16": hip.F16, "f32": hip.F32}[out]
    cb = 4 if out == "f32" else 2
    ldc = n + 4
    da, db = hip.DeviceBuffer.from_array(ap), hip.DeviceBuffer.from_array(bp)
    dc = hip.DeviceBuffer(m * ldc * cb)
    dc.fill_bytes(0xFF)
    hip.gemm(t, t, c_t, m, n, k, da.ptr, ld, hip.ROW_MAJOR, db.ptr, ld, hip.COL_MAJOR, dc.ptr,
             ldc, sa, sb, bk, tile=tile)
    hip.synchronize()
    got = _to_f32(hip, dc, c_t, m, ldc)
    ref = cpuref.gemm_nt(a_f[:, :kp], b_f[:, :kp])
    tol = (1e-4, 1e-4) if (out == "f32" and kind != "fp8") else (ATOL, RTOL)
    assert_close(got[:, :n], ref, atol=tol[0], rtol=tol[1], what=f"{kind} truncated ragged")
    assert np.isfinite(got[:, :n]).all()


@pytest.mark.parametrize("kind,out,m,n,k,bk,tile,splits", [
    ("bf16", "bf16", 256, 256, 8192, 0, 256, 16),   # 1 tile: 16 k-ranges of 512
    ("bf16", "f32", 300, 260, 5000, 0, 256, 9),     # the last range ends in a half k-step
    ("bf16", "bf16", 300, 260, 5000, 0, 128, 5),
    ("f16", "f16", 512, 512, 6000, 70, 128, 3),     # K' = 5950 ends 30 elements into a half k-step
    ("bf16", "bf16", 256, 256, 8192, 0, 0, 0),      # chosen by shape
    ("bf16", "f32", 300, 260, 5000, 0, 0, 0),
    ("f16", "f16", 512, 512, 6000, 70, 0, 0),
    ("fp8", "bf16", 512, 256, 4096, 0, 0, 0),       # scales applied once, after the ranges are summed
    ("fp8", "f32", 256, 300, 3072, 0, 256, 3),
])
def test_split_k(hip, kind, out, m, n, k, bk, tile, splits):
    """Few tiles and a long K': K' split into ranges that run side by side
    (fp32 planes of C in the device scratch), summed in range order; the
    split forced on either tile size, or chosen by shape (on a 256-CU device
    every such case here splits).  Every element is checked, C sits in a
    wider pitch whose columns past N keep their fill, and a second call gives
    the same bits."""
    kp = (k // bk) * bk if bk else k
    ldc = -(-(n + 8) // 8) * 8   # 16-byte rows for every C type
    say(f"gemm split-K {kind} {m}x{n}x{k} bk={bk} -> {out} tile={tile} splits={splits}")
    a = rng(31).normal(size=(m, k)).astype(np.float32)
    bt = rng(32).normal(size=(n, k)).astype(np.float32)
    if kind == "fp8":
        qa, sa, a_f = fp8_quantise(a)
        qb, sb, b_f = fp8_quantise(bt)
        t = hip.F8E4M3
    else:
        a /= np.sqrt(kp)
        bt /= np.sqrt(kp)
        rnd = bf16_round if kind == "bf16" else f16_round
        (qa, a_f), (qb, b_f) = rnd(a), rnd(bt)
        sa = sb = 1.0
        t = hip.BF16 if kind == "bf16" else hip.F16
    c_t = {"bf16": hip.BF16, "f16": hip.F16, "f32": hip.F32}[out]
    cb = 4 if out == "f32" else 2
    da, db = hip.DeviceBuffer.from_array(qa), hip.DeviceBuffer.from_array(qb)
    dc = hip.DeviceBuffer(m * ldc * cb)
    raws = []
    for _ in range(2):
        dc.fill_bytes(0xFF)
        hip.gemm(t, t, c_t, m, n, k, da.ptr, k, hip.ROW_MAJOR, db.ptr, k, hip.COL_MAJOR,
                 dc.ptr, ldc, sa, sb, bk, tile=tile, splits=splits)
        hip.synchronize()
        raws.append(dc.download(np.uint32 if cb == 4 else np.uint16, (m, ldc)))
    assert (raws[0] == raws[1]).all(), "split-K result differs between two calls"
    got = _to_f32(hip, dc, c_t, m, ldc)
    ref = cpuref.gemm_nt(a_f[:, :kp], b_f[:, :kp])
    tol = (1e-4, 1e-4) if (out == "f32" and kind != "fp8") else (ATOL, RTOL)
    assert_close(got[:, :n], ref, atol=tol[0], rtol=tol[1], what=f"{kind} split-K")
    assert (raws[0][:, n:] == (0xFFFFFFFF if cb == 4 else 0xFFFF)).all()


@pytest.mark.parametrize("kind,out", [("bf16", "bf16"), ("bf16", "f32"), ("f16", "f16"),
                                      ("f16", "f32"), ("fp8", "bf16"), ("fp8", "f32")])
@pytest.mark.parametrize("m,n,k,bk,tile", [(128, 128, 64, 0, 0), (200, 300, 320, 0, 0),
                                           (130, 1028, 448, 0, 0), (255, 260, 192, 50, 0),
                                           (128, 256, 8192, 0, 0), (192, 1024, 2048, 0, 0),
                                           (1, 128, 64, 0, 128), (64, 512, 256, 0, 128),
                                           (100, 300, 320, 0, 128), (16, 1024, 4096, 0, 128),
                                           (127, 260, 192, 50, 128)])
def test_tile128(hip, kind, out, m, n, k, bk, tile):
    """M or N in [128, 256): 128 x 128 tiles through LDS
    (the last tile row / column moved back to end at M / N, C in a wider
    pitch; N % 8 == 4 puts the last column tile's rows 8 bytes off a 16-byte
    boundary), K' truncated inside a half k-step (255 x 260 x 192, bk = 50),
    and K' long enough to be split (128 x 256 x 8192).  M below one tile:
    the rows past M load as zeros and are not stored (a row of C past M keeps
    its fill)."""
    kp = (k // bk) * bk if bk else k
    ldc = -(-(n + 8) // 8) * 8   # 16-byte rows for every C type
    say(f"gemm tile128 {kind} {m}x{n}x{k} bk={bk} -> {out} tile={tile}")
    a = rng(41).normal(size=(m, k)).astype(np.float32)
    bt = rng(42).normal(size=(n, k)).astype(np.float32)
    if kind == "fp8":
        qa, sa, a_f = fp8_quantise(a)
        qb, sb, b_f = fp8_quantise(bt)
        t = hip.F8E4M3
    else:
        a /= np.sqrt(kp)
        bt /= np.sqrt(kp)
        rnd = bf16_round if kind == "bf16" else f16_round
        (qa, a_f), (qb, b_f) = rnd(a), rnd(bt)
        sa = sb = 1.0
        t = hip.BF16 if kind == "bf16" else hip.F16
    c_t = {"bf16": hip.BF16, "f16": hip.F16, "f32": hip.F32}[out]
    cb = 4 if out == "f32" else 2
    da, db = hip.DeviceBuffer.from_array(qa), hip.DeviceBuffer.from_array(qb)
    # one spare row past M: the forced 128 x 128 tile must not write it
    dc = hip.DeviceBuffer((m + 1) * ldc * cb)
    dc.fill_bytes(0xFF)
    hip.gemm(t, t, c_t, m, n, k, da.ptr, k, hip.ROW_MAJOR, db.ptr, k, hip.COL_MAJOR,
             dc.ptr, ldc, sa, sb, bk, tile=tile)
    hip.synchronize()
    got = _to_f32(hip, dc, c_t, m, ldc)
    ref = cpuref.gemm_nt(a_f[:, :kp], b_f[:, :kp])
    tol = (1e-4, 1e-4) if (out == "f32" and kind != "fp8") else (ATOL, RTOL)
    assert_close(got[:, :n], ref, atol=tol[0], rtol=tol[1], what=f"{kind} tile128")
    raw = dc.download(np.uint32 if cb == 4 else np.uint16, (m + 1, ldc))
    fill = 0xFFFFFFFF if cb == 4 else 0xFFFF
    assert (raw[:m, n:] == fill).all() and (raw[m] == fill).all()


@pytest.mark.parametrize("kind,out,m,n,k,ldc_pad,bk", [
    ("bf16", "bf16", 512, 64, 256, 8, 0),      # N below one tile
    ("f16", "f16", 1024, 100, 320, 0, 0),
    ("bf16", "f32", 256, 1, 64, 3, 0),
    ("bf16", "bf16", 512, 1023, 128, 0, 0),    # N not a multiple of 4
    ("f16", "f32", 300, 258, 200, 1, 50),      # K' = 200 from bk = 50
    ("bf16", "bf16", 256, 256, 64, 3, 0),      # C's rows not 16-byte aligned
    ("bf16", "bf16", 512, 64, 8192, 0, 0),     # and K' split
    ("fp8", "bf16", 512, 258, 256, 0, 0),
    ("fp8", "bf16", 512, 64, 320, 0, 0),
    ("fp8", "f32", 256, 300, 320, 5, 0),
])
def test_transposed_form(hip, kind, out, m, n, k, ldc_pad, bk):
    """Shapes the direct LDS form cannot take (N below one tile, N not a
    multiple of 4, C's rows not 16-byte aligned) with M a multiple of 4 and at
    least one tile run C^T = B . A^T on the LDS kernels into fp32 planes,
    written back transposed with element stores.  Every element is checked,
    the pitch past N keeps its fill, and a second call gives the same bits."""
    kp = (k // bk) * bk if bk else k
    ldc = n + ldc_pad
    say(f"gemm transposed {kind} {m}x{n}x{k} ldc={ldc} bk={bk} -> {out}")
    a = rng(51).normal(size=(m, k)).astype(np.float32)
    bt = rng(52).normal(size=(n, k)).astype(np.float32)
    if kind == "fp8":
        qa, sa, a_f = fp8_quantise(a)
        qb, sb, b_f = fp8_quantise(bt)
        t = hip.F8E4M3
    else:
        a /= np.sqrt(kp)
        bt /= np.sqrt(kp)
        rnd = bf16_round if kind == "bf16" else f16_round
        (qa, a_f), (qb, b_f) = rnd(a), rnd(bt)
        sa = sb = 1.0
        t = hip.BF16 if kind == "bf16" else hip.F16
    c_t = {"bf16": hip.BF16, "f16": hip.F16, "f32": hip.F32}[out]
    cb = 4 if out == "f32" else 2
    da, db = hip.DeviceBuffer.from_array(qa), hip.DeviceBuffer.from_array(qb)
    dc = hip.DeviceBuffer(m * ldc * cb)
    raws = []
    for _ in range(2):
        dc.fill_bytes(0xFF)
        hip.gemm(t, t, c_t, m, n, k, da.ptr, k, hip.ROW_MAJOR, db.ptr, k, hip.COL_MAJOR,
                 dc.ptr, ldc, sa, sb, bk)
        hip.synchronize()
        raws.append(dc.download(np.uint32 if cb == 4 else np.uint16, (m, ldc)))
    assert (raws[0] == raws[1]).all(), "transposed form differs between two calls"
    got = _to_f32(hip, dc, c_t, m, ldc)
    ref = cpuref.gemm_nt(a_f[:, :kp], b_f[:, :kp])
    tol = (1e-4, 1e-4) if (out == "f32" and kind != "fp8") else (ATOL, RTOL)
    assert_close(got[:, :n], ref, atol=tol[0], rtol=tol[1], what=f"{kind} transposed")
    assert (raws[0][:, n:] == (0xFFFFFFFF if cb == 4 else 0xFFFF)).all()


def test_split_k_scratch_across_streams_and_growth(hip):
    """The split and transposed forms share one scratch buffer per device.
    Calls queued on two streams without waiting in between must not see each
    other's planes (the library orders them with an event), and a call that
    needs more scratch than an earlier one grows it while the earlier work
    may still be running.  Sequence: small split on stream 1, large split on
    stream 2 (grows the scratch), transposed form on stream 1, small split on
    stream 2, each with its own inputs; every result against the oracle."""
    say("gemm scratch: two streams, growth")
    cases = [(256, 256, 4096, 1), (512, 512, 8192, 2), (512, 64, 2048, 1), (256, 256, 2048, 2)]
    s1, s2 = hip.Stream(), hip.Stream()
    streams = {1: s1, 2: s2}
    runs = []
    for idx, (m, n, k, sid) in enumerate(cases):
        a = (rng(60 + 2 * idx).normal(size=(m, k)) / np.sqrt(k)).astype(np.float32)
        bt = (rng(61 + 2 * idx).normal(size=(n, k)) / np.sqrt(k)).astype(np.float32)
        (qa, a_f), (qb, b_f) = bf16_round(a), bf16_round(bt)
        da, db = hip.DeviceBuffer.from_array(qa), hip.DeviceBuffer.from_array(qb)
        dc = hip.DeviceBuffer(m * n * 4)
        dc.fill_bytes(0xFF)
        runs.append((m, n, a_f, b_f, da, db, dc))
    hip.synchronize()
    for (m, n, k, sid), (_, _, _, _, da, db, dc) in zip(cases, runs):
        hip.gemm(hip.BF16, hip.BF16, hip.F32, m, n, k, da.ptr, k, hip.ROW_MAJOR, db.ptr, k,
                 hip.COL_MAJOR, dc.ptr, n, 1.0, 1.0, 0, streams[sid])
    s1.synchronize()
    s2.synchronize()
    for idx, (m, n, a_f, b_f, da, db, dc) in enumerate(runs):
        got = dc.download(np.float32, (m, n))
        assert_close(got, cpuref.gemm_nt(a_f, b_f), atol=1e-4, rtol=1e-4,
                     what=f"scratch case {idx}")
        for x in (da, db, dc):
            x.close()
    s1.close()
    s2.close()


@pytest.mark.parametrize("m,n,k,out", [(256, 256, 1 << 20, "f32"), (256, 256, 1 << 20, "bf16"),
                                       (200, 512, 1 << 19, "f32")])
def test_gemm_long_k(hip, m, n, k, out):
    """K' of 2^19 and 2^20 bf16 elements (1-2 MiB rows, 512 MiB operands):
    half-k-step counts, k-range offsets and the split sums far past the sizes
    benchmarked.  Every element is written and finite; 16 seeded rows (with
    the first and last) against a float64 product of the same bf16 inputs."""
    say(f"gemm long K {m}x{n}x{k} -> {out}")
    a = (rng(91).normal(size=(m, k)) / np.sqrt(k)).astype(np.float32)
    bt = (rng(92).normal(size=(n, k)) / np.sqrt(k)).astype(np.float32)
    (qa, a_f), (qb, b_f) = bf16_round(a), bf16_round(bt)
    del a, bt
    c_t = hip.F32 if out == "f32" else hip.BF16
    got = _run(hip, hip.BF16, c_t, qa, qb, m, n, k)
    assert np.isfinite(got).all()
    rows = sorted({0, m - 1} | set(rng(93).integers(0, m, size=14).tolist()))
    ref = a_f[rows].astype(np.float64) @ b_f.astype(np.float64).T
    tol = (1e-4, 1e-4) if out == "f32" else (ATOL, RTOL)
    assert_close(got[rows], ref, atol=tol[0], rtol=tol[1], what=f"long K rows {rows[:3]}...")


@pytest.mark.parametrize("m,n,k", [(1 << 20, 256, 128), (1 << 20, 200, 64), (1 << 20, 100, 64),
                                   ((1 << 20) + 3, 130, 96)])
def test_gemm_tall(hip, m, n, k):
    """M of 2^20 rows (and 2^20 + 3): the LDS kernels' tile grid and row
    offsets, and the any-shape kernel (N = 100 and M not a multiple of 4,
    whose C^T planes would pass the transposed form's scratch limit) with
    its 64-row tiles in grid y.  bf16 in and out; every element written and
    finite; 64 seeded rows (with the first and last) against a float64
    product of the same bf16 inputs."""
    say(f"gemm tall {m}x{n}x{k}")
    a = (rng(95).normal(size=(m, k)) / np.sqrt(k)).astype(np.float32)
    bt = (rng(96).normal(size=(n, k)) / np.sqrt(k)).astype(np.float32)
    (qa, a_f), (qb, b_f) = bf16_round(a), bf16_round(bt)
    del a, bt
    got = _run(hip, hip.BF16, hip.BF16, qa, qb, m, n, k)
    assert np.isfinite(got).all()
    rows = sorted({0, m - 1} | set(rng(97).integers(0, m, size=62).tolist()))
    ref = a_f[rows].astype(np.float64) @ b_f.astype(np.float64).T
    assert_close(got[rows], ref, atol=ATOL, rtol=RTOL, what="tall GEMM rows")
