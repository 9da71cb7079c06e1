"""GPU parity of sile_hip_gemm with B row-major [K, N] (N contiguous), the
canonical matmul's own layout (crates/sile-tile-ir/src/passes/lowering/canonical_matmul.rs:55-57,
226-370: bi += ldb), against the oracle's canonical matmul on the same
(de)quantised inputs (cpuref.gemm_nt on B transposed).

16-bit operands on shapes the LDS kernels take read B's tiles transposed
(sile_gemm_nn*); fp8 and every other shape write B column-major into the
device scratch first.  Bounds: |g - r| <= 2e-2 + 1e-2 |r| for 16-bit / fp8
outputs, 1e-4 absolute and relative for fp32 outputs of 16-bit operands;
every output finite where the inputs are, and C outside [M, N] untouched."""
import numpy as np
import pytest

from oracle import cpuref
from tests.helpers import assert_close, bf16_round, f16_round, fp8_quantise, rng, say

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def _operands(kind, m, n, k, kp, seed, ldb):
    """A [M, K] bits, B [K, ldb] row-major bits, scales, and the fp32 values
    the oracle multiplies: A [M, K'] and B^T [N, K']."""
    a = (rng(seed).normal(size=(m, k)) / np.sqrt(max(kp, 1))).astype(np.float32)
    b = np.zeros((k, ldb), np.float32)
    b[:, :n] = rng(seed + 1).normal(size=(k, n)) / np.sqrt(max(kp, 1))
    if kind == "fp8":
        qa, sa, a_f = fp8_quantise(a)
        qb, sb, b_f = fp8_quantise(b)
        return qa, qb, sa, sb, a_f[:, :kp], np.ascontiguousarray(b_f[:kp, :n].T)
    rnd = bf16_round if kind == "bf16" else f16_round
    (qa, a_f), (qb, b_f) = rnd(a), rnd(b)
    return qa, qb, 1.0, 1.0, a_f[:, :kp], np.ascontiguousarray(b_f[:kp, :n].T)


def _gemm(hip, kind, out, m, n, k, qa, qb, sa, sb, ldb, ldc=None, bk=0, tile=0, splits=0):
    t = {"bf16": hip.BF16, "f16": hip.F16, "fp8": hip.F8E4M3}[kind]
    c_t = {"bf16": hip.BF16, "f16": hip.F16, "f32": hip.F32}[out]
    ldc = ldc or n
    cb = 4 if c_t == hip.F32 else 2
    da, db = hip.DeviceBuffer.from_array(qa), hip.DeviceBuffer.from_array(qb)
    dc = hip.DeviceBuffer(m * ldc * cb)
    dc.fill_bytes(0xFF)   # NaN pattern: skipped cells and writes past N show
    hip.gemm(t, t, c_t, m, n, k, da.ptr, k, hip.ROW_MAJOR, db.ptr, ldb, hip.ROW_MAJOR, dc.ptr,
             ldc, sa, sb, bk, tile=tile, splits=splits)
    hip.synchronize()
    if c_t == hip.F32:
        full = dc.download(np.float32, (m, ldc))
    else:
        bits = dc.download(np.uint16, (m, ldc))
        full = (cpuref.f32_from_bf16(bits) if c_t == hip.BF16
                else bits.view(np.float16).astype(np.float32))
    if ldc > n:
        assert np.isnan(full[:, n:]).all(), "C written past N"
    return full[:, :n]


def _check(got, ref, out, what):
    if out == "f32":
        assert_close(got, ref, atol=1e-4, rtol=1e-4, what=what)
    else:
        assert_close(got, ref, atol=ATOL, rtol=RTOL, what=what)
    assert np.isfinite(got).all(), what


@pytest.mark.parametrize("kind,out", [("bf16", "bf16"), ("bf16", "f32"), ("f16", "f16"),
                                      ("f16", "f32")])
@pytest.mark.parametrize("tile", [0, 256, 128])
@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (512, 768, 320), (300, 264, 192),
                                   (257, 1032, 448), (128, 128, 96)])
def test_row_major_b_lds_kernels(hip, kind, out, tile, m, n, k):
    """The transposing LDS kernels on both tile sizes: ragged M and N (the
    last tile moved back), K' ending inside a half k-step (448 = 7 half
    k-steps)."""
    if tile == 256 and (m < 256 or n < 256):
        pytest.skip("256 x 256 tiles need M, N >= 256")
    say(f"gemm B row-major {kind}->{out} {m}x{n}x{k} tile={tile}")
    qa, qb, sa, sb, a_f, bt_f = _operands(kind, m, n, k, k, m + n + k, n)
    got = _gemm(hip, kind, out, m, n, k, qa, qb, sa, sb, n, tile=tile)
    _check(got, cpuref.gemm_nt(a_f, bt_f), out, f"B row-major {kind} {m}x{n}x{k}")


@pytest.mark.parametrize("kind,tile", [("bf16", 256), ("bf16", 128), ("f16", 0), ("fp8", 0)])
@pytest.mark.parametrize("k,bk", [(192, 50), (192, 7), (192, 100), (320, 70), (48, 33)])
def test_row_major_b_truncated_k_nonfinite_tail(hip, kind, tile, k, bk):
    """K' = (K / bk) * bk: B's rows past K' (Inf, and NaN in A's columns) reach
    LDS with the last k-step and are masked out; B in a wider pitch."""
    m, n = 256, 512
    kp = (k // bk) * bk
    ldb = n + 8
    say(f"gemm B row-major {kind} K={k} bk={bk} (K'={kp}) non-finite tail, tile={tile}")
    qa, qb, sa, sb, a_f, bt_f = _operands(kind, m, n, k, kp, 21 + k + bk, ldb)
    if kind == "fp8":
        qa[:, kp:] = 0x7F
        qb[kp:, :] = 0xFF
    else:
        qa[:, kp:] = 0x7FC0 if kind == "bf16" else 0x7E00
        qb[kp:, :] = 0x7F80 if kind == "bf16" else 0x7C00
    out = "f32"
    got = _gemm(hip, kind, out, m, n, k, qa, qb, sa, sb, ldb, bk=bk, tile=tile)
    ref = cpuref.gemm_nt(a_f, bt_f)
    if kind == "fp8":
        assert_close(got, ref, atol=ATOL, rtol=RTOL, what="fp8 B row-major truncated")
        assert np.isfinite(got).all()
    else:
        _check(got, ref, out, f"{kind} B row-major truncated")


@pytest.mark.parametrize("kind,out,m,n,k,splits,tile", [
    ("bf16", "bf16", 256, 256, 8192, 4, 256),
    ("bf16", "f32", 300, 264, 5000, 3, 128),
    ("f16", "f16", 128, 512, 4096, 0, 0),    # split chosen by shape
])
def test_row_major_b_split_k(hip, kind, out, m, n, k, splits, tile):
    say(f"gemm B row-major split {kind}->{out} {m}x{n}x{k} splits={splits} tile={tile}")
    qa, qb, sa, sb, a_f, bt_f = _operands(kind, m, n, k, k, 31 + k, n)
    got = _gemm(hip, kind, out, m, n, k, qa, qb, sa, sb, n, tile=tile, splits=splits)
    _check(got, cpuref.gemm_nt(a_f, bt_f), out, "B row-major split")
    # deterministic: a second call gives the same bits
    got2 = _gemm(hip, kind, out, m, n, k, qa, qb, sa, sb, n, tile=tile, splits=splits)
    np.testing.assert_array_equal(got, got2)


@pytest.mark.parametrize("kind,out,m,n,k,ldb_pad,ldc_pad", [
    ("fp8", "bf16", 512, 512, 256, 0, 0),     # fp8: B transposed in scratch
    ("fp8", "f32", 300, 260, 320, 16, 3),
    ("bf16", "bf16", 512, 100, 256, 0, 0),    # N below one tile
    ("bf16", "f32", 256, 260, 192, 0, 0),     # N not a multiple of 8
    ("f16", "f16", 256, 512, 128, 1, 0),      # B's rows not 16-byte aligned
    ("bf16", "bf16", 1, 1, 8, 0, 0),          # the any-shape kernel (A's rows 16 bytes)
    ("bf16", "f32", 16, 300, 136, 0, 5),
    ("bf16", "bf16", 130, 64, 200, 0, 1),     # the transposed form after the transpose
])
def test_row_major_b_other_shapes(hip, kind, out, m, n, k, ldb_pad, ldc_pad):
    say(f"gemm B row-major (scratch path) {kind}->{out} {m}x{n}x{k} ldb+{ldb_pad} ldc+{ldc_pad}")
    ldb = n + ldb_pad
    qa, qb, sa, sb, a_f, bt_f = _operands(kind, m, n, k, k, 41 + m + n + k, ldb)
    got = _gemm(hip, kind, out, m, n, k, qa, qb, sa, sb, ldb, ldc=n + ldc_pad)
    ref = cpuref.gemm_nt(a_f, bt_f)
    if kind == "fp8" or out != "f32":
        assert_close(got, ref, atol=ATOL, rtol=RTOL, what="B row-major other shapes")
        assert np.isfinite(got).all()
    else:
        _check(got, ref, out, "B row-major other shapes")
