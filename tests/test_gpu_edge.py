"""Empty and degenerate inputs through the C ABI, as the reference's program
loop treats them: a grid of zero programs or an empty output does nothing
(crates/sile-backend/src/cpu/codegen.rs:409-431, the `pid < total` loop), and
the canonical matmul with K below one BK (k_limit = 0) writes C = 0
(crates/sile-tile-ir/src/passes/lowering/canonical_matmul.rs:58-73)."""
import numpy as np
import pytest

from tests.helpers import say

pytestmark = pytest.mark.gpu

# (a type, c type)
GEMM_TYPES = [("bf16", "bf16"), ("bf16", "f32"), ("f16", "f16"), ("f8", "bf16"), ("f8", "f32"),
              ("f32", "f32")]


def _t(hip, name):
    return {"bf16": hip.BF16, "f16": hip.F16, "f8": hip.F8E4M3, "f32": hip.F32}[name]


@pytest.mark.parametrize("a_name,c_name", GEMM_TYPES)
@pytest.mark.parametrize("m,n", [(256, 256), (300, 260), (5, 7)])
def test_gemm_k_prime_zero_writes_zeros(hip, a_name, c_name, m, n):
    """K = 16 with bk = 32: K' = 0, so every cell of C is +0.0 (any M, N);
    the padding columns between N and ldc stay untouched."""
    say(f"gemm K'=0 {a_name}->{c_name} {m}x{n}")
    a_t, c_t = _t(hip, a_name), _t(hip, c_name)
    k, bk = 16, 32
    eb, cb = hip.dtype_bytes(a_t), hip.dtype_bytes(c_t)
    ldc = n + 8
    da = hip.DeviceBuffer(m * k * eb)
    db = hip.DeviceBuffer(n * k * eb)
    da.fill_bytes(0x7F)  # NaN / large patterns: no term may be read
    db.fill_bytes(0x7F)
    dc = hip.DeviceBuffer(m * ldc * cb)
    dc.fill_bytes(0xFF)
    b_layout = hip.COL_MAJOR
    hip.gemm(a_t, a_t, c_t, m, n, k, da.ptr, k, hip.ROW_MAJOR, db.ptr, k, b_layout, dc.ptr, ldc,
             1.0, 1.0, bk)
    hip.synchronize()
    words = dc.download(np.uint16, (m, ldc * cb // 2))
    assert (words[:, : n * cb // 2] == 0).all()
    assert (words[:, n * cb // 2:] == 0xFFFF).all()


@pytest.mark.parametrize("a_name,c_name", GEMM_TYPES)
def test_gemm_empty_output_is_a_no_op(hip, a_name, c_name):
    say(f"gemm empty {a_name}->{c_name}")
    a_t, c_t = _t(hip, a_name), _t(hip, c_name)
    dc = hip.DeviceBuffer(4096)
    dc.fill_bytes(0xAB)
    for m, n in ((0, 256), (256, 0), (0, 0)):
        # no operand is read when C is empty: NULL A and B are accepted
        hip.gemm(a_t, a_t, c_t, m, n, 64, 0, 64, hip.ROW_MAJOR, 0, 64, hip.COL_MAJOR, dc.ptr,
                 max(n, 1), 1.0, 1.0, 0)
    hip.synchronize()
    assert (dc.download(np.uint8, (4096,)) == 0xAB).all()


def test_softmax_and_reduce_empty_inputs(hip):
    """rows = 0 does nothing; a row of zero columns has no softmax or reduce."""
    say("softmax / reduce empty")
    dy = hip.DeviceBuffer(1024)
    dy.fill_bytes(0xAB)
    hip.softmax_rows(hip.F16, hip.F16, 0, 64, 0, 64, dy.ptr, 64)
    hip.reduce_rows(hip.REDUCE_MAX, hip.F32, 0, 64, 0, 64, dy.ptr)
    hip.synchronize()
    assert (dy.download(np.uint8, (1024,)) == 0xAB).all()
    dx = hip.DeviceBuffer(1024)
    with pytest.raises(hip.SileError) as e:
        hip.softmax_rows(hip.F16, hip.F16, 4, 0, dx.ptr, 0, dy.ptr, 0)
    assert e.value.kind == "Shape"
    with pytest.raises(hip.SileError) as e:
        hip.reduce_rows(hip.REDUCE_SUM, hip.F32, 4, 0, dx.ptr, 0, dy.ptr)
    assert e.value.kind == "Shape"


def test_flash_attention_empty_inputs(hip):
    say("flash attention empty")
    do = hip.DeviceBuffer(1024)
    do.fill_bytes(0xAB)
    for b, h, s in ((0, 32, 256), (4, 0, 256), (4, 32, 0)):
        hip.flash_attn_fwd(hip.F16, b, h, s, 128, 0, 0, 0, do.ptr, 0.088, True)
    hip.synchronize()
    assert (do.download(np.uint8, (1024,)) == 0xAB).all()
