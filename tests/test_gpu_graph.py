"""GPU: op calls captured into a HIP graph (sile_hip_graph_begin / end) and
replayed.

A graph of GEMMs (one that splits K' when run eagerly, one that takes the
transposed form eagerly, one plain), a row softmax and a causal flash
attention is replayed three times, with eager split GEMMs on another stream
and device synchronisations in between.  Every replay is checked: the ops
whose captured form equals the eager one bit for bit against the eager
result, the two GEMMs whose scratch-using forms are left out under capture
against the oracle (|g - r| <= 2e-2 + 1e-2 |r|, fp32 out 1e-4) and against
the first replay bit for bit.
"""
import numpy as np
import pytest

from oracle import cpuref
from tests.helpers import assert_close, bf16_round, rng, say

pytestmark = pytest.mark.gpu


def _bf16_operands(seed, m, n, k):
    a = (rng(seed).normal(size=(m, k)) / np.sqrt(k)).astype(np.float32)
    bt = (rng(seed + 1).normal(size=(n, k)) / np.sqrt(k)).astype(np.float32)
    (qa, a_f), (qb, b_f) = bf16_round(a), bf16_round(bt)
    return qa, qb, cpuref.gemm_nt(a_f, b_f)


def test_graph_replays_op_calls(hip):
    say("graph: capture gemm x3 + softmax + flash attention, replay x3")
    st, other = hip.Stream(), hip.Stream()
    gemms = []
    # (m, n, k, out): split K' eagerly; transposed form eagerly (N < 128); plain 128 tiles
    for idx, (m, n, k, out) in enumerate([(256, 256, 8192, hip.F32), (512, 64, 256, hip.BF16),
                                          (512, 512, 512, hip.BF16)]):
        qa, qb, ref = _bf16_operands(70 + 2 * idx, m, n, k)
        cb = 4 if out == hip.F32 else 2
        bufs = (hip.DeviceBuffer.from_array(qa), hip.DeviceBuffer.from_array(qb),
                hip.DeviceBuffer(m * n * cb))
        gemms.append((m, n, k, out, cb, ref, bufs))
    rows, cols = 64, 4096
    x = (rng(80).normal(size=(rows, cols)) * 2.0).astype(np.float16)
    dx, dy = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer(rows * cols * 2)
    b, h, s, d = 1, 2, 512, 128
    qkv = [rng(81 + i).normal(size=(b, h, s, d)).astype(np.float16) for i in range(3)]
    dq, dk, dv = (hip.DeviceBuffer.from_array(t) for t in qkv)
    do = hip.DeviceBuffer(b * h * s * d * 2)
    scale = 1.0 / np.sqrt(d)

    def calls(stream):
        for m, n, k, out, cb, ref, (da, db, dc) in gemms:
            hip.gemm(hip.BF16, hip.BF16, out, m, n, k, da.ptr, k, hip.ROW_MAJOR, db.ptr, k,
                     hip.COL_MAJOR, dc.ptr, n, 1.0, 1.0, 0, stream)
        hip.softmax_rows(hip.F16, hip.F16, rows, cols, dx.ptr, cols, dy.ptr, cols, stream)
        hip.flash_attn_fwd(hip.F16, b, h, s, d, dq.ptr, dk.ptr, dv.ptr, do.ptr, scale, True,
                           stream)

    def outputs():
        res = [dc.download(np.uint32 if cb == 4 else np.uint16, (m, n))
               for m, n, k, out, cb, ref, (da, db, dc) in gemms]
        return res + [dy.download(np.uint16, (rows, cols)), do.download(np.uint16, (b, h, s, d))]

    def clear():
        for *_, (da, db, dc) in gemms:
            dc.fill_bytes(0xFF)
        dy.fill_bytes(0xFF)
        do.fill_bytes(0xFF)
        hip.synchronize()

    clear()
    calls(st)
    st.synchronize()
    eager = outputs()

    # eager work that uses the device scratch, queued between the replays
    qa, qb, ref_o = _bf16_operands(90, 256, 512, 8192)
    ea, eb = hip.DeviceBuffer.from_array(qa), hip.DeviceBuffer.from_array(qb)
    ec = hip.DeviceBuffer(256 * 512 * 4)

    with hip.Graph(st) as graph:
        calls(st)
    first = None
    for rep in range(3):
        clear()
        graph.launch()
        hip.gemm(hip.BF16, hip.BF16, hip.F32, 256, 512, 8192, ea.ptr, 8192, hip.ROW_MAJOR,
                 eb.ptr, 8192, hip.COL_MAJOR, ec.ptr, 512, 1.0, 1.0, 0, other)
        st.synchronize()
        other.synchronize()
        got = outputs()
        say(f"graph replay {rep}")
        # plain GEMM, softmax and attention: the captured launches are the eager ones
        for i in (2, 3, 4):
            assert (got[i] == eager[i]).all(), f"replay {rep}: output {i} differs from eager"
        # the two GEMMs that run without the scratch under capture: the oracle
        for i in (0, 1):
            m, n, k, out, cb, ref, _ = gemms[i]
            val = (got[i].view(np.float32) if cb == 4
                   else cpuref.f32_from_bf16(got[i]))
            tol = (1e-4, 1e-4) if cb == 4 else (2e-2, 1e-2)
            assert_close(val, ref, atol=tol[0], rtol=tol[1], what=f"replay {rep} gemm {i}")
        if first is None:
            first = got
        else:
            for i in range(5):
                assert (got[i] == first[i]).all(), f"replay {rep}: output {i} changed"
        assert_close(ec.download(np.float32, (256, 512)), ref_o, atol=1e-4, rtol=1e-4,
                     what=f"eager split GEMM beside replay {rep}")
    graph.close()
    for buf in [x for *_, bufs in gemms for x in bufs] + [dx, dy, dq, dk, dv, do, ea, eb, ec]:
        buf.close()
    st.close()
    other.close()
