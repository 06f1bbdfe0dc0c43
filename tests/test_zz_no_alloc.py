"""The allocation-free GEMV entry point (qtts_gemv_device_static) against
qtts_gemm_device through the C-ABI: identical bits on two calls in a row
(the second smaller, so stale scratch from the first would show), on the
split-K path whose partials and counters live in the module's device array,
and on the unsplit path; out-of-range shapes are refused."""
import ctypes as C

import numpy as np
import pytest

import qtts
from bench import Hip

pytestmark = pytest.mark.gpu


def _run(ctx, hip, K, N, rows, seed):
    w = qtts.DeviceQ4(ctx, qtts.Q4Weight.synthetic(seed, f"static.{K}.{N}", K, N))
    x = qtts.synth_normal_f32(seed, "static.x", rows * K)
    dx, dref, dgot = hip.malloc(4 * rows * K), hip.malloc(4 * rows * N), hip.malloc(4 * rows * N)
    try:
        hip.h2d(dx, x)
        w.gemm_device(dx, rows, dref)
        ctx.check(ctx.lib.qtts_gemv_device_static(w.h, C.c_void_p(dx), rows, C.c_void_p(dgot), None))
        ctx.synchronize()
        ref = np.empty(rows * N, np.float32)
        got = np.empty(rows * N, np.float32)
        for dst, src in ((ref, dref), (got, dgot)):
            rc = hip.lib.hipMemcpy(C.c_void_p(dst.ctypes.data), C.c_void_p(src), C.c_size_t(dst.nbytes), 2)
            assert rc == 0
        return w, got, ref
    finally:
        for p in (dx, dref, dgot):
            hip.free(p)


@pytest.mark.parametrize("shapes", [[(6144, 2048, 3), (4096, 1024, 2)], [(8192, 4096, 4), (2048, 1024, 1)]])
def test_static_gemv_matches_gemm_device(ctx, shapes):
    hip = Hip()
    for i, (K, N, rows) in enumerate(shapes):
        w, got, ref = _run(ctx, hip, K, N, rows, 90 + i)
        assert np.array_equal(got, ref), (K, N, rows, float(np.max(np.abs(got - ref))))
        w.close()


def test_static_gemv_limits(ctx):
    hip = Hip()
    w = qtts.DeviceQ4(ctx, qtts.Q4Weight.synthetic(95, "static.big", 64, 16416))
    dx, dy = hip.malloc(4 * 64 * 5), hip.malloc(4 * 16416 * 5)
    try:
        for rows in (0, 5):
            assert ctx.lib.qtts_gemv_device_static(w.h, C.c_void_p(dx), rows, C.c_void_p(dy), None) == qtts.QTTS_ERANGE
        assert ctx.lib.qtts_gemv_device_static(w.h, C.c_void_p(dx), 1, C.c_void_p(dy), None) == qtts.QTTS_ERANGE
        assert ctx.lib.qtts_gemv_device_static(None, C.c_void_p(dx), 1, C.c_void_p(dy), None) == qtts.QTTS_EINVAL
    finally:
        hip.free(dx)
        hip.free(dy)
        w.close()
