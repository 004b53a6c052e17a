"""frq_mm_dev_noalloc (no counterpart in the reference: the linear for
callers that cannot allocate) against frq_mm_dev, through the C ABI: the
same bits for int8 decode batches, the int8 MFMA GEMM, int4 and q4a, over
two calls in a row, the second with a smaller input (the static scratch
keeps the first call's contents); a call that needs more scratch than the
static array holds is refused with FRQ_ERR_ARG; and on a fresh context the
calls leave the device's free memory unchanged, where frq_mm_dev grows the
context's workspace."""
import ctypes as C

import numpy as np
import pytest

import fieldrun_amd as fa
from fieldrun_amd import convert, hip, synth

pytestmark = pytest.mark.gpu


def run(w, a, noalloc):
    m, n = a.shape[0], w.n
    da = hip.DeviceArray.from_numpy(a)
    do = hip.DeviceArray((m, n), np.float32)
    do.zero()
    (w.mm_dev_noalloc if noalloc else w.mm_dev)(da.ptr, m, do.ptr)
    w.ctx.sync()
    return do.numpy()


def same_bits(x, y):
    return np.array_equal(x.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("k,n,ms", [(4096, 1024, (16, 3)), (896, 4864, (1, 1)), (4864, 896, (8, 2)),
                                    (896, 4864, (128, 40)), (768, 2304, (64, 17))])
def test_noalloc_int8_matches_mm_dev(ctx, k, n, ms):
    wt, scale = synth.int8_weight(n, k, 41 + k)
    w = ctx.upload_i8(wt, scale)
    for i, m in enumerate(ms):
        a = synth.activations(m, k, 300 + 7 * i + m)
        ref = run(w, a, False)
        got = run(w, a, True)
        assert same_bits(got, ref), (m, k, n)
    w.free()


def test_noalloc_int4_and_q4a_match_mm_dev(ctx):
    k, n = 2304, 1024
    packed, s16, g = synth.int4_weight(n, k, 5)
    w4 = ctx.upload_i4(packed, s16, k, g)
    rng = np.random.default_rng(9)
    src = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    qp, qs, qm, qg = convert.put_q4a(src, True)
    wq = ctx.upload_q4a(qp, qs, qm, k, qg)
    for w in (w4, wq):
        for i, m in enumerate((8, 2, 1)):
            a = synth.activations(m, k, 500 + i, outlier_scale=1.0)
            assert same_bits(run(w, a, True), run(w, a, False)), (w.dtype, m)
        w.free()


def test_noalloc_refuses_what_does_not_fit(ctx):
    k, n = 14336, 4096
    wt, scale = synth.int8_weight(n, k, 3)
    w = ctx.upload_i8(wt, scale)
    m = 2048
    da = hip.DeviceArray((m, k), np.float32)
    da.zero()
    do = hip.DeviceArray((m, n), np.float32)
    with pytest.raises(fa.FrqError) as e:
        w.mm_dev_noalloc(da.ptr, m, do.ptr)
    assert e.value.code == fa.FRQ_ERR_ARG and "scratch" in str(e.value)
    # and the entry point still works after the refusal
    a = synth.activations(4, k, 11)
    assert same_bits(run(w, a, True), run(w, a, False))
    w.free()


def test_noalloc_allocates_nothing(ctx):
    """The defining property: calls on a fresh context (its workspace still
    empty) through the int8 decode batch, the int8 MFMA GEMM, int4 and q4a
    leave the device's free memory where it was; the same calls through
    frq_mm_dev on that context allocate its workspace (the control that
    the measurement sees an allocation)."""
    rng = np.random.default_rng(13)
    wt, scale = synth.int8_weight(4864, 896, 61)
    w8 = ctx.upload_i8(wt, scale)
    packed, s16, g = synth.int4_weight(1024, 2304, 62)
    w4 = ctx.upload_i4(packed, s16, 2304, g)
    qp, qs, qm, qg = convert.put_q4a(rng.standard_normal((1024, 2304), dtype=np.float32) * np.float32(0.02), True)
    wq = ctx.upload_q4a(qp, qs, qm, 2304, qg)
    calls = []
    for w, m, k, n, so in ((w8, 8, 896, 4864, 20.0), (w8, 64, 896, 4864, 20.0), (w4, 8, 2304, 1024, 1.0),
                           (wq, 2, 2304, 1024, 1.0)):
        da = hip.DeviceArray.from_numpy(synth.activations(m, k, 70 + m, outlier_scale=so))
        do = hip.DeviceArray((m, n), np.float32)
        calls.append((w, m, da, do))
    for w, m, da, do in calls:  # the kernels' code loaded, on the test's context
        w.mm_dev_noalloc(da.ptr, m, do.ptr)
    ctx.sync()
    fresh = fa.Context(0)
    before = hip.mem_info()[0]
    for w, m, da, do in calls:
        assert fa.lib.frq_mm_dev_noalloc(fresh.h, w.h, C.c_void_p(da.ptr), m, C.c_void_p(do.ptr)) == 0
    assert fa.lib.frq_sync(fresh.h) == 0
    assert hip.mem_info()[0] == before
    for w, m, da, do in calls:
        assert fa.lib.frq_mm_dev(fresh.h, w.h, C.c_void_p(da.ptr), m, C.c_void_p(do.ptr)) == 0
    assert fa.lib.frq_sync(fresh.h) == 0
    assert hip.mem_info()[0] < before
    fresh.close()
    for w in (w8, w4, wq):
        w.free()
