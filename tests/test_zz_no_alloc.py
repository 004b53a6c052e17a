"""frq_mm_dev_noalloc (no counterpart in the reference: the linear for
callers that cannot allocate) against frq_mm_dev, through the C ABI: the
same bits for int8 decode batches, the int8 MFMA GEMM, int4 and q4a, over
two calls in a row, the second with a smaller input (the static scratch
keeps the first call's contents); a call that needs more scratch than the
static array holds is refused with FRQ_ERR_ARG."""
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
