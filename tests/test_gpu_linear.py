"""Parity of the gfx950 int8 / int4 linear (libfrq.so through the C ABI)
against the CPU oracle on the same seeded inputs.

Bars: activation quant (a8, sa, outliers) and the i32 accumulators
bit-exact; int8 f32 outputs bit-exact on the GEMV path (same operation
order as the oracle) and on the MFMA path within
  |gpu - oracle| <= 1e-6 * |scale| * (|sa*acc| + sum_t |av_t * w_t|)
per element (the outlier correction runs on 24-bit fixed-point MFMA there);
int4 within 1e-5 of sum |a*w| per element (north_star allows 1e-4).
"""
import numpy as np
import pytest

import oracle
from fieldrun_amd import synth, convert

pytestmark = pytest.mark.gpu


def case(m, k, n, seed, outliers=True):
    a = synth.activations(m, k, seed, 20.0 if outliers else 1.0)
    wt, scale = synth.int8_weight(n, k, seed)
    return a, wt, scale


def check_quant(a, a8, sa, oi, ov):
    for i in range(a.shape[0]):
        q8, qsa, qoi, qov = oracle.quant_row(a[i])
        t = len(qoi)
        assert np.array_equal(a8[i], q8), f"a8 row {i}"
        assert sa[i].view(np.uint32) == np.float32(qsa).view(np.uint32), f"sa row {i}"
        assert np.array_equal(oi[i, :t], qoi), f"oidx row {i}"
        assert np.array_equal(ov[i, :t].view(np.uint32), qov.view(np.uint32)), f"oval row {i}"


def corr_mag(a, wt, scale, acc):
    mags = []
    for i in range(a.shape[0]):
        _, sa, oi, ov = oracle.quant_row(a[i])
        c = np.abs(wt[:, oi].astype(np.float64)) @ np.abs(ov.astype(np.float64))
        mags.append(np.abs(scale) * (np.abs(np.float64(sa) * acc[i].astype(np.float64)) + c))
    return np.array(mags)


@pytest.mark.parametrize("m,k,n", [(1, 896, 4864), (1, 4864, 896), (2, 4096, 1000), (3, 1000, 257),
                                   (4, 768, 3072), (1, 37, 5), (1, 33, 300), (2, 32, 64), (1, 1, 7),
                                   (1, 14336, 512), (3, 18944, 64), (1, 18944, 300), (1, 9000, 77),
                                   (1, 20480, 40), (5, 896, 4864), (8, 4864, 896), (16, 4096, 1024),
                                   (16, 14336, 256), (11, 33, 300), (16, 1000, 3000), (2, 896, 40000),
                                   (1, 24576, 300), (1, 30001, 64), (1, 65536, 33)])
def test_i8_gemv_bit_exact(ctx, m, k, n):
    a, wt, scale = case(m, k, n, 100 + m * 7 + k + n)
    w = ctx.upload_i8(wt, scale)
    out, acc, a8, sa, oi, ov = w.mm_debug(a)
    check_quant(a, a8, sa, oi, ov)
    ref, racc = oracle.mm_i8(a, wt, scale, with_acc=True)
    assert np.array_equal(acc, racc)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(w.mm(a).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("m,k,n", [(17, 896, 4864), (130, 512, 301), (64, 37, 50), (20, 20, 30), (200, 128, 129),
                                   (1024, 3584, 512), (300, 5000, 257), (600, 18944, 300), (40, 20480, 64),
                                   (2048, 4096, 256), (1100, 1000, 1001)])
def test_i8_mm_exact_bit_exact(ctx, m, k, n):
    """frq_mm_exact_dev at M > 16: the GEMM's exact int32 sums, then the
    M > 1 arm's sequential outlier correction with every column block's
    weights in LDS (16, 8 or 4 columns by K; ragged N and M, K below the
    outlier count), bit for bit against the oracle."""
    a, wt, scale = case(m, k, n, 300 + m + k + n)
    w = ctx.upload_i8(wt, scale)
    ref = oracle.mm_i8_mt(a, wt, scale, 16)
    got = w.mm_exact(a)
    bad = np.argwhere(got.view(np.uint32) != ref.view(np.uint32))
    assert len(bad) == 0, (len(bad), bad[:4].tolist())


@pytest.mark.parametrize("m,k,n", [(5, 896, 4864), (16, 4096, 1024), (128, 896, 640), (130, 512, 300),
                                   (64, 37, 50), (16, 14336, 256), (33, 4864, 896), (200, 128, 129),
                                   (128, 14336, 512), (2048, 128, 14336)])
def test_i8_gemm_acc_exact_out_within_tol(ctx, m, k, n):
    a, wt, scale = case(m, k, n, 200 + m + k + n)
    w = ctx.upload_i8(wt, scale)
    out, acc, a8, sa, oi, ov = w.mm_debug(a)
    check_quant(a, a8, sa, oi, ov)
    ref, racc = oracle.mm_i8(a, wt, scale, with_acc=True)
    assert np.array_equal(acc, racc)
    mag = corr_mag(a, wt, scale, racc)
    err = np.abs(out.astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= 1e-6 * mag + 1e-30), float((err / (mag + 1e-30)).max())
    rel = err.max(axis=1) / np.abs(ref).max(axis=1)
    assert rel.max() <= 1e-5


def test_i8_activation_edge_cases(ctx):
    k, n = 200, 96
    wt, scale = synth.int8_weight(n, k, 7)
    w = ctx.upload_i8(wt, scale)
    rows = [np.zeros(k), np.ones(k), -np.ones(k), np.round(np.linspace(-3, 3, k) * 2) / 2,
            np.where(np.arange(k) % 3 == 0, 5.0, 1.0), np.full(k, 1e-40),
            np.concatenate([[np.inf, -np.inf], np.ones(k - 2)]),
            np.concatenate([[3e38, -3e38], np.linspace(0, 1, k - 2)])]
    a = np.array(rows, np.float32)
    for mm in (a[:4], a):  # GEMV path (M <= 4) and MFMA path (M = 8)
        out, acc, a8, sa, oi, ov = w.mm_debug(mm)
        check_quant(mm, a8, sa, oi, ov)
        ref, racc = oracle.mm_i8(mm, wt, scale, with_acc=True)
        assert np.array_equal(acc, racc)
        assert np.array_equal(np.isnan(out), np.isnan(ref))
        assert np.array_equal(np.isinf(out), np.isinf(ref))
        fin = np.isfinite(ref)
        assert np.array_equal(out[~fin & ~np.isnan(ref)], ref[~fin & ~np.isnan(ref)])
        if len(mm) <= 4:
            assert np.array_equal(out[fin], ref[fin])
        else:
            with np.errstate(invalid="ignore", over="ignore"):
                mag = corr_mag(mm, wt, scale, racc)
            ok = fin & np.isfinite(mag)
            assert np.all(np.abs(out[ok].astype(np.float64) - ref[ok]) <= 1e-6 * mag[ok] + 1e-30)


def test_i8_nan_is_an_error_like_the_reference(ctx):
    import fieldrun_amd as fa
    wt, scale = synth.int8_weight(64, 100, 8)
    w = ctx.upload_i8(wt, scale)
    for m in (1, 9):
        a = np.ones((m, 100), np.float32)
        a[m - 1, 50] = np.nan
        with pytest.raises(fa.FrqError) as ei:
            w.mm(a)
        assert ei.value.code == fa.FRQ_ERR_NAN
    # the context stays usable, and K <= 32 with NaN does not raise
    a = np.ones((1, 100), np.float32)
    assert np.array_equal(w.mm(a), oracle.mm_i8(a, wt, scale))
    wt2, sc2 = synth.int8_weight(8, 20, 9)
    w2 = ctx.upload_i8(wt2, sc2)
    b = np.ones((1, 20), np.float32)
    b[0, 3] = np.nan
    assert np.all(np.isnan(w2.mm(b)) == np.isnan(oracle.mm_i8(b, wt2, sc2)))


def test_i8_bundle_upload_matches_transposed(ctx):
    rng = np.random.default_rng(5)
    src = (rng.standard_normal((300, 700)) * 0.02).astype(np.float32)  # (out, in)
    w_kn, s16 = convert.put_i8(src, transpose=True)
    a = synth.activations(3, 700, 11)
    wb = ctx.upload_i8_bundle(w_kn, s16)
    wt = np.ascontiguousarray(oracle.i8_transpose(w_kn))
    sc = s16.astype(np.float32)
    wd = ctx.upload_i8(wt, sc)
    ref = oracle.mm_i8(a, wt, sc)
    assert np.array_equal(wb.mm(a).view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(wd.mm(a).view(np.uint32), ref.view(np.uint32))
    a6 = synth.activations(6, 700, 12)
    assert np.array_equal(wb.mm(a6), wd.mm(a6))


@pytest.mark.parametrize("k,n", synth.SWEEP_KN)
def test_i8_sweep_full_shapes(ctx, k, n):
    """configs[1] shapes at full size: M=1, 4 and 16 fully against the
    oracle, M=128 and M=2048 on sampled rows (rows are independent)."""
    a, wt, scale = case(2048, k, n, synth.seed(1))
    w = ctx.upload_i8(wt, scale)
    out1, acc1, *_ = w.mm_debug(a[:1])
    ref1, racc1 = oracle.mm_i8(a[:1], wt, scale, with_acc=True)
    assert np.array_equal(acc1, racc1) and np.array_equal(out1, ref1)
    rows = np.array([0, 1, 127, 1000, 2047])
    for m in (128, 2048):
        out, acc, *_ = w.mm_debug(a[:m])
        r = rows[rows < m]
        ref, racc = oracle.mm_i8(a[r], wt, scale, with_acc=True)
        assert np.array_equal(acc[r], racc)
        mag = corr_mag(a[r], wt, scale, racc)
        assert np.all(np.abs(out[r].astype(np.float64) - ref) <= 1e-6 * mag + 1e-30)
    # the decode batches (M = 2 .. 16, ragged ones included: token rows past
    # M are zero lanes of the 16-row MFMA tile): every row bit-exact (the
    # multi-row MFMA path keeps the reference's epilogue order)
    for m in (2, 3, 4, 7, 16):
        ref = oracle.mm_i8_mt(a[:m], wt, scale, 16)
        assert np.array_equal(w.mm(a[:m]).view(np.uint32), ref.view(np.uint32)), m


# ------------------------------------------------------------------ int4 ----
def i4_mag(a, packed, s16, k, g):
    nib = convert.unpack_i4(packed, k).astype(np.float64)
    sc = s16.astype(np.float64)[:, np.arange(k) // g]
    return np.abs(a.astype(np.float64)) @ np.abs(nib * sc).T


@pytest.mark.parametrize("m,n,k", [(1, 2048, 2304), (1, 9216, 2304), (1, 2304, 9216), (1, 100, 64),
                                   (1, 70, 37), (1, 33, 100), (2, 300, 2304), (16, 512, 2304),
                                   (5, 70, 37), (64, 256, 1024), (1, 100, 2336), (3, 1000, 2336),
                                   (16, 2304, 9216), (7, 33, 64), (13, 4000, 96), (1, 151, 18944)])
def test_i4_parity(ctx, m, n, k):
    packed, s16, g = synth.int4_weight(n, k, 300 + n + k)
    a = synth.activations(m, k, 400 + m, outlier_scale=1.0)
    w = ctx.upload_i4(packed, s16, k, g)
    out = w.mm(a)
    ref = oracle.mm_i4(a, packed, s16.astype(np.float32), k, g)
    blocked = (m <= 16 and g == 32 and k % 32 == 0)
    if blocked:  # int8-MFMA path (24-bit fixed-point activations per group)
        mag = i4_mag(a, packed, s16, k, g)
        assert np.all(np.abs(out - ref) <= 1e-5 * mag + 1e-30)
    else:  # same operation order as the oracle: bit-exact
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_i4_blocked_nonfinite_and_extreme_groups(ctx):
    """Groups with inf / NaN / extreme activations take the exact AVX2-order
    group sum on the MFMA path; the rest of the row stays within tolerance."""
    k, n = 2304, 300
    packed, s16, g = synth.int4_weight(n, k, 77)
    a = synth.activations(4, k, 78, outlier_scale=1.0)
    a[0, 40] = np.inf
    a[1, 100] = -np.inf
    a[2, 7] = np.nan
    a[3, 200:232] = 1e-38  # a group of tiny values (digit scale out of range)
    a[3, 500] = 3e38
    w = ctx.upload_i4(packed, s16, k, g)
    with np.errstate(invalid="ignore", over="ignore"):
        out = w.mm(a)
        ref = oracle.mm_i4(a, packed, s16.astype(np.float32), k, g)
        mag = i4_mag(a, packed, s16, k, g)
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    inf = np.isinf(ref)
    assert np.array_equal(out[inf], ref[inf])
    ok = np.isfinite(ref) & np.isfinite(mag)
    assert np.all(np.abs(out[ok] - ref[ok]) <= 1e-5 * mag[ok] + 1e-30)


def test_i4_repeated_calls_of_other_shapes(ctx):
    """Back-to-back int4 calls of different shapes (sharing the context's
    workspace) give the same results as fresh ones."""
    shapes = [(1, 9216, 2304), (16, 2304, 9216), (1, 2048, 2304)]
    ws, refs, acts = [], [], []
    for i, (m, n, k) in enumerate(shapes):
        packed, s16, g = synth.int4_weight(n, k, 900 + i)
        a = synth.activations(m, k, 910 + i, outlier_scale=1.0)
        w = ctx.upload_i4(packed, s16, k, g)
        ws.append(w)
        acts.append(a)
        refs.append(w.mm(a))
    for _ in range(3):
        for w, a, r in zip(ws, acts, refs):
            assert np.array_equal(w.mm(a).view(np.uint32), r.view(np.uint32))


def test_i4_reference_kat_through_gpu(ctx):
    """i4_q4a_dot_matches_manual (src/bundle.rs:1306-1314): [0xE1,0xF3] . 1s = 1.0."""
    w = ctx.upload_i4(np.array([[0xE1, 0xF3]], np.uint8), np.array([[1.0]], np.float16), 4, 4)
    assert w.mm(np.ones((1, 4), np.float32))[0, 0] == 1.0


@pytest.mark.parametrize("m,k,n", [(1, 896, 4864), (3, 4096, 300), (40, 896, 640), (300, 4864, 896)])
def test_i8_device_entry_points_match_host(ctx, m, k, n):
    """frq_quant_i8_dev + frq_mm_i8_q_dev (device pointers, row-major a8 of
    pitch frq_quant_pitch(K)) give the same bits as frq_mm_i8_debug."""
    import fieldrun_amd as fa
    from fieldrun_amd import hip
    a, wt, scale = case(m, k, n, 500 + m + k)
    w = ctx.upload_i8(wt, scale)
    out_h, _, a8_h, sa_h, oi_h, ov_h = w.mm_debug(a)
    kp = fa.quant_pitch(k)
    da = hip.DeviceArray.from_numpy(a)
    a8 = hip.DeviceArray((m, kp), np.int8)
    sa = hip.DeviceArray((m,), np.float32)
    oi = hip.DeviceArray((m, 32), np.uint32)
    ov = hip.DeviceArray((m, 32), np.float32)
    out = hip.DeviceArray((m, n), np.float32)
    ctx.quant_dev(da.ptr, m, k, a8.ptr, sa.ptr, oi.ptr, ov.ptr)
    w.mm_q_dev(a8.ptr, sa.ptr, oi.ptr, ov.ptr, m, out.ptr)
    ctx.sync()
    assert np.array_equal(a8.numpy()[:, :k], a8_h)
    assert np.array_equal(sa.numpy(), sa_h)
    assert np.array_equal(out.numpy().view(np.uint32), out_h.view(np.uint32))


@pytest.mark.parametrize("m,k,n", [(1, 896, 4864), (4, 4864, 896), (16, 300, 257), (17, 896, 4864),
                                   (128, 3584, 640), (300, 5000, 257), (2048, 3584, 512), (40, 20480, 64)])
def test_i8_acc_dev_matches_oracle(ctx, m, k, n):
    """frq_mm_i8_acc_dev on frq_quant_i8_dev's rows: the i32 sums of every
    (row, column) bit for bit against the oracle's i8dot (the GEMV, skinny
    and MFMA GEMM dots; the GEMM is the exact path's, whose sums
    frq_mm_exact_dev's epilogue scales)."""
    import fieldrun_amd as fa
    from fieldrun_amd import hip
    a, wt, scale = case(m, k, n, 700 + m + k + n)
    w = ctx.upload_i8(wt, scale)
    kp = fa.quant_pitch(k)
    da = hip.DeviceArray.from_numpy(a)
    a8 = hip.DeviceArray((m, kp), np.int8)
    sa = hip.DeviceArray((m,), np.float32)
    oi = hip.DeviceArray((m, 32), np.uint32)
    ov = hip.DeviceArray((m, 32), np.float32)
    acc = hip.DeviceArray((m, n), np.int32)
    ctx.quant_dev(da.ptr, m, k, a8.ptr, sa.ptr, oi.ptr, ov.ptr)
    w.mm_acc_dev(a8.ptr, m, acc.ptr)
    ctx.sync()
    _, racc = oracle.mm_i8(a, wt, scale, with_acc=True)
    assert np.array_equal(acc.numpy(), racc)


def same_or_both_nan(x, y):
    x, y = np.asarray(x, np.float32), np.asarray(y, np.float32)
    nx, ny = np.isnan(x), np.isnan(y)
    return np.array_equal(nx, ny) and np.array_equal(x[~nx].view(np.uint32), y[~ny].view(np.uint32))


@pytest.mark.parametrize("n,k,g", [(9216, 2304, 32), (2304, 9216, 32), (300, 18944, 32), (5, 2304, 64),
                                   (1000, 4096, 64), (257, 96, 32), (3, 64, 64), (4097, 2048, 32)])
def test_i4_m1_stream_special_values(ctx, n, k, g):
    """The streamed M == 1 kernel (nibbles widened through f16 into
    v_fma_mix_f32) against i4_dot_avx2's order on raw random nibbles, f16
    scales including subnormal ones, and activations holding +-inf, NaN,
    +-0, f32 subnormals and values near the f32 maximum; g = 32 and 64,
    ragged row ranges, one group a row, rows long enough to cap the items
    a thread holds."""
    rng = np.random.default_rng(n * 7 + k + g)
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    ng = k // g
    s16 = (rng.uniform(0.5, 1.5, (n, ng)) * 0.01).astype(np.float16)
    s16.flat[rng.integers(0, s16.size, 8)] = np.float16(3e-7)  # f16 subnormals
    a = rng.standard_normal((1, k)).astype(np.float32)
    pos = rng.choice(k, 12, replace=False)
    a[0, pos] = np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 1e-40, -3e-42, 3e38, -3e38, 1.5e-38, 7.0, -8.0],
                         np.float32)
    w = ctx.upload_i4(packed, s16, k, g)
    got = w.mm(a)
    ref = oracle.mm_i4(a, packed, s16.astype(np.float32), k, g)
    assert same_or_both_nan(got, ref)
    # a finite row: every bit
    a2 = rng.standard_normal((1, k)).astype(np.float32)
    a2[0, pos[:4]] = np.array([1e-40, -1e-39, 2e30, -2e30], np.float32)
    assert np.array_equal(w.mm(a2).view(np.uint32), oracle.mm_i4(a2, packed, s16.astype(np.float32), k, g).view(np.uint32))
    w.free()


@pytest.mark.parametrize("n,k", [(9216, 2304), (2304, 9216), (2048, 2304), (1000, 4096), (7, 64)])
def test_i4_m1_bit_exact_avx2_order(ctx, n, k):
    """M == 1 int4 with K % 32 == 0 and g = 32: bit-identical to
    i4_dot_avx2's order (src/bundle.rs:199-225), the x86 production path."""
    packed, s16, g = synth.int4_weight(n, k, n + k)
    w = ctx.upload_i4(packed, s16, k, g)
    a = synth.activations(1, k, k, outlier_scale=1.0)
    got = w.mm(a)
    ref = oracle.mm_i4(a, packed, s16.astype(np.float32), k, g)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    w.free()
