"""frq_mm_rows_dev: m independent rows, each bit-identical to Bundle::mm at
M == 1 (src/bundle.rs:644-919; the int4 arm in i4_dot_avx2's order,
199-225 and 767-776).  This is the linear of a batched decode step where
every row is its own sequence (Gemma::generate, src/gemma.rs:416, once per
sequence).  Every row is checked against the M == 1 device call and, at
small sizes, against the CPU oracle's M == 1 product."""
import numpy as np
import pytest

import oracle
from fieldrun_amd import synth

pytestmark = pytest.mark.gpu


def raw_i4(n, k, g, seed):
    """Random packed nibbles (every value, -8 included) and f16 scales of
    both signs, (N, K/2) and (N, K/g)."""
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, (n, (k + 1) // 2), dtype=np.uint8)
    s16 = (rng.standard_normal((n, (k + g - 1) // g)) * 0.01).astype(np.float16)
    return packed, s16


def acts(m, k, seed):
    """Activations with the decode's spread, plus a zero row, a -0 row and
    a row of one sign (sign-of-zero and cancellation corners)."""
    a = synth.activations(m, k, seed, outlier_scale=8.0)
    if m >= 3:
        a[1] = 0.0
        a[2] = -0.0
    if m >= 4:
        a[3] = np.abs(a[3])
    return a


def per_row(w, a):
    return np.concatenate([w.mm(a[i:i + 1]) for i in range(a.shape[0])])


SHAPES = [
    # (m, n, k, g): the Gemma-2 2B decode linears at batch 16 ...
    (16, 4096, 2304, 32), (16, 2304, 2048, 32), (16, 2304, 9216, 32), (16, 18432, 2304, 32),
    # ... partial batches, slices that end mid-way (K / g not a multiple of
    # 16), row counts off the workgroup's, both group sizes
    (1, 300, 2048, 32), (3, 257, 96, 32), (5, 1000, 4160, 64), (8, 33, 64, 64),
    (12, 700, 1536, 64), (15, 2311, 800, 32), (16, 4, 32, 32), (2, 5000, 512, 64),
]


@pytest.mark.parametrize("m,n,k,g", SHAPES)
def test_i4_rows_match_m1(ctx, m, n, k, g):
    packed, s16 = raw_i4(n, k, g, 7000 + n + k)
    a = acts(m, k, 7100 + m)
    w = ctx.upload_i4(packed, s16, k, g)
    out = w.mm_rows(a)
    ref = per_row(w, a)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    if m >= 3:
        assert not np.signbit(out[1:3]).any()  # a zero row sums to +0
    w.free()


@pytest.mark.parametrize("m,n,k,g", [(3, 257, 96, 32), (8, 33, 64, 64), (5, 120, 4160, 64), (16, 64, 2304, 32)])
def test_i4_rows_match_oracle(ctx, m, n, k, g):
    packed, s16 = raw_i4(n, k, g, 7200 + n + k)
    a = acts(m, k, 7300 + m)
    w = ctx.upload_i4(packed, s16, k, g)
    out = w.mm_rows(a)
    sc = s16.astype(np.float32)
    ref = np.concatenate([oracle.mm_i4(a[i:i + 1], packed, sc, k, g) for i in range(m)])
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    w.free()


def test_i4_rows_nonfinite(ctx):
    """inf and NaN activations propagate as at M == 1 (the M == 1 arm has no
    NaN check for int4)."""
    m, n, k, g = 6, 130, 1024, 32
    packed, s16 = raw_i4(n, k, g, 7400)
    a = acts(m, k, 7401)
    a[0, 5] = np.inf
    a[4, 700] = -np.inf
    a[5, 3] = np.nan
    w = ctx.upload_i4(packed, s16, k, g)
    out, ref = w.mm_rows(a), per_row(w, a)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    w.free()


def test_rows_int8_and_q4a(ctx):
    """The int8 and q4a weights through the same entry point."""
    rng = np.random.default_rng(7500)
    m, n, k = 7, 300, 1024
    a = acts(m, k, 7501)
    wt = rng.integers(-127, 128, (n, k), dtype=np.int8)
    scale = (rng.random(n) * 0.01 + 1e-3).astype(np.float32)
    w8 = ctx.upload_i8(wt, scale)
    assert np.array_equal(w8.mm_rows(a).view(np.uint32), per_row(w8, a).view(np.uint32))
    from fieldrun_amd import convert
    src = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    qp, qs, qm, qg = convert.put_q4a(src, transpose=True)
    wq = ctx.upload_q4a(qp, qs, qm, k, qg)
    assert np.array_equal(wq.mm_rows(a).view(np.uint32), per_row(wq, a).view(np.uint32))
    w8.free()
    wq.free()


def test_rows_repeated_mixed_shapes(ctx):
    """Back-to-back row batches of other shapes and sizes keep their bits."""
    cases = [(16, 2304, 9216, 32), (4, 512, 2048, 64), (16, 4096, 2304, 32), (1, 2304, 9216, 32)]
    ws, xs, refs = [], [], []
    for i, (m, n, k, g) in enumerate(cases):
        packed, s16 = raw_i4(n, k, g, 7600 + i)
        w = ctx.upload_i4(packed, s16, k, g)
        x = acts(m, k, 7700 + i)
        ws.append(w)
        xs.append(x)
        refs.append(per_row(w, x))
    for _ in range(2):
        for w, x, r in zip(ws, xs, refs):
            assert np.array_equal(w.mm_rows(x).view(np.uint32), r.view(np.uint32))
    for w in ws:
        w.free()
