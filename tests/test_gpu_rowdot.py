"""Parity of the gfx950 unembed row dot (Bundle::rowdot_f32 and
rowdot_f32_subset, src/bundle.rs:958-1015) against the CPU oracle: every
output bit-identical (f32 / f16: the fold from -0.0; rowi8: scale times the
AVX2 eight-lane order for the full dot, the fold for the subset)."""
import numpy as np
import pytest

import oracle
from fieldrun_amd import FrqError, hip

pytestmark = pytest.mark.gpu


def table(kind, rows, d, seed):
    rng = np.random.default_rng(seed)
    if kind == "f32":
        return (rng.standard_normal((rows, d)) * 0.02).astype(np.float32), None
    if kind == "f16":
        return (rng.standard_normal((rows, d)) * 0.02).astype(np.float16), None
    q = rng.integers(-127, 128, (rows, d)).astype(np.int8)
    s = rng.uniform(1e-4, 3e-4, rows).astype(np.float16).astype(np.float32)
    return q, s


def oracle_data(kind, data):
    return data.view(np.uint16) if kind == "f16" else data


def same_bits(a, b):
    """Bit-identical, NaNs matched by position (their payloads differ between
    x86's default NaN and the GPU's)."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


@pytest.mark.parametrize("kind", ["f32", "f16", "rowi8"])
@pytest.mark.parametrize("rows,d", [(1, 1), (7, 7), (64, 8), (65, 9), (300, 63), (257, 64), (513, 65),
                                    (1000, 127), (999, 129), (2000, 768), (1500, 2304), (300, 3000)])
def test_rowdot_bit_exact(ctx, kind, rows, d):
    data, scale = table(kind, rows, d, rows * 7 + d)
    x = np.random.default_rng(d).standard_normal(d).astype(np.float32)
    t = ctx.upload_rows(kind, data, scale)
    got = t.rowdot_f32(x)
    want = oracle.rowdot_f32(kind, oracle_data(kind, data), x, scale)
    assert same_bits(got, want)
    # the subset: candidates in any order, repeats, and ids outside [0, rows)
    rng = np.random.default_rng(rows + d)
    cand = np.concatenate([rng.integers(0, rows, 50), [-1, rows, rows + 5, -(1 << 40), 0, rows - 1]])
    rng.shuffle(cand)
    gs = t.rowdot_f32_subset(x, cand)
    ws = oracle.rowdot_f32_subset(kind, oracle_data(kind, data), x, cand, scale)
    assert same_bits(gs, ws)
    assert np.isneginf(gs[(cand < 0) | (cand >= rows)]).all()
    t.free()


def test_rowdot_gpt2_vocab_device_entry_points(ctx):
    rows, d = 50257, 768
    data, _ = table("f16", rows, d, 5)
    x = np.random.default_rng(6).standard_normal(d).astype(np.float32)
    t = ctx.upload_rows("f16", data, None)
    dx = hip.DeviceArray.from_numpy(x)
    do = hip.DeviceArray((rows,), np.float32)
    t.rowdot_f32_dev(dx.ptr, do.ptr)
    ctx.sync()
    want = oracle.rowdot_f32("f16", data.view(np.uint16), x)
    assert same_bits(do.numpy(), want)
    cand = np.array([3, 50256, 50257, -2, 17], np.int64)
    dc = hip.DeviceArray.from_numpy(cand)
    dso = hip.DeviceArray((len(cand),), np.float32)
    t.rowdot_f32_subset_dev(dx.ptr, dc.ptr, len(cand), dso.ptr)
    ctx.sync()
    assert same_bits(dso.numpy(), oracle.rowdot_f32_subset("f16", data.view(np.uint16), x, cand))
    t.free()


@pytest.mark.parametrize("kind", ["f32", "f16", "rowi8"])
def test_rowdot_special_values_and_order(ctx, kind):
    # non-finite activations propagate as in the reference (no panic on this
    # path); the order case of the oracle test holds on the device too
    rows, d = 130, 40
    data, scale = table(kind, rows, d, 11)
    x = np.random.default_rng(12).standard_normal(d).astype(np.float32)
    x[3], x[17], x[33] = np.inf, -np.inf, np.nan
    t = ctx.upload_rows(kind, data, scale)
    assert same_bits(t.rowdot_f32(x), oracle.rowdot_f32(kind, oracle_data(kind, data), x, scale))
    t.free()
    x = np.array([2.0 ** 24] + [1.0] * 8, np.float32)
    one = np.ones((3, 9))
    sc = np.ones(3, np.float32)
    dt = {"f32": np.float32, "f16": np.float16, "rowi8": np.int8}[kind]
    t = ctx.upload_rows(kind, one.astype(dt), sc if kind == "rowi8" else None)
    full = t.rowdot_f32(x)
    assert np.all(full == (2.0 ** 24 + 8 if kind == "rowi8" else 2.0 ** 24))
    assert np.all(t.rowdot_f32_subset(x, [0, 2]) == 2.0 ** 24)
    t.free()


def test_rowdot_edges(ctx):
    # d == 0: the fold's -0.0 (f32 / f16 / subset) and the lanes' +0.0
    x = np.zeros(0, np.float32)
    t = ctx.upload_rows("f16", np.zeros((5, 0), np.float16))
    got = t.rowdot_f32(x)
    assert np.all(got == 0) and np.all(np.signbit(got))
    t.free()
    t = ctx.upload_rows("rowi8", np.zeros((5, 0), np.int8), np.ones(5, np.float32))
    got = t.rowdot_f32(x)
    assert np.all(got == 0) and not np.any(np.signbit(got))
    sub = t.rowdot_f32_subset(x, [4])
    assert sub[0] == 0 and np.signbit(sub[0])
    assert t.rowdot_f32_subset(x, np.zeros(0, np.int64)).shape == (0,)
    t.free()
    # a row table is not a linear weight, and a linear weight has no row dot
    t = ctx.upload_rows("f32", np.ones((4, 8), np.float32))
    with pytest.raises(FrqError):
        t.mm(np.ones((1, 8), np.float32))
    t.free()
    from fieldrun_amd import synth
    wt, scale = synth.int8_weight(16, 64, 1)
    w = ctx.upload_i8(wt, scale)
    import fieldrun_amd as fa
    out = np.empty(16, np.float32)
    rc = fa.lib.frq_rowdot_f32(ctx.h, w.h, np.ones(64, np.float32).ctypes.data, out.ctypes.data)
    assert rc == fa.FRQ_ERR_DTYPE
    w.free()
