"""The decode kernels' sequential f32 fold (the Rust iterator sum behind
RMSNorm's mean square and the softmax sums: src/gemma.rs:66-77,
src/rope.rs:26-37, 42-52) as the device computes it, a speculative
segmented fold, against the plain one-at-a-time f32 chain on the host, bit
for bit: rows whose rounding stays near the exact sum (the speculation
hits), rows that drift far from it (constant rows: every segment refolded),
heavy tails, non-finite values, the lengths around the segment split, and
a nonzero start."""
import numpy as np
import pytest

import fieldrun_amd as fa

pytestmark = pytest.mark.gpu


def host_fold(x, init):
    out = np.empty(x.shape[0], np.float32)
    for r in range(x.shape[0]):
        s = np.float32(init)
        for v in x[r]:
            s = np.float32(s + v)
        out[r] = s
    return out


@pytest.mark.parametrize("n", [1, 7, 255, 256, 511, 512, 513, 768, 2100, 2304, 3584, 18944])
def test_seq_fold_bit_exact(ctx, n):
    rng = np.random.default_rng(n)
    rows = []
    for scale in (0.05, 1.0, 30.0):
        rows.append((rng.standard_normal(n) * scale) ** 2)                     # squares of activations
    v = rng.standard_normal(n)
    v[rng.choice(n, max(1, n // 100), replace=False)] *= 20.0
    rows.append(v * v)                                                          # with outlier channels
    rows.append(np.exp(rng.standard_normal(n) * 3 - 5))                        # softmax-like
    rows.append(np.full(n, 0.1))                                                # constant: drifts far
    rows.append(np.clip(rng.standard_cauchy(n), -1e3, 1e3))                     # heavy tails, signs
    x = np.array(rows, np.float32)
    for init in (-0.0, 0.37):
        got = fa.seq_fold_f32(ctx, x, init)
        ref = host_fold(x, init)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (n, init)


def test_seq_fold_non_finite(ctx):
    n = 3584
    x = np.ones((4, n), np.float32)
    x[0, 100] = np.inf
    x[1, 3000] = np.nan
    x[2, :] = 3.0e38  # overflows to inf part way
    x[3, 2000] = -np.inf
    got = fa.seq_fold_f32(ctx, x)
    ref = host_fold(x, -0.0)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
