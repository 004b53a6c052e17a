"""Affine int4 (q4a) linears on the device against the oracle
(Bundle::mm's Q4A arm, src/bundle.rs:802-845): M == 1 bit-identical to
q4a_dot_avx2's order and M > 1 to the dequantise + sequential-k GEMM order,
over Gemma-2-2b shapes, odd K, groups that start mid-byte and the reader's
default group of 64; and a q4a linear written to a bundle and read back."""
import numpy as np
import pytest

import fieldrun_amd as fa
import oracle
from fieldrun_amd import synth
from fieldrun_amd.bundle import BundleWriter, manifest

pytestmark = pytest.mark.gpu


def q4a_weight(n, k, g, s):
    rng = np.random.default_rng(s)
    packed = rng.integers(0, 256, (n, (k + 1) // 2), dtype=np.uint8)
    if k % 2:
        packed[:, -1] &= 0x0F
    ng = (k + g - 1) // g
    s16 = rng.uniform(0.002, 0.02, (n, ng)).astype(np.float16)
    m16 = rng.uniform(-0.15, 0.0, (n, ng)).astype(np.float16)
    return packed, s16, m16


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("n,k,g", [(9216, 2304, 32), (2304, 9216, 32), (2048, 2304, 32), (300, 37, 16),
                                   (257, 100, 64), (64, 26, 13), (1000, 4096, 64), (33, 8, 32),
                                   (512, 1024, 32), (300, 2048, 64)])
@pytest.mark.parametrize("m", [1, 3, 16, 20])
def test_q4a_mm_bit_exact(ctx, n, k, g, m):
    packed, s16, m16 = q4a_weight(n, k, g, n + k + g)
    w = ctx.upload_q4a(packed, s16, m16, k, g)
    a = synth.activations(m, k, m + k, outlier_scale=1.0)
    got = w.mm(a)
    ref = oracle.mm_q4a(a, packed, s16.astype(np.float32), m16.astype(np.float32), k, g)
    assert same_bits(got, ref)
    w.free()


def test_q4a_bundle_round_trip(ctx, tmp_path):
    rng = np.random.default_rng(11)
    stem = str(tmp_path / "q")
    src = (rng.standard_normal((96, 70)) * 0.05).astype(np.float32)     # (out, in)
    bw = BundleWriter(stem)
    bw.put_lin("l0.mlp.up_proj", src, "q4a")
    bw.finish(manifest("rope", [1, 2, 1, 32, 70, 96, 10, 0]))
    b = fa.Bundle(stem, ctx)
    dt, shape, group, _ = b.info("l0.mlp.up_proj")
    assert (dt, shape, group) == ("q4a", (96, 70), 32)
    packed, s16, m16, g = oracle.put_q4a(src, True)
    assert np.array_equal(b.arr("l0.mlp.up_proj"), packed)
    for mrows in (1, 5):
        a = synth.activations(mrows, 70, mrows, outlier_scale=1.0)
        ref = oracle.mm_q4a(a, packed, oracle.f16_to_f32(s16), oracle.f16_to_f32(m16), 70, g)
        assert same_bits(b.mm(a, "l0.mlp.up_proj"), ref)
    b.close()
