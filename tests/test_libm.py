"""The library's f32 expf / expm1f / tanhf (the decode kernels' exp and
tanh; expf_sel is expf's branch-free form) against the system libm the
reference's f32::exp / f32::tanh call:
identical bits over a sweep of the whole f32 range (every 4093rd bit
pattern) and the special values.  (All 2^32 inputs were compared once, on
the host build: no difference.)"""
import numpy as np
import pytest

import fieldrun_amd as fa
import oracle


def sweep():
    u = np.arange(0, 1 << 32, 4093, dtype=np.uint64).astype(np.uint32)
    special = np.array([0x00000000, 0x80000000, 0x7f800000, 0xff800000, 0x7fc00000, 0x00000001, 0x80000001,
                        0x3f800000, 0xbf800000, 0x42b17218, 0x42b17217, 0xc2cff1b4, 0xc2cff1b5, 0x41b00000,
                        0x24000000, 0x33000000, 0x3eb17218, 0x3f851592, 0x4195b844, 0x4202422f],
                       np.uint32)
    return np.concatenate([u, special]).view(np.float32)


def same(a, b):
    return np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(
        a[~np.isnan(a)].view(np.uint32), b[~np.isnan(b)].view(np.uint32))


@pytest.mark.parametrize("fn", ["expf", "expm1f", "tanhf", "expf_sel"])
def test_libm_host_build_matches_system_libm(fn):
    x = sweep()
    assert same(fa.libm_f32(fn, x), oracle.libm_f32(fn.replace("_sel", ""), x))


@pytest.mark.gpu
@pytest.mark.parametrize("fn", ["expf", "expm1f", "tanhf", "expf_sel"])
def test_libm_device_matches_system_libm(ctx, fn):
    x = np.concatenate([sweep(), np.random.default_rng(3).standard_normal(1 << 20).astype(np.float32) * 30])
    assert same(fa.libm_f32(fn, x, ctx), oracle.libm_f32(fn.replace("_sel", ""), x))
