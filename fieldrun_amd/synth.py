"""Seeded synthetic workloads of the BASELINE configs (host-side numpy).

Seeds are 0xF1E1D000 + config_index*1000 + replica.  Generated once on the
host; the same arrays feed the HIP path and the CPU oracle.
"""
from __future__ import annotations

import numpy as np

from . import convert

SEED0 = 0xF1E1D000

# the isolated int8 linear sweep
SWEEP_M = (1, 4, 16, 128, 2048)
SWEEP_KN = ((896, 4864), (4864, 896), (896, 151936), (4096, 14336), (14336, 4096))


def seed(config: int, replica: int = 0) -> int:
    return SEED0 + config * 1000 + replica


def outlier_channels(k: int, rng: np.random.Generator) -> np.ndarray:
    """round(0.01 K) fixed channels (the same for every row)."""
    n = max(1, int(round(0.01 * k)))
    return np.sort(rng.choice(k, n, replace=False))


def activations(m: int, k: int, s: int, outlier_scale: float = 20.0) -> np.ndarray:
    """A ~ N(0,1) (M,K) f32 with 1% of the channels multiplied by 20."""
    rng = np.random.default_rng(s)
    chans = outlier_channels(k, np.random.default_rng(s ^ 0x5A5A))
    a = rng.standard_normal((m, k), dtype=np.float32)
    a[:, chans] *= np.float32(outlier_scale)
    return a


def int8_weight(n: int, k: int, s: int):
    """W (N,K) int8 uniform in [-127,127]; f32 row scales that are
    f16-representable values in [1e-4, 3e-4]."""
    rng = np.random.default_rng(s + 1)
    wt = rng.integers(-127, 128, (n, k), dtype=np.int8)
    scale = rng.uniform(1e-4, 3e-4, n).astype(np.float16).astype(np.float32)
    return wt, scale


def int4_weight(n: int, k: int, s: int, std: float = 0.02):
    """put_i4 of N(0, std) weights, shape (out=N, in=K): packed, f16 scales, g."""
    rng = np.random.default_rng(s + 2)
    src = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(std)).astype(np.float32)
    return convert.put_i4(src, transpose=True)


def moe_layer(E: int, d: int, mi: int, s: int, act: int = 0, std: float = 0.02):
    """Experts as put_i8 stores them: (in,out) int8 + f32 scales (from f16)."""
    rng = np.random.default_rng(s + 3)
    gw = mi if act == 0 else 2 * mi

    def lin(out, inp):
        src = (rng.standard_normal((out, inp), dtype=np.float32) * np.float32(std)).astype(np.float32)
        w, s16 = convert.put_i8(src, transpose=True)
        return w, s16.astype(np.float32)

    gate, gs, up, us, down, ds = [], [], [], [], [], []
    for _ in range(E):
        w, sc = lin(gw, d); gate.append(w); gs.append(sc)
        if act == 0:
            w, sc = lin(mi, d); up.append(w); us.append(sc)
        w, sc = lin(d, mi); down.append(w); ds.append(sc)
    return gate, gs, up, us, down, ds
