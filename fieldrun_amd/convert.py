"""Bundle-writer quantisers (the build side of the bundle format).

Vectorised restatements of BundleWriter's quantisers in
/root/reference/src/convert.rs, used to write synthetic random-init weights
in exactly the layout fieldrun's converter produces:
  put_i8        convert.rs:344-360  per-output-column symmetric int8
  put_i4        convert.rs:189-216  group-wise symmetric int4, g = min(32, in)
  put_embed_i8  convert.rs:265-279  row-major per-row int8
Scales are returned as numpy float16 (put_f16, convert.rs:147-155: IEEE
round-to-nearest-even, which numpy's float32 -> float16 cast also is).
"""
from __future__ import annotations

import numpy as np


def _as_out_in(data: np.ndarray, transpose: bool) -> np.ndarray:
    """Logical W as (out, in): nn.Linear sources are (out, in) (transpose=True),
    GPT-2 Conv1D sources are (in, out) (transpose=False)."""
    data = np.asarray(data, np.float32)
    return data if transpose else data.T


def put_i8(data: np.ndarray, transpose: bool):
    """-> (w (in, out) int8 row-major, scale float16 [out])."""
    w = _as_out_in(data, transpose)  # (out, in)
    sc = np.maximum(np.abs(w).max(axis=1, initial=0.0) / np.float32(127.0), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.rint(w / sc[:, None]), -127, 127).astype(np.int8)
    return np.ascontiguousarray(q.T), sc.astype(np.float16)


def put_i4(data: np.ndarray, transpose: bool):
    """-> (packed (out, ceil(in/2)) uint8, scale float16 (out, ng), g)."""
    w = _as_out_in(data, transpose)
    out, inp = w.shape
    g = min(32, max(inp, 1))
    ng = (inp + g - 1) // g
    pad = ng * g - inp
    wp = np.pad(w, ((0, 0), (0, pad)))
    amax = np.abs(wp.reshape(out, ng, g)).max(axis=2)
    sc = np.maximum(amax / np.float32(7.0), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.rint(w / np.repeat(sc, g, axis=1)[:, :inp]), -7, 7).astype(np.int64) & 0xF
    if inp % 2:
        q = np.pad(q, ((0, 0), (0, 1)))
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return packed, sc.astype(np.float16), g


def put_q4a(data: np.ndarray, transpose: bool):
    """Affine group int4 (src/convert.rs:223-260) -> (packed (out, ceil(in/2))
    uint8 unsigned nibbles, scale float16 (out, ng), min float16 (out, ng), g):
    per group scale = max((max - min) / 15, 1e-8), q = clamp(round_ties_even(
    (v - min) / scale), 0, 15) from the f32 scale and min."""
    w = _as_out_in(data, transpose)
    out, inp = w.shape
    g = min(32, max(inp, 1))
    ng = (inp + g - 1) // g
    pad = ng * g - inp
    wv = w.reshape(out, -1)
    mn = np.stack([wv[:, i * g:min((i + 1) * g, inp)].min(axis=1) for i in range(ng)], axis=1) if inp else \
        np.zeros((out, 0), np.float32)
    mx = np.stack([wv[:, i * g:min((i + 1) * g, inp)].max(axis=1) for i in range(ng)], axis=1) if inp else \
        np.zeros((out, 0), np.float32)
    sc = np.maximum((mx - mn) / np.float32(15.0), np.float32(1e-8)).astype(np.float32)
    rep = lambda v: np.repeat(v, g, axis=1)[:, :inp]
    q = np.clip(np.rint((w - rep(mn)) / rep(sc)), 0, 15).astype(np.int64)
    del pad
    if inp % 2:
        q = np.pad(q, ((0, 0), (0, 1)))
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return packed, sc.astype(np.float16), mn.astype(np.float32).astype(np.float16), g


def put_embed_i8(data: np.ndarray):
    """-> (q (vocab, d) int8, scale float16 [vocab])."""
    data = np.asarray(data, np.float32)
    sc = np.maximum(np.abs(data).max(axis=1, initial=0.0) / np.float32(127.0), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.rint(data / sc[:, None]), -127, 127).astype(np.int8)
    return q, sc.astype(np.float16)


def unpack_i4(packed: np.ndarray, k: int) -> np.ndarray:
    """(out, ceil(k/2)) packed -> (out, k) int8 in [-8, 7]; even index = low nibble."""
    lo = (packed & 0x0F).astype(np.int8)
    hi = (packed >> 4).astype(np.int8)
    nib = np.stack([lo, hi], axis=2).reshape(packed.shape[0], -1)[:, :k]
    return np.where(nib >= 8, nib - 16, nib).astype(np.int8)
