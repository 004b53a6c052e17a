"""The bundle writer: fieldrun's on-disk format (FORMAT.md, v1) from numpy.

Restates BundleWriter of /root/reference/src/convert.rs:124-366 — the build
side that turns weights into `<stem>.fieldrun.json` (manifest) +
`<stem>.fieldrun.bin` (blob): each put_* appends an array's little-endian
bytes to the blob and an {name, dtype, shape, offset, bytes[, group]} entry
to the manifest, in write order.  The quantisers are convert.py's (pinned
against the oracle's restatement of convert.rs):

  put_f16 / put_f32     147-172   f16 (IEEE round-to-nearest-even) / f32
  put_small             176-178   f32 if dtype == "f32", else f16
  put_lin               181-190   (out, in) source -> int8 / int4 / f16 / f32
  put_i4                196-216   group-wise int4 (out, in) packed + f16 scales
  put_q4a               223-260   affine group int4 + f16 scales and mins
  put_embed_i8 / _embed 265-291   row-major per-row int8 (rowi8) or small
  put_i8                344-360   per-output-column int8 (in, out) + f16 scales
  finish                362-365   the manifest with "arrays" appended

The reader is the library's (Bundle in fieldrun_amd, frq_bundle_open).
"""
from __future__ import annotations

import json
import os

import numpy as np

from . import convert


class BundleWriter:
    def __init__(self, stem: str):
        self.stem = os.fspath(stem)
        self._bin = open(self.stem + ".fieldrun.bin", "wb")
        self.arrays: list[dict] = []
        self.offset = 0

    def _write(self, raw: bytes | np.ndarray):
        if isinstance(raw, np.ndarray):  # the array's own bytes, no copy
            raw = np.ascontiguousarray(raw)
            self._bin.write(memoryview(raw.reshape(-1).view(np.uint8)))
            return raw.nbytes
        self._bin.write(raw)
        return len(raw)

    def entry(self, name: str, dtype: str, shape, nbytes: int, group: int | None = None):
        e = {"name": name, "dtype": dtype, "shape": [int(s) for s in shape], "offset": self.offset,
             "bytes": int(nbytes)}
        if group is not None:
            e["group"] = int(group)
        self.arrays.append(e)
        self.offset += nbytes

    def put_f16(self, name: str, data, shape=None):
        a = np.asarray(data, np.float32)
        shape = a.shape if shape is None else shape
        n = self._write(np.ascontiguousarray(a.astype("<f2")))
        self.entry(name, "f16", shape, n)

    def put_f32(self, name: str, data, shape=None):
        a = np.asarray(data, np.float32)
        shape = a.shape if shape is None else shape
        n = self._write(np.ascontiguousarray(a.astype("<f4")))
        self.entry(name, "f32", shape, n)

    def put_small(self, name: str, data, shape=None, dtype: str = "f16"):
        if dtype == "f32":
            self.put_f32(name, data, shape)
        else:
            self.put_f16(name, data, shape)

    def put_i8(self, name: str, data, transpose: bool):
        """int8 per output column; `transpose`: data is (out, in) (nn.Linear),
        else (in, out) (GPT-2 Conv1D).  Stored (in, out) + f16 __scale [out]."""
        w, s16 = convert.put_i8(data, transpose)
        n = self._write(np.ascontiguousarray(w))
        self.entry(name, "i8", w.shape, n)
        self.put_f16(name + "__scale", s16.astype(np.float32))

    def put_i4(self, name: str, data, transpose: bool):
        """Group-wise symmetric int4, g = min(32, in), stored (out, in) packed
        with f16 (out, ceil(in/g)) __scale and the "group" field."""
        packed, s16, g = convert.put_i4(data, transpose)
        out = packed.shape[0]
        inp = np.asarray(data).shape[1] if transpose else np.asarray(data).shape[0]
        n = self._write(np.ascontiguousarray(packed))
        self.entry(name, "i4", (out, inp), n, group=g)
        self.put_f16(name + "__scale", s16.astype(np.float32))

    def put_q4a(self, name: str, data, transpose: bool):
        """Affine group int4 (convert.rs:223-260): stored (out, in) packed
        unsigned nibbles with the "group" field and f16 (out, ng) __scale and
        __min siblings."""
        packed, s16, m16, g = convert.put_q4a(data, transpose)
        out = packed.shape[0]
        inp = np.asarray(data).shape[1] if transpose else np.asarray(data).shape[0]
        n = self._write(np.ascontiguousarray(packed))
        self.entry(name, "q4a", (out, inp), n, group=g)
        self.put_f16(name + "__scale", s16.astype(np.float32))
        self.put_f16(name + "__min", m16.astype(np.float32))

    def put_lin(self, name: str, data, dtype: str):
        """A weight linear from an (out, in) source: "int8" / "int4" / "q4a",
        or f16 / f32 transposed to (in, out)."""
        if dtype == "int8":
            return self.put_i8(name, data, True)
        if dtype == "int4":
            return self.put_i4(name, data, True)
        if dtype == "q4a":
            return self.put_q4a(name, data, True)
        self.put_small(name, np.ascontiguousarray(np.asarray(data, np.float32).T), None, dtype)

    def put_embed_i8(self, name: str, data):
        """Row-major per-row int8 (vocab, d), dtype tag rowi8, f16 __scale
        (vocab,)."""
        q, s16 = convert.put_embed_i8(data)
        n = self._write(np.ascontiguousarray(q))
        self.entry(name, "rowi8", q.shape, n)
        self.put_f16(name + "__scale", s16.astype(np.float32))

    def put_embed(self, name: str, data, embed_dtype: str, dtype: str = "f16"):
        if embed_dtype == "int8" and np.asarray(data).ndim == 2:
            self.put_embed_i8(name, data)
        else:
            self.put_small(name, data, None, dtype)

    def finish(self, manifest: dict):
        """Write the manifest ({"format", "version", "arch", "config", ...}
        as given) with the arrays appended, and close the blob."""
        self._bin.close()
        m = dict(manifest)
        m["arrays"] = self.arrays
        with open(self.stem + ".fieldrun.json", "w") as f:
            json.dump(m, f, separators=(",", ":"))


def manifest(arch: str, config, config_f=None, eos=None) -> dict:
    """The header convert.rs writes (e.g. 509-510 for gpt2)."""
    m = {"format": "fieldrun-bundle", "version": 1, "arch": arch, "config": [int(c) for c in config]}
    if config_f is not None:
        m["config_f"] = [float(c) for c in config_f]
    if eos is not None:
        m["eos"] = [int(e) for e in eos]
    return m
