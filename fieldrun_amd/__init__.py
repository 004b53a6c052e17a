"""fieldrun_amd — MI355X (gfx950) quantised-linear hot path of fieldrun.

Python binding of libfrq.so (include/frq.h) through ctypes.  The library is
the product: there is no CPU fallback, and importing this package raises if
libfrq.so has not been built (``python fieldrun_amd/build.py``).

The classes mirror the reference's interface for this path
(/root/reference/src/bundle.rs):

  Weight.mm(a)            Bundle::mm(a, name) for one int8 / int4 weight
                          (src/bundle.rs:644-919)
  MoeBank.forward(...)    the routed expert branch of qwen3moe::moe_branch
                          (src/qwen3moe.rs:120-158) / gemma4 (131-187)
  MoeBank.expert_mm(...)  Bundle::expert_mm (src/bundle.rs:457-461)
  Bundle.load(stem)       Bundle::load (src/bundle.rs:314-376): manifest +
                          mapped blob; Bundle.mm / rowdot_f32 / expert bank
                          upload each array once onto the context's device
  RowTable.rowdot_f32(x)  Bundle::rowdot_f32 (src/bundle.rs:958-987), the
                          unembed over an f32 / f16 / rowi8 (vocab, d) table,
                          and rowdot_f32_subset (995-1015)

Errors the reference raises by panicking come back as FrqError carrying the
library's status code and message.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libfrq.so")

FRQ_OK, FRQ_ERR_ARG, FRQ_ERR_HIP, FRQ_ERR_NAN = 0, 1, 2, 3
FRQ_ERR_DTYPE, FRQ_ERR_FORMAT, FRQ_ERR_MISSING, FRQ_ERR_NODEV = 4, 5, 6, 7
FRQ_DT_I8, FRQ_DT_I4, FRQ_DT_F32, FRQ_DT_F16, FRQ_DT_ROWI8, FRQ_DT_Q4A = 1, 2, 3, 4, 5, 6
FRQ_ACT_SILU, FRQ_ACT_GELU_TANH = 0, 1

# name -> (restype, argtypes); every symbol include/frq.h declares
_P, _S, _I = C.c_void_p, C.c_size_t, C.c_int
SIGNATURES = {
    "frq_last_error": (C.c_char_p, []),
    "frq_version": (C.c_char_p, []),
    "frq_device_count": (_I, []),
    "frq_init": (_P, [_I]),
    "frq_free": (None, [_P]),
    "frq_set_stream": (_I, [_P, _P]),
    "frq_get_stream": (_P, [_P]),
    "frq_sync": (_I, [_P]),
    "frq_upload_i8": (_P, [_P, _P, _P, _S, _S]),
    "frq_upload_i8_bundle": (_P, [_P, _P, _P, _S, _S]),
    "frq_upload_i4": (_P, [_P, _P, _P, _S, _S, _S]),
    "frq_upload_rows": (_P, [_P, _I, _P, _P, _S, _S]),
    "frq_w_free": (None, [_P]),
    "frq_w_info": (_I, [_P, _P, _P, _P, _P]),
    "frq_mm": (_I, [_P, _P, _P, _S, _P]),
    "frq_mm_dev": (_I, [_P, _P, _P, _S, _P]),
    "frq_mm_exact_dev": (_I, [_P, _P, _P, _S, _P]),
    "frq_mm_rows_dev": (_I, [_P, _P, _P, _S, _P]),
    "frq_mm_dev_noalloc": (_I, [_P, _P, _P, _S, _P]),
    "frq_mm_i8_debug": (_I, [_P, _P, _P, _S, _P, _P, _P, _P, _P, _P]),
    "frq_quant_pitch": (_S, [_S]),
    "frq_quant_i8_dev": (_I, [_P, _P, _S, _S, _P, _P, _P, _P]),
    "frq_mm_i8_q_dev": (_I, [_P, _P, _P, _P, _P, _P, _S, _P]),
    "frq_mm_i8_acc_dev": (_I, [_P, _P, _P, _S, _P]),
    "frq_moe_upload_i8": (_P, [_P, _S, _S, _S, _I, _P, _P, _P, _P, _P, _P]),
    "frq_moe_upload": (_P, [_P, _I, _S, _S, _S, _I, _S, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "frq_moe_info": (_I, [_P, _P, _P, _P, _P, _P]),
    "frq_moe_free": (None, [_P]),
    "frq_moe": (_I, [_P, _P, _P, _S, _P, _S, _I, _P, _P]),
    "frq_moe_dev": (_I, [_P, _P, _P, _S, _P, _S, _I, _P, _P]),
    "frq_moe_route": (_I, [_P, _P, _S, _S, _S, _I, _P, _P, _P]),
    "frq_expert_mm": (_I, [_P, _P, _I, _S, _P, _S, _P]),
    "frq_rowdot_f32": (_I, [_P, _P, _P, _P]),
    "frq_rowdot_f32_dev": (_I, [_P, _P, _P, _P]),
    "frq_rowdot_f32_subset": (_I, [_P, _P, _P, _P, _S, _P]),
    "frq_rowdot_f32_subset_dev": (_I, [_P, _P, _P, _P, _S, _P]),
    "frq_bundle_open": (_I, [C.c_char_p, _P]),
    "frq_bundle_close": (None, [_P]),
    "frq_bundle_header": (_I, [_P, _P, _S, _P, _P, _P, _P]),
    "frq_bundle_array": (_I, [_P, C.c_char_p, _P, _S, _P, _P, _P, _P, _P]),
    "frq_bundle_weight": (_I, [_P, _P, C.c_char_p, _P]),
    "frq_bundle_moe": (_I, [_P, _P, C.c_char_p, _S, _I, _P]),
    "frq_upload_q4a": (_P, [_P, _P, _P, _P, _S, _S, _S]),
    "frq_gpt2_load": (_I, [_P, _P, _I, _P]),
    "frq_gpt2_free": (None, [_P]),
    "frq_gpt2_info": (_I, [_P, _P, _P, _P, _P, _P]),
    "frq_gpt2_set_graphs": (_I, [_P, _I]),
    "frq_gpt2_generate": (_I, [_P, _P, _P, _S, _S, _P, _P]),
    "frq_gpt2_predict": (_I, [_P, _P, _P, _S, _P, _P]),
    "frq_libm_f32": (_I, [_P, _I, _P, _S, _P]),
    "frq_seq_fold_f32": (_I, [_P, _P, _S, _S, C.c_float, _P]),
    "frq_gemma_load": (_I, [_P, _P, _I, _P]),
    "frq_rope_load": (_I, [_P, _P, _I, _P]),
    "frq_gemma_free": (None, [_P]),
    "frq_gemma_info": (_I, [_P, _P, _P, _P]),
    "frq_gemma_set_graphs": (_I, [_P, _I]),
    "frq_gemma_generate": (_I, [_P, _P, _P, _S, _S, _P, _P]),
    "frq_gemma_generate_batch": (_I, [_P, _P, _P, _S, _S, _S, _P, _P]),
    "frq_gemma_predict": (_I, [_P, _P, _P, _S, _P, _P]),
}


class FrqError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"frq error {code}: {msg}")
        self.code = code


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python fieldrun_amd/build.py` "
            "(the HIP library is the only implementation; there is no CPU fallback)")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


lib = _load()


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


def _check(rc: int):
    if rc != FRQ_OK:
        raise FrqError(rc, lib.frq_last_error().decode())


def device_count() -> int:
    return lib.frq_device_count()


def quant_pitch(k: int) -> int:
    return lib.frq_quant_pitch(k)


class Context:
    """One device, one stream, one workspace (frq_ctx)."""

    def __init__(self, device: int = 0):
        self.h = lib.frq_init(device)
        if not self.h:
            raise FrqError(FRQ_ERR_NODEV, lib.frq_last_error().decode())
        self.device = device

    def close(self):
        if self.h:
            lib.frq_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream_handle: int | None):
        _check(lib.frq_set_stream(self.h, stream_handle))

    def sync(self):
        _check(lib.frq_sync(self.h))

    def quant_dev(self, a_ptr: int, m: int, k: int, a8_ptr: int, sa_ptr: int, oidx_ptr: int,
                  oval_ptr: int):
        """Activation quant of the I8 arm on device pointers (a8 pitch quant_pitch(k))."""
        _check(lib.frq_quant_i8_dev(self.h, a_ptr, m, k, a8_ptr, sa_ptr, oidx_ptr, oval_ptr))

    # ---- uploads ----
    def upload_i8(self, wt_nk: np.ndarray, scale: np.ndarray) -> "Weight":
        wt_nk = np.ascontiguousarray(wt_nk, dtype=np.int8)
        scale = np.ascontiguousarray(scale, dtype=np.float32)
        n, k = wt_nk.shape
        h = lib.frq_upload_i8(self.h, _ptr(wt_nk), _ptr(scale), n, k)
        if not h:
            raise FrqError(FRQ_ERR_HIP, lib.frq_last_error().decode())
        return Weight(self, h, FRQ_DT_I8, n, k)

    def upload_i8_bundle(self, w_kn: np.ndarray, scale_f16: np.ndarray) -> "Weight":
        w_kn = np.ascontiguousarray(w_kn, dtype=np.int8)
        s = np.ascontiguousarray(scale_f16, dtype=np.float16).view(np.uint16)
        k, n = w_kn.shape
        h = lib.frq_upload_i8_bundle(self.h, _ptr(w_kn), _ptr(s), k, n)
        if not h:
            raise FrqError(FRQ_ERR_HIP, lib.frq_last_error().decode())
        return Weight(self, h, FRQ_DT_I8, n, k)

    def upload_i4(self, packed: np.ndarray, scale_f16: np.ndarray, k: int, g: int) -> "Weight":
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        s = np.ascontiguousarray(scale_f16, dtype=np.float16).view(np.uint16)
        n = packed.shape[0]
        h = lib.frq_upload_i4(self.h, _ptr(packed), _ptr(s), n, k, g)
        if not h:
            raise FrqError(FRQ_ERR_HIP, lib.frq_last_error().decode())
        return Weight(self, h, FRQ_DT_I4, n, k, g)

    def upload_q4a(self, packed: np.ndarray, scale_f16: np.ndarray, min_f16: np.ndarray, k: int,
                   g: int) -> "Weight":
        """Affine int4: packed (N, ceil(K/2)) unsigned nibbles, f16 scale and
        min (N, ceil(K/g)); w = scale*q + min."""
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        s = np.ascontiguousarray(scale_f16, dtype=np.float16).view(np.uint16)
        mn = np.ascontiguousarray(min_f16, dtype=np.float16).view(np.uint16)
        n = packed.shape[0]
        h = lib.frq_upload_q4a(self.h, _ptr(packed), _ptr(s), _ptr(mn), n, k, g)
        if not h:
            raise FrqError(FRQ_ERR_HIP, lib.frq_last_error().decode())
        return Weight(self, h, FRQ_DT_Q4A, n, k, g)

    def upload_rows(self, kind: str, data: np.ndarray, scale: np.ndarray | None = None) -> "RowTable":
        """A row-major (rows, d) embedding table for rowdot_f32: kind 'f32'
        (float32 data), 'f16' (float16 data) or 'rowi8' (int8 data plus the
        f32 row scale, the upcast `__scale` sibling)."""
        if kind == "f32":
            dt, data = FRQ_DT_F32, np.ascontiguousarray(data, dtype=np.float32)
        elif kind == "f16":
            dt, data = FRQ_DT_F16, np.ascontiguousarray(data, dtype=np.float16).view(np.uint16)
        elif kind == "rowi8":
            dt, data = FRQ_DT_ROWI8, np.ascontiguousarray(data, dtype=np.int8)
        else:
            raise FrqError(FRQ_ERR_DTYPE, f"unknown row table kind {kind!r}")
        sc = None if scale is None else np.ascontiguousarray(scale, dtype=np.float32)
        rows, d = data.shape
        h = lib.frq_upload_rows(self.h, dt, _ptr(data), _ptr(sc), rows, d)
        if not h:
            raise FrqError(FRQ_ERR_ARG, lib.frq_last_error().decode())
        return RowTable(self, h, dt, rows, d)

    def upload_moe_i8(self, gate, gate_scale, up, up_scale, down, down_scale,
                      act: int = FRQ_ACT_SILU) -> "MoeBank":
        """Lists over experts of (in,out) int8 arrays and f32 [out] scales."""
        E = len(gate)
        d, gw = gate[0].shape
        mi = down[0].shape[0]
        keep = []

        def arr(lst, dt):
            ptrs = (C.c_void_p * E)()
            for i, a in enumerate(lst):
                a = np.ascontiguousarray(a, dtype=dt)
                keep.append(a)
                ptrs[i] = a.ctypes.data
            return ptrs

        g_p, gs_p = arr(gate, np.int8), arr(gate_scale, np.float32)
        d_p, ds_p = arr(down, np.int8), arr(down_scale, np.float32)
        if act == FRQ_ACT_SILU:
            u_p, us_p = arr(up, np.int8), arr(up_scale, np.float32)
        else:
            u_p = us_p = None
        h = lib.frq_moe_upload_i8(self.h, E, d, mi, act, g_p, gs_p, u_p, us_p, d_p, ds_p)
        if not h:
            raise FrqError(FRQ_ERR_HIP, lib.frq_last_error().decode())
        return MoeBank(self, h, E, d, mi, act)

    def upload_moe(self, dtype: str, d: int, mi: int, gate, down, up=None, gate_scale=None, up_scale=None,
                   down_scale=None, gate_min=None, up_min=None, down_min=None, act: int = FRQ_ACT_SILU,
                   g: int = 0) -> "MoeBank":
        """An expert bank in the dtype its bundle stores (frq_moe_upload):
        lists over experts of the stored arrays.  'i8': (in, out) int8 with
        f16-bit [out] scales; 'i4' / 'q4a': packed (out, ceil(in/2)) uint8 with
        f16-bit (out, ceil(in/g)) scales (and q4a mins); 'f16': (in, out)
        f16 bits; 'f32': (in, out) float32.  d / mi: the layer's widths."""
        code, raw_dt = {"i8": (FRQ_DT_I8, np.int8), "i4": (FRQ_DT_I4, np.uint8), "q4a": (FRQ_DT_Q4A, np.uint8),
                        "f16": (FRQ_DT_F16, np.uint16), "f32": (FRQ_DT_F32, np.float32)}[dtype]
        E = len(gate)
        keep = []

        def arr(lst, dt):
            if lst is None:
                return None
            ptrs = (C.c_void_p * E)()
            for i, a in enumerate(lst):
                a = np.ascontiguousarray(a, dtype=dt)
                keep.append(a)
                ptrs[i] = a.ctypes.data
            return ptrs

        silu = act == FRQ_ACT_SILU
        h = lib.frq_moe_upload(self.h, code, E, d, mi, act, g, arr(gate, raw_dt), arr(gate_scale, np.uint16),
                               arr(gate_min, np.uint16), arr(up, raw_dt) if silu else None,
                               arr(up_scale, np.uint16) if silu else None, arr(up_min, np.uint16) if silu else None,
                               arr(down, raw_dt), arr(down_scale, np.uint16), arr(down_min, np.uint16))
        if not h:
            raise FrqError(FRQ_ERR_ARG, lib.frq_last_error().decode())
        return MoeBank(self, h, E, d, mi, act)

    def moe_route(self, logits: np.ndarray, topk: int, norm_topk: bool = True,
                  per_expert_scale: np.ndarray | None = None):
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        T, E = logits.shape
        sel = np.empty((T, topk), np.int32)
        w = np.empty((T, topk), np.float32)
        pes = None if per_expert_scale is None else np.ascontiguousarray(per_expert_scale, np.float32)
        _check(lib.frq_moe_route(self.h, _ptr(logits), T, E, topk, int(norm_topk), _ptr(pes),
                                 _ptr(sel), _ptr(w)))
        return sel, w


class Weight:
    """A weight resident in HBM (frq_w)."""

    def __init__(self, ctx: Context, h, dtype: int, n: int, k: int, g: int = 0):
        self.ctx, self.h, self.dtype, self.n, self.k, self.g = ctx, h, dtype, n, k, g

    def free(self):
        if self.h:
            lib.frq_w_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def mm(self, a: np.ndarray) -> np.ndarray:
        """Bundle::mm: (M,K) f32 -> (M,N) f32."""
        a = np.ascontiguousarray(a, dtype=np.float32)
        if a.ndim != 2 or a.shape[1] != self.k:
            raise FrqError(FRQ_ERR_ARG, f"activation shape {a.shape} does not match K={self.k}")
        out = np.empty((a.shape[0], self.n), np.float32)
        _check(lib.frq_mm(self.ctx.h, self.h, _ptr(a), a.shape[0], _ptr(out)))
        return out

    def mm_dev(self, a_ptr: int, m: int, out_ptr: int):
        """Device-pointer variant, enqueued on the context stream."""
        _check(lib.frq_mm_dev(self.ctx.h, self.h, a_ptr, m, out_ptr))

    def mm_exact_dev(self, a_ptr: int, m: int, out_ptr: int):
        """Bundle::mm bit-identical to the reference's order at any M
        (frq_mm_exact_dev), enqueued on the context stream."""
        _check(lib.frq_mm_exact_dev(self.ctx.h, self.h, a_ptr, m, out_ptr))

    def mm_rows_dev(self, a_ptr: int, m: int, out_ptr: int):
        """m independent rows, each bit-identical to Bundle::mm at M == 1
        (frq_mm_rows_dev), enqueued on the context stream."""
        _check(lib.frq_mm_rows_dev(self.ctx.h, self.h, a_ptr, m, out_ptr))

    def mm_rows(self, a: np.ndarray) -> np.ndarray:
        """mm_rows_dev on host arrays: (M,K) f32 -> (M,N) f32."""
        from . import hip
        a = np.ascontiguousarray(a, dtype=np.float32)
        if a.ndim != 2 or a.shape[1] != self.k:
            raise FrqError(FRQ_ERR_ARG, f"activation shape {a.shape} does not match K={self.k}")
        da = hip.DeviceArray.from_numpy(a)
        do = hip.DeviceArray((a.shape[0], self.n), np.float32)
        try:
            self.mm_rows_dev(da.ptr, a.shape[0], do.ptr)
            self.ctx.sync()
            return do.numpy()
        finally:
            da.free()
            do.free()

    def mm_exact(self, a: np.ndarray) -> np.ndarray:
        """mm_exact_dev on host arrays: (M,K) f32 -> (M,N) f32."""
        from . import hip
        a = np.ascontiguousarray(a, dtype=np.float32)
        if a.ndim != 2 or a.shape[1] != self.k:
            raise FrqError(FRQ_ERR_ARG, f"activation shape {a.shape} does not match K={self.k}")
        da = hip.DeviceArray.from_numpy(a)
        do = hip.DeviceArray((a.shape[0], self.n), np.float32)
        try:
            self.mm_exact_dev(da.ptr, a.shape[0], do.ptr)
            self.ctx.sync()
            return do.numpy()
        finally:
            da.free()
            do.free()

    def mm_dev_noalloc(self, a_ptr: int, m: int, out_ptr: int):
        """mm_dev with no device allocation: the scratch is the library's
        static per-GPU array (frq_mm_dev_noalloc; shared by every call on
        the GPU, so overlapping calls race)."""
        _check(lib.frq_mm_dev_noalloc(self.ctx.h, self.h, a_ptr, m, out_ptr))

    def mm_q_dev(self, a8_ptr: int, sa_ptr: int, oidx_ptr: int, oval_ptr: int, m: int, out_ptr: int):
        """int8 dot + epilogue on a batch quantised by Context.quant_dev."""
        _check(lib.frq_mm_i8_q_dev(self.ctx.h, self.h, a8_ptr, sa_ptr, oidx_ptr, oval_ptr, m, out_ptr))

    def mm_acc_dev(self, a8_ptr: int, m: int, acc_ptr: int):
        """int8: the i32 sums alone (the exact path's GEMM at m > 16) on a
        batch quantised by Context.quant_dev."""
        _check(lib.frq_mm_i8_acc_dev(self.ctx.h, self.h, a8_ptr, m, acc_ptr))

    def mm_debug(self, a: np.ndarray):
        """int8: (out, acc, a8, sa, oidx, oval) — the reference's locals."""
        a = np.ascontiguousarray(a, dtype=np.float32)
        m = a.shape[0]
        out = np.empty((m, self.n), np.float32)
        acc = np.empty((m, self.n), np.int32)
        a8 = np.empty((m, self.k), np.int8)
        sa = np.empty(m, np.float32)
        oi = np.empty((m, 32), np.uint32)
        ov = np.empty((m, 32), np.float32)
        _check(lib.frq_mm_i8_debug(self.ctx.h, self.h, _ptr(a), m, _ptr(out), _ptr(acc),
                                   _ptr(a8), _ptr(sa), _ptr(oi), _ptr(ov)))
        return out, acc, a8, sa, oi, ov


class RowTable(Weight):
    """A row-major embedding / unembedding table resident in HBM (frq_w)."""

    def rowdot_f32(self, x: np.ndarray) -> np.ndarray:
        """Bundle::rowdot_f32: out[r] = dot(W[r], x) for every row."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        if x.shape[0] != self.k:
            raise FrqError(FRQ_ERR_ARG, f"x has {x.shape[0]} entries, the rows {self.k}")
        out = np.empty(self.n, np.float32)
        _check(lib.frq_rowdot_f32(self.ctx.h, self.h, _ptr(x), _ptr(out)))
        return out

    def rowdot_f32_dev(self, x_ptr: int, out_ptr: int):
        _check(lib.frq_rowdot_f32_dev(self.ctx.h, self.h, x_ptr, out_ptr))

    def rowdot_f32_subset(self, x: np.ndarray, cand) -> np.ndarray:
        """Bundle::rowdot_f32_subset: out[i] = dot(W[cand[i]], x); ids outside
        [0, rows) score -inf."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        if x.shape[0] != self.k:
            raise FrqError(FRQ_ERR_ARG, f"x has {x.shape[0]} entries, the rows {self.k}")
        cand = np.ascontiguousarray(cand, dtype=np.int64).reshape(-1)
        out = np.empty(cand.shape[0], np.float32)
        _check(lib.frq_rowdot_f32_subset(self.ctx.h, self.h, _ptr(x), _ptr(cand), cand.shape[0], _ptr(out)))
        return out

    def rowdot_f32_subset_dev(self, x_ptr: int, cand_ptr: int, ncand: int, out_ptr: int):
        _check(lib.frq_rowdot_f32_subset_dev(self.ctx.h, self.h, x_ptr, cand_ptr, ncand, out_ptr))


class MoeBank:
    """All routed experts of one layer, resident in HBM (frq_moe_w)."""

    def __init__(self, ctx, h, E, d, mi, act):
        self.ctx, self.h, self.E, self.d, self.mi, self.act = ctx, h, E, d, mi, act
        dt, g = C.c_int(), C.c_size_t()
        _check(lib.frq_moe_info(h, C.byref(dt), None, None, None, C.byref(g)))
        self.dtype, self.g = dt.value, g.value

    def free(self):
        if self.h:
            lib.frq_moe_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def forward(self, x: np.ndarray, logits: np.ndarray, topk: int, norm_topk: bool = True,
                per_expert_scale: np.ndarray | None = None) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        T = x.shape[0]
        out = np.empty((T, self.d), np.float32)
        pes = None if per_expert_scale is None else np.ascontiguousarray(per_expert_scale, np.float32)
        _check(lib.frq_moe(self.ctx.h, self.h, _ptr(x), T, _ptr(logits), topk, int(norm_topk),
                           _ptr(pes), _ptr(out)))
        return out

    def forward_dev(self, x_ptr, T, logits_ptr, topk, norm_topk, pes_ptr, out_ptr):
        _check(lib.frq_moe_dev(self.ctx.h, self.h, x_ptr, T, logits_ptr, topk, int(norm_topk),
                               pes_ptr, out_ptr))

    def expert_mm(self, which: int, e: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out_dim = {0: self.mi if self.act == FRQ_ACT_SILU else 2 * self.mi, 1: self.mi, 2: self.d}[which]
        y = np.empty((x.shape[0], out_dim), np.float32)
        _check(lib.frq_expert_mm(self.ctx.h, self.h, which, e, _ptr(x), x.shape[0], _ptr(y)))
        return y


class Bundle:
    """A fieldrun bundle (<stem>.fieldrun.json + .fieldrun.bin) opened by the
    library's reader (Bundle::load, src/bundle.rs:314-376).  Arrays are views
    of the mapped blob; mm / rowdot_f32 upload a weight on first use onto the
    context's device (the resident set of the GPU path) and call the
    kernels."""

    def __init__(self, stem: str, ctx: "Context | None" = None):
        self.h = None
        out = C.c_void_p()
        _check(lib.frq_bundle_open(os.fspath(stem).encode(), C.byref(out)))
        self.h = out.value
        self.ctx = ctx
        self._dev = {}
        arch = C.create_string_buffer(64)
        nc, nf = C.c_size_t(0), C.c_size_t(0)
        _check(lib.frq_bundle_header(self.h, arch, 64, None, C.byref(nc), None, C.byref(nf)))
        cfg = (C.c_int64 * max(nc.value, 1))()
        cff = (C.c_double * max(nf.value, 1))()
        _check(lib.frq_bundle_header(self.h, arch, 64, cfg, C.byref(nc), cff, C.byref(nf)))
        self.arch = arch.value.decode()
        self.config = [int(cfg[i]) for i in range(nc.value)]
        self.config_f = [float(cff[i]) for i in range(nf.value)]

    @classmethod
    def load(cls, stem: str, ctx: "Context | None" = None) -> "Bundle":
        return cls(stem, ctx)

    def close(self):
        for w in self._dev.values():
            w.free()
        self._dev = {}
        if self.h:
            lib.frq_bundle_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self, name: str):
        """(dtype, shape, group, nbytes) of a stored array."""
        dt = C.create_string_buffer(16)
        shape = (C.c_size_t * 8)()
        nd, grp, data, nb = C.c_size_t(8), C.c_size_t(0), C.c_void_p(), C.c_size_t(0)
        _check(lib.frq_bundle_array(self.h, name.encode(), dt, 16, shape, C.byref(nd), C.byref(grp),
                                    C.byref(data), C.byref(nb)))
        return dt.value.decode(), tuple(shape[i] for i in range(nd.value)), grp.value, nb.value

    def arr(self, name: str) -> np.ndarray:
        """The stored bytes of an array as a read-only numpy view in its stored
        type (f32, f16 bits as float16, i8 / rowi8 as int8, i4 / q4a packed
        bytes as uint8)."""
        dt, shape, _, nb = self.info(name)
        data = C.c_void_p()
        nd = C.c_size_t(0)
        _check(lib.frq_bundle_array(self.h, name.encode(), None, 0, None, C.byref(nd), None, C.byref(data), None))
        np_dt = {"f32": np.float32, "f16": np.float16, "i8": np.int8, "rowi8": np.int8}.get(dt, np.uint8)
        if nb == 0:
            return np.zeros(shape if np_dt is not np.uint8 else (0,), np_dt)
        buf = (C.c_uint8 * nb).from_address(data.value)
        a = np.frombuffer(buf, np.uint8).view(np_dt)
        if dt in ("i4", "q4a"):
            a = a.reshape(shape[0], -1)
        else:
            a = a.reshape(shape)
        a.flags.writeable = False
        return a

    def dims(self, name: str):
        """Bundle::dims: the logical (rows, cols) of a 2-D array."""
        _, shape, _, _ = self.info(name)
        return shape[0], shape[1]

    def weight(self, name: str):
        """The device copy of an array (uploaded once, owned by the bundle)."""
        if name not in self._dev:
            if self.ctx is None:
                raise FrqError(FRQ_ERR_ARG, "this bundle was opened without a device context")
            out = C.c_void_p()
            _check(lib.frq_bundle_weight(self.ctx.h, self.h, name.encode(), C.byref(out)))
            h = out.value
            dtype, n, k, g = C.c_int(0), C.c_size_t(0), C.c_size_t(0), C.c_size_t(0)
            _check(lib.frq_w_info(h, C.byref(dtype), C.byref(n), C.byref(k), C.byref(g)))
            cls = RowTable if dtype.value in (FRQ_DT_F32, FRQ_DT_F16, FRQ_DT_ROWI8) else Weight
            self._dev[name] = cls(self.ctx, h, dtype.value, n.value, k.value, g.value)
        return self._dev[name]

    def mm(self, a: np.ndarray, name: str) -> np.ndarray:
        """Bundle::mm(a, name) for an i8 / i4 linear, on the device."""
        return self.weight(name).mm(a)

    def rowdot_f32(self, name: str, x: np.ndarray) -> np.ndarray:
        """Bundle::rowdot_f32(name, x) over an f32 / f16 / rowi8 table."""
        return self.weight(name).rowdot_f32(x)

    def rowdot_f32_subset(self, name: str, x: np.ndarray, cand) -> np.ndarray:
        return self.weight(name).rowdot_f32_subset(x, cand)

    def moe(self, prefix: str, n_exp: int, act: int = FRQ_ACT_SILU) -> "MoeBank":
        """The routed expert bank of one MoE layer ({prefix}experts.{e}.*)."""
        if self.ctx is None:
            raise FrqError(FRQ_ERR_ARG, "this bundle was opened without a device context")
        out = C.c_void_p()
        _check(lib.frq_bundle_moe(self.ctx.h, self.h, prefix.encode(), n_exp, act, C.byref(out)))
        h = out.value
        d, mi = C.c_size_t(), C.c_size_t()
        _check(lib.frq_moe_info(h, None, None, C.byref(d), C.byref(mi), None))
        return MoeBank(self.ctx, h, n_exp, d.value, mi.value, act)


class Gpt2:
    """Gpt2 of src/composition.rs on the device: Gpt2::new over an arch
    "gpt2" bundle (52-56), Model::generate (317-341; kv_int8: the int8
    cache, 251-270) and Model::predict (304-308), every step resident in
    HBM.  `bundle` is a Bundle opened with this context."""

    def __init__(self, bundle: "Bundle", kv_int8: bool = False, ctx: "Context | None" = None):
        self.ctx = ctx or bundle.ctx
        if self.ctx is None:
            raise FrqError(FRQ_ERR_ARG, "this bundle was opened without a device context")
        self.h = None
        out = C.c_void_p()
        _check(lib.frq_gpt2_load(self.ctx.h, bundle.h, int(kv_int8), C.byref(out)))
        self.h = out.value
        dims = [C.c_size_t(0) for _ in range(5)]
        _check(lib.frq_gpt2_info(self.h, *[C.byref(v) for v in dims]))
        self.n_layer, self.n_head, self.d, self.n_pos, self.vocab = (v.value for v in dims)
        self.kv_int8 = bool(kv_int8)

    def free(self):
        if self.h:
            lib.frq_gpt2_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def set_graphs(self, on: bool):
        _check(lib.frq_gpt2_set_graphs(self.h, int(on)))

    def generate(self, prompt, n_new: int, with_logits: bool = False):
        prompt = np.ascontiguousarray(prompt, dtype=np.int64)
        out = np.empty(n_new, np.int64)
        lg = np.empty((n_new, self.vocab), np.float32) if with_logits else None
        _check(lib.frq_gpt2_generate(self.ctx.h, self.h, _ptr(prompt), len(prompt), n_new, _ptr(out),
                                     None if lg is None else _ptr(lg)))
        return (out, lg) if with_logits else out

    def predict(self, ids, with_logits: bool = False):
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        tok = np.zeros(1, np.int64)
        lg = np.empty(self.vocab, np.float32) if with_logits else None
        _check(lib.frq_gpt2_predict(self.ctx.h, self.h, _ptr(ids), len(ids), _ptr(tok),
                                    None if lg is None else _ptr(lg)))
        return (int(tok[0]), lg) if with_logits else int(tok[0])


def seq_fold_f32(ctx: "Context", x: np.ndarray, init: float = -0.0) -> np.ndarray:
    """out[r] = init + x[r, 0] + ... + x[r, n-1] in f32 index order (the
    reference's iterator sum), by the device's speculative segmented fold
    (frq_seq_fold_f32, the decode kernels' RMSNorm and softmax sums)."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    out = np.empty(x.shape[0], np.float32)
    _check(lib.frq_seq_fold_f32(ctx.h, _ptr(x), x.shape[0], x.shape[1], C.c_float(init), _ptr(out)))
    return out


LIBM_FNS = {"expf": 0, "expm1f": 1, "tanhf": 2, "expf_sel": 3}


def libm_f32(fn: str, x: np.ndarray, ctx: "Context | None" = None) -> np.ndarray:
    """The library's f32 expf / expm1f / tanhf (the libm algorithms the
    reference's f32::exp / f32::tanh reach), on ctx's device or the host."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    _check(lib.frq_libm_f32(None if ctx is None else ctx.h, LIBM_FNS[fn], _ptr(x), x.size, _ptr(out)))
    return out


class Gemma:
    """Gemma of src/gemma.rs on the device: Gemma::new over an arch "gemma"
    bundle (52-60), Model::generate (403-431; kv_int8: 364-384) and
    Model::predict (436-441), every step resident in HBM."""

    _loader = "frq_gemma_load"

    def __init__(self, bundle: "Bundle", kv_int8: bool = False, ctx: "Context | None" = None):
        self.ctx = ctx or bundle.ctx
        if self.ctx is None:
            raise FrqError(FRQ_ERR_ARG, "this bundle was opened without a device context")
        self.h = None
        out = C.c_void_p()
        _check(getattr(lib, self._loader)(self.ctx.h, bundle.h, int(kv_int8), C.byref(out)))
        self.h = out.value
        dims = [C.c_size_t(0) for _ in range(3)]
        _check(lib.frq_gemma_info(self.h, *[C.byref(v) for v in dims]))
        self.n_layer, self.d, self.vocab = (v.value for v in dims)

    def free(self):
        if self.h:
            lib.frq_gemma_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def set_graphs(self, on: bool):
        _check(lib.frq_gemma_set_graphs(self.h, int(on)))

    def generate(self, prompt, n_new: int, with_logits: bool = False):
        prompt = np.ascontiguousarray(prompt, dtype=np.int64)
        out = np.empty(n_new, np.int64)
        lg = np.empty((n_new, self.vocab), np.float32) if with_logits else None
        _check(lib.frq_gemma_generate(self.ctx.h, self.h, _ptr(prompt), len(prompt), n_new, _ptr(out),
                                      None if lg is None else _ptr(lg)))
        return (out, lg) if with_logits else out

    def generate_batch(self, prompts, n_new: int, with_logits: bool = False):
        """Each row of prompts (nb, n_prompt) its own generate, the decode
        steps of all rows together: tokens (nb, n_new) [and logits (nb,
        n_new, vocab)] as nb calls of generate give them."""
        prompts = np.ascontiguousarray(np.atleast_2d(prompts), dtype=np.int64)
        nb, n_prompt = prompts.shape
        out = np.empty((nb, n_new), np.int64)
        lg = np.empty((nb, n_new, self.vocab), np.float32) if with_logits else None
        _check(lib.frq_gemma_generate_batch(self.ctx.h, self.h, _ptr(prompts), nb, n_prompt, n_new, _ptr(out),
                                            None if lg is None else _ptr(lg)))
        return (out, lg) if with_logits else out

    def predict(self, ids, with_logits: bool = False):
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        tok = np.zeros(1, np.int64)
        lg = np.empty(self.vocab, np.float32) if with_logits else None
        _check(lib.frq_gemma_predict(self.ctx.h, self.h, _ptr(ids), len(ids), _ptr(tok),
                                     None if lg is None else _ptr(lg)))
        return (int(tok[0]), lg) if with_logits else int(tok[0])


class Rope(Gemma):
    """Rope of src/rope.rs (Llama / Qwen2.5 / Qwen3 / Mistral) on the device:
    Rope::new over an arch "rope" bundle (56-64), Model::generate
    (1147-1170) and predict (730-734), in the same engine as Gemma."""

    _loader = "frq_rope_load"
