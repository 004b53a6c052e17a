"""CPU oracle of fieldrun's quantised-linear hot path — TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package.  It wraps oracle/libfrq_oracle.so (built from
frq_oracle.c by oracle/Makefile), a C restatement of /root/reference
src/bundle.rs, src/convert.rs and the MoE branches of src/qwen3moe.rs /
src/gemma4.rs; each C function cites the reference lines it follows.  The
pinning status of each function is listed in frq_oracle.h.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libfrq_oracle.so")


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = C.CDLL(LIB_PATH)
    P, S, I, F = C.c_void_p, C.c_size_t, C.c_int, C.c_float
    sig = {
        "fro_f16_to_f32": (F, [C.c_uint16]),
        "fro_f32_to_f16": (C.c_uint16, [F]),
        "fro_f16_to_f32_n": (None, [P, P, S]),
        "fro_put_i8": (None, [P, S, S, I, P, P]),
        "fro_put_i4": (S, [P, S, S, I, P, P]),
        "fro_put_embed_i8": (None, [P, S, S, P, P]),
        "fro_i8_transpose": (None, [P, S, S, P]),
        "fro_i8dot": (C.c_int32, [P, P, S]),
        "fro_quant_row": (I, [P, S, P, P, P, P, P]),
        "fro_mm_i8": (I, [P, S, S, P, P, S, P, P]),
        "fro_mm_i8_mt": (I, [P, S, S, P, P, S, P, I]),
        "fro_i8dot_avx512bw": (C.c_int32, [P, P, S]),
        "fro_set_i8dot": (I, [I]),
        "fro_i4_dot": (F, [P, P, P, S, S]),
        "fro_i4_dot_avx2": (F, [P, P, P, S, S]),
        "fro_mm_i4": (I, [P, S, S, P, P, S, S, P]),
        "fro_expert_mm_i8": (None, [P, S, P, P, S, S, P]),
        "fro_expert_f32": (I, [P, S, S, P]),
        "fro_expert_mm": (I, [P, P, S, S, S, P]),
        "fro_moe_ex_mt": (I, [P, S, S, P, S, S, I, P, S, I, P, P, P, P, I]),
        "fro_mm_dot": (F, [P, S, P, S, S]),
        "fro_sgemm": (None, [P, S, S, P, S, P]),
        "fro_silu": (F, [F]),
        "fro_gelu_tanh": (F, [F]),
        "fro_moe_route": (None, [P, S, S, S, I, P, P, P, P]),
        "fro_moe": (I, [P, S, S, P, S, S, I, P, S, I, P, P, P, P, P, P, P]),
        "fro_moe_mt": (I, [P, S, S, P, S, S, I, P, S, I, P, P, P, P, P, P, P, I]),
        "fro_rowdot_f32": (None, [I, P, P, S, S, P, P]),
        "fro_rowdot_f32_subset": (None, [I, P, P, S, S, P, P, S, P]),
        "fro_layernorm": (None, [P, S, S, P, P, P]),
        "fro_nd_sum": (F, [P, S]),
        "fro_libm_f32": (None, [I, P, S, P]),
        "fro_put_q4a": (S, [P, S, S, I, P, P, P]),
        "fro_q4a_dot": (F, [P, P, P, P, S, S]),
        "fro_q4a_dot_avx2": (F, [P, P, P, P, S, S]),
        "fro_mm_q4a": (I, [P, S, S, P, P, P, S, S, P]),
        "fro_mm_i4_mt": (I, [P, S, S, P, P, S, S, P, I]),
        "fro_rmsnorm": (None, [P, S, S, P, F, P]),
        "fro_gemma_generate": (I, [P, P, S, S, I, I, P, P]),
        "fro_gpt2_generate": (I, [P, P, S, S, I, I, P, P]),
        "fro_gpt2_predict": (I, [P, P, S, I, P, P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


lib = _load()


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


class OracleNaN(RuntimeError):
    """The reference panics (partial_cmp().unwrap()) on this input."""


# ---- f16 ----
def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib.fro_f16_to_f32_n(_p(h), _p(out), h.size)
    return out


def f32_to_f16_bits(x: float) -> int:
    return int(lib.fro_f32_to_f16(float(x)))


# ---- quantisers (src/convert.rs) ----
def put_i8(data: np.ndarray, transpose: bool):
    """-> (w (in,out) int8, scale f16 bits [out] uint16)."""
    data = _c(data, np.float32)
    rows, cols = data.shape
    out, inp = (rows, cols) if transpose else (cols, rows)
    w = np.empty((inp, out), np.int8)
    s = np.empty(out, np.uint16)
    lib.fro_put_i8(_p(data), rows, cols, int(transpose), _p(w), _p(s))
    return w, s


def put_i4(data: np.ndarray, transpose: bool):
    """-> (packed (out, ceil(in/2)) uint8, scale f16 bits (out, ng), g)."""
    data = _c(data, np.float32)
    rows, cols = data.shape
    out, inp = (rows, cols) if transpose else (cols, rows)
    g = min(32, max(inp, 1))
    ng = (inp + g - 1) // g
    packed = np.empty((out, (inp + 1) // 2), np.uint8)
    s = np.empty((out, ng), np.uint16)
    g2 = lib.fro_put_i4(_p(data), rows, cols, int(transpose), _p(packed), _p(s))
    assert g2 == g
    return packed, s, g


def put_embed_i8(data: np.ndarray):
    data = _c(data, np.float32)
    v, d = data.shape
    q = np.empty((v, d), np.int8)
    s = np.empty(v, np.uint16)
    lib.fro_put_embed_i8(_p(data), v, d, _p(q), _p(s))
    return q, s


def i8_transpose(w_kn: np.ndarray) -> np.ndarray:
    w_kn = _c(w_kn, np.int8)
    k, n = w_kn.shape
    out = np.empty((n, k), np.int8)
    lib.fro_i8_transpose(_p(w_kn), k, n, _p(out))
    return out


# ---- int8 path (src/bundle.rs:688-756, 1036-1053) ----
def i8dot(a: np.ndarray, w: np.ndarray) -> int:
    a, w = _c(a, np.int8), _c(w, np.int8)
    return int(lib.fro_i8dot(_p(a), _p(w), a.size))


def quant_row(a: np.ndarray):
    """-> (a8, sa, oidx[:t], oval[:t]); raises OracleNaN like the reference."""
    a = _c(a, np.float32)
    k = a.size
    a8 = np.empty(k, np.int8)
    sa = C.c_float()
    oi = np.zeros(32, np.uint32)
    ov = np.zeros(32, np.float32)
    t = C.c_size_t()
    rc = lib.fro_quant_row(_p(a), k, _p(a8), C.byref(sa), _p(oi), _p(ov), C.byref(t))
    if rc:
        raise OracleNaN("NaN activation")
    return a8, np.float32(sa.value), oi[: t.value].copy(), ov[: t.value].copy()


def mm_i8(a: np.ndarray, wt_nk: np.ndarray, scale: np.ndarray, with_acc: bool = False):
    a = _c(a, np.float32)
    wt_nk, scale = _c(wt_nk, np.int8), _c(scale, np.float32)
    m, k = a.shape
    n = wt_nk.shape[0]
    out = np.empty((m, n), np.float32)
    acc = np.empty((m, n), np.int32) if with_acc else None
    rc = lib.fro_mm_i8(_p(a), m, k, _p(wt_nk), _p(scale), n, _p(out), _p(acc))
    if rc:
        raise OracleNaN("NaN activation")
    return (out, acc) if with_acc else out


def set_i8dot(variant: str) -> bool:
    """The i8 dot of the oracle's int8 linears: "scalar" (the reference's
    `_scalar_i8_bench` build; default) or "avx512bw" (i8dot_avx512bw, the
    production x86 dispatch).  False when the host lacks AVX-512BW."""
    return bool(lib.fro_set_i8dot({"scalar": 0, "avx512bw": 1}[variant]))


def i8dot_avx512bw(a: np.ndarray, w: np.ndarray) -> int:
    a, w = _c(a, np.int8), _c(w, np.int8)
    return int(lib.fro_i8dot_avx512bw(_p(a), _p(w), a.size))


def mm_i8_mt(a, wt_nk, scale, nthreads: int):
    a = _c(a, np.float32)
    wt_nk, scale = _c(wt_nk, np.int8), _c(scale, np.float32)
    m, k = a.shape
    n = wt_nk.shape[0]
    out = np.empty((m, n), np.float32)
    rc = lib.fro_mm_i8_mt(_p(a), m, k, _p(wt_nk), _p(scale), n, _p(out), int(nthreads))
    if rc:
        raise OracleNaN("NaN activation")
    return out


# ---- int4 path (src/bundle.rs:90-113, 199-225, 760-799) ----
def i4_dot(prow, a, scale, g, k):
    prow, a, scale = _c(prow, np.uint8), _c(a, np.float32), _c(scale, np.float32)
    return np.float32(lib.fro_i4_dot(_p(prow), _p(a), _p(scale), g, k))


def i4_dot_avx2(prow, a, scale, g, k):
    prow, a, scale = _c(prow, np.uint8), _c(a, np.float32), _c(scale, np.float32)
    return np.float32(lib.fro_i4_dot_avx2(_p(prow), _p(a), _p(scale), g, k))


def mm_i4(a, packed, scale_f32, k, g):
    a = _c(a, np.float32)
    packed, scale_f32 = _c(packed, np.uint8), _c(scale_f32, np.float32)
    m = a.shape[0]
    n = packed.shape[0]
    out = np.empty((m, n), np.float32)
    lib.fro_mm_i4(_p(a), m, k, _p(packed), _p(scale_f32), n, g, _p(out))
    return out


# ---- experts / MoE (src/bundle.rs:404-461, src/qwen3moe.rs:120-158) ----
def expert_mm_i8(x, raw_in_out, scale):
    x, raw_in_out, scale = _c(x, np.float32), _c(raw_in_out, np.int8), _c(scale, np.float32)
    m = x.shape[0]
    inp, out = raw_in_out.shape
    y = np.empty((m, out), np.float32)
    lib.fro_expert_mm_i8(_p(x), m, _p(raw_in_out), _p(scale), inp, out, _p(y))
    return y


class _Expert(C.Structure):
    _fields_ = [("dtype", C.c_int), ("raw", C.c_void_p), ("scale", C.c_void_p), ("mins", C.c_void_p),
                ("g", C.c_size_t)]


EXPERT_DTYPES = {"i8": 1, "i4": 2, "f32": 3, "f16": 4, "q4a": 6}


def expert(dtype, raw, scale=None, mins=None, g=0, inp=None, out=None):
    """One stored expert weight (fro_expert_t) as a dict:
    i8  raw (in,out) int8, scale f32 [out];
    i4  raw (out, ceil(in/2)) uint8 nibbles, scale f32 (out, ceil(in/g)), g, inp;
    q4a as i4 plus mins f32 (out, ceil(in/g));
    f16 raw (in,out) uint16 f16 bits;  f32 raw (in,out) float32."""
    if dtype in ("i8", "f16", "f32"):
        dt = {"i8": np.int8, "f16": np.uint16, "f32": np.float32}[dtype]
        raw = _c(raw, dt)
        inp, out = raw.shape
    else:
        raw = _c(raw, np.uint8)
        out = raw.shape[0]
        assert inp is not None and g > 0
    return {"dtype": dtype, "raw": raw, "scale": None if scale is None else _c(scale, np.float32),
            "mins": None if mins is None else _c(mins, np.float32), "g": int(g), "inp": int(inp), "out": int(out)}


def _ex_struct(e):
    return _Expert(EXPERT_DTYPES[e["dtype"]], e["raw"].ctypes.data, None if e["scale"] is None else e["scale"].ctypes.data,
                   None if e["mins"] is None else e["mins"].ctypes.data, e["g"])


def expert_f32(e):
    """expert_f32 (src/bundle.rs:404-454): the weight as f32 (in, out)."""
    v = np.empty((e["inp"], e["out"]), np.float32)
    st = _ex_struct(e)
    if lib.fro_expert_f32(C.byref(st), e["inp"], e["out"], _p(v)) != 0:
        raise ValueError(f"expert dtype {e['dtype']!r} unsupported")
    return v


def expert_mm(x, e):
    """expert_mm (src/bundle.rs:457-461): x (m, in) . expert_f32."""
    x = _c(x, np.float32)
    m = x.shape[0]
    y = np.empty((m, e["out"]), np.float32)
    st = _ex_struct(e)
    if lib.fro_expert_mm(C.byref(st), _p(x), m, e["inp"], e["out"], _p(y)) != 0:
        raise ValueError(f"expert dtype {e['dtype']!r} unsupported")
    return y


def mm_dot(x, w):
    """One element of a.dot: matrixmultiply 0.3.10's order over k (fro_mm_dot)."""
    x, w = _c(x, np.float32), _c(w, np.float32)
    return float(lib.fro_mm_dot(_p(x), 1, _p(w), 1, x.size))


def moe_ex(x, logits, topk, norm_topk, gate, up, down, act=0, per_expert_scale=None, nthreads: int = 1):
    """The routed expert layer over experts of any stored dtype (lists of
    expert() dicts; up unused for act 1): fro_moe_ex_mt."""
    x, logits = _c(x, np.float32), _c(logits, np.float32)
    T, d = x.shape
    E = logits.shape[1]
    mi = down[0]["inp"]
    arr = lambda lst: (_Expert * E)(*[_ex_struct(e) for e in lst])  # noqa: E731
    g_, d_ = arr(gate), arr(down)
    u_ = arr(up) if act == 0 else None
    pes = None if per_expert_scale is None else _c(per_expert_scale, np.float32)
    out = np.empty((T, d), np.float32)
    rc = lib.fro_moe_ex_mt(_p(x), T, d, _p(logits), E, topk, int(norm_topk), _p(pes), mi, act, g_, u_, d_, _p(out),
                           int(nthreads))
    if rc != 0:
        raise ValueError("unsupported expert dtype")
    return out


def silu(x: float) -> float:
    return float(lib.fro_silu(float(x)))


def gelu_tanh(x: float) -> float:
    return float(lib.fro_gelu_tanh(float(x)))


def moe_route(logits, topk, norm_topk=True, per_expert_scale=None):
    logits = _c(logits, np.float32)
    T, E = logits.shape
    sel = np.empty((T, topk), np.int32)
    w = np.empty((T, topk), np.float32)
    probs = np.empty((T, E), np.float32)
    pes = None if per_expert_scale is None else _c(per_expert_scale, np.float32)
    lib.fro_moe_route(_p(logits), T, E, topk, int(norm_topk), _p(pes), _p(sel), _p(w), _p(probs))
    return sel, w, probs


def moe(x, logits, topk, norm_topk, gate, gate_scale, up, up_scale, down, down_scale,
        act=0, per_expert_scale=None, nthreads: int = 1):
    """The routed expert layer (fro_moe; fro_moe_mt when nthreads > 1, the
    same output: experts' matmuls in parallel, one ascending-id combine)."""
    x, logits = _c(x, np.float32), _c(logits, np.float32)
    T, d = x.shape
    E = logits.shape[1]
    mi = down[0].shape[0]
    keep = []

    def arr(lst, dt):
        ptrs = (C.c_void_p * E)()
        for i, a in enumerate(lst):
            a = _c(a, dt)
            keep.append(a)
            ptrs[i] = a.ctypes.data
        return ptrs

    gp, gsp = arr(gate, np.int8), arr(gate_scale, np.float32)
    dp, dsp = arr(down, np.int8), arr(down_scale, np.float32)
    if act == 0:
        up_, usp = arr(up, np.int8), arr(up_scale, np.float32)
    else:
        up_ = usp = None
    pes = None if per_expert_scale is None else _c(per_expert_scale, np.float32)
    out = np.empty((T, d), np.float32)
    if nthreads > 1:
        lib.fro_moe_mt(_p(x), T, d, _p(logits), E, topk, int(norm_topk), _p(pes), mi, act,
                       gp, gsp, up_, usp, dp, dsp, _p(out), int(nthreads))
    else:
        lib.fro_moe(_p(x), T, d, _p(logits), E, topk, int(norm_topk), _p(pes), mi, act,
                    gp, gsp, up_, usp, dp, dsp, _p(out))
    return out


# ---- the unembed row dot ----
ROW_DTYPES = {"f32": (3, np.float32), "f16": (4, np.uint16), "rowi8": (5, np.int8)}


def rowdot_f32(kind: str, data, x, scale=None):
    """Bundle::rowdot_f32 over a (rows, d) table; kind 'f32' (float data),
    'f16' (uint16 f16 bits) or 'rowi8' (int8 + f32 scale per row)."""
    code, dt = ROW_DTYPES[kind]
    data = _c(data, dt)
    rows, d = data.shape
    x = _c(x, np.float32)
    sc = _c(scale, np.float32) if scale is not None else None
    out = np.empty(rows, np.float32)
    lib.fro_rowdot_f32(code, _p(data), _p(sc), rows, d, _p(x), _p(out))
    return out


def rowdot_f32_subset(kind: str, data, x, cand, scale=None):
    """Bundle::rowdot_f32_subset: out[i] = dot(W[cand[i]], x), -inf for ids
    outside [0, rows)."""
    code, dt = ROW_DTYPES[kind]
    data = _c(data, dt)
    rows, d = data.shape
    x = _c(x, np.float32)
    cand = _c(cand, np.int64)
    sc = _c(scale, np.float32) if scale is not None else None
    out = np.empty(len(cand), np.float32)
    lib.fro_rowdot_f32_subset(code, _p(data), _p(sc), rows, d, _p(x), _p(cand), len(cand), _p(out))
    return out


# ---- GPT-2 with a KV cache (src/composition.rs) ----
def read_bundle(stem: str):
    """(manifest, {name: array}) of a fieldrun bundle, read with numpy from
    the manifest and a memory map of the blob (FORMAT.md v1): f32 / f16 /
    i8 / rowi8 arrays in their stored type and shape, i4 / q4a as packed
    uint8 rows.  Test-side: independent of the library's reader."""
    import json
    m = json.load(open(stem + ".fieldrun.json"))
    blob = np.memmap(stem + ".fieldrun.bin", np.uint8, "r")
    out = {}
    for a in m["arrays"]:
        dt = {"f32": np.float32, "f16": np.float16, "i8": np.int8, "rowi8": np.int8}.get(a.get("dtype", "f32"), np.uint8)
        raw = blob[a["offset"]:a["offset"] + a["bytes"]]
        v = np.frombuffer(raw, dt)
        out[a["name"]] = v.reshape(a["shape"]) if dt is not np.uint8 else v.reshape(a["shape"][0], -1)
    return m, out


class _Gpt2W(C.Structure):
    _fields_ = [("n_layer", C.c_size_t), ("n_head", C.c_size_t), ("d", C.c_size_t), ("n_pos", C.c_size_t),
                ("vocab", C.c_size_t), ("wte", C.c_void_p), ("wpe", C.c_void_p), ("ln_f_g", C.c_void_p),
                ("ln_f_b", C.c_void_p), ("ln_g", C.c_void_p), ("ln_b", C.c_void_p), ("wt", C.c_void_p),
                ("scale", C.c_void_p), ("bias", C.c_void_p)]


class Gpt2:
    """The oracle's GPT-2 over a bundle's arrays (Gpt2::new,
    composition.rs:52-56: config [n_layer, n_head, d, n_pos, vocab]).  f16
    vectors are upcast exactly; each int8 linear is stored transposed to the
    (N, K) order Bundle::load keeps (src/bundle.rs:345-355)."""

    def __init__(self, manifest, arrs, nthreads: int = 8):
        L, H, d, npos, vocab = (int(c) for c in manifest["config"][:5])
        f32 = lambda n: np.ascontiguousarray(arrs[n], np.float32)
        self.keep = []

        def ptrs(lst):
            self.keep.extend(lst)
            arr = (C.c_void_p * max(len(lst), 1))(*[a.ctypes.data for a in lst])
            self.keep.append(arr)
            return C.cast(arr, C.c_void_p)

        self.wte = np.ascontiguousarray(arrs["wte"]).view(np.uint16)
        self.wpe, self.lnfg, self.lnfb = f32("wpe"), f32("ln_f.weight"), f32("ln_f.bias")
        lg, lb, wt, sc, bi = [], [], [], [], []
        for l in range(L):
            for ln in ("ln_1", "ln_2"):
                lg.append(f32(f"h{l}.{ln}.weight"))
                lb.append(f32(f"h{l}.{ln}.bias"))
            for name in ("attn.c_attn", "attn.c_proj", "mlp.c_fc", "mlp.c_proj"):
                w = f"h{l}.{name}.weight"
                wt.append(np.ascontiguousarray(arrs[w].T))
                sc.append(f32(w + "__scale"))
                bi.append(f32(f"h{l}.{name}.bias"))
        self.s = _Gpt2W(L, H, d, npos, vocab, self.wte.ctypes.data, self.wpe.ctypes.data,
                        self.lnfg.ctypes.data, self.lnfb.ctypes.data, ptrs(lg), ptrs(lb), ptrs(wt),
                        ptrs(sc), ptrs(bi))
        self.vocab, self.nthreads = vocab, nthreads

    def generate(self, prompt, n_new: int, kv_int8: bool = False, with_logits: bool = False):
        prompt = _c(prompt, np.int64)
        out = np.empty(n_new, np.int64)
        lg = np.empty((n_new, self.vocab), np.float32) if with_logits else None
        rc = lib.fro_gpt2_generate(C.byref(self.s), _p(prompt), len(prompt), n_new, int(kv_int8),
                                   self.nthreads, _p(out), _p(lg))
        if rc == 3:
            raise OracleNaN("NaN in activations or logits")
        if rc:
            raise IndexError("token or position beyond the bundle's tables")
        return (out, lg) if with_logits else out

    def predict(self, ids, with_logits: bool = False):
        ids = _c(ids, np.int64)
        tok = np.zeros(1, np.int64)
        lg = np.empty(self.vocab, np.float32) if with_logits else None
        rc = lib.fro_gpt2_predict(C.byref(self.s), _p(ids), len(ids), self.nthreads, _p(tok), _p(lg))
        if rc == 3:
            raise OracleNaN("NaN in activations or logits")
        if rc:
            raise IndexError("token or position beyond the bundle's tables")
        return (int(tok[0]), lg) if with_logits else int(tok[0])


def nd_sum(x) -> float:
    x = _c(x, np.float32)
    return float(lib.fro_nd_sum(_p(x), x.size))


def layernorm(x, g, b):
    x = _c(x, np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    out = np.empty_like(x2)
    lib.fro_layernorm(_p(x2), x2.shape[0], x2.shape[1], _p(_c(g, np.float32)), _p(_c(b, np.float32)), _p(out))
    return out.reshape(x.shape)


def libm_f32(fn: str, x) -> np.ndarray:
    """The system libm's expf / expm1f / tanhf: what the reference's f32 math
    calls."""
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib.fro_libm_f32({"expf": 0, "expm1f": 1, "tanhf": 2}[fn], _p(x), x.size, _p(out))
    return out


# ---- affine int4 (q4a) ----
def put_q4a(data: np.ndarray, transpose: bool):
    """put_q4a (src/convert.rs:223-260): (packed (out, ceil(in/2)) u8,
    scale f16 bits, min f16 bits (out, ng), g)."""
    data = _c(data, np.float32)
    rows, cols = data.shape
    out, inp = (rows, cols) if transpose else (cols, rows)
    g = min(32, max(inp, 1))
    ng = (inp + g - 1) // g
    packed = np.empty((out, (inp + 1) // 2), np.uint8)
    s16 = np.empty((out, ng), np.uint16)
    m16 = np.empty((out, ng), np.uint16)
    g = lib.fro_put_q4a(_p(data), rows, cols, int(transpose), _p(packed), _p(s16), _p(m16))
    return packed, s16, m16, g


def q4a_dot(prow, a, scale, mins, g, k):
    return lib.fro_q4a_dot(_p(_c(prow, np.uint8)), _p(_c(a, np.float32)), _p(_c(scale, np.float32)),
                           _p(_c(mins, np.float32)), g, k)


def q4a_dot_avx2(prow, a, scale, mins, g, k):
    return lib.fro_q4a_dot_avx2(_p(_c(prow, np.uint8)), _p(_c(a, np.float32)), _p(_c(scale, np.float32)),
                                _p(_c(mins, np.float32)), g, k)


def mm_q4a(a, packed, scale_f32, min_f32, k, g):
    """Bundle::mm's Q4A arm: a (M, K) f32 -> (M, N)."""
    a = _c(a, np.float32)
    packed = _c(packed, np.uint8)
    n = packed.shape[0]
    out = np.empty((a.shape[0], n), np.float32)
    lib.fro_mm_q4a(_p(a), a.shape[0], k, _p(packed), _p(_c(scale_f32, np.float32)), _p(_c(min_f32, np.float32)),
                   n, g, _p(out))
    return out


# ---- Gemma-2 with a KV cache (src/gemma.rs) ----
class _Lin(C.Structure):
    _fields_ = [("dtype", C.c_int), ("n", C.c_size_t), ("k", C.c_size_t), ("g", C.c_size_t),
                ("packed", C.c_void_p), ("wt", C.c_void_p), ("scale", C.c_void_p), ("mins", C.c_void_p)]


class _GemmaW(C.Structure):
    _fields_ = [("n_layer", C.c_size_t), ("n_head", C.c_size_t), ("n_kv", C.c_size_t), ("hd", C.c_size_t),
                ("d", C.c_size_t), ("ffn", C.c_size_t), ("vocab", C.c_size_t), ("window", C.c_size_t),
                ("theta", C.c_float), ("eps", C.c_float), ("attn_cap", C.c_float), ("qscale", C.c_float),
                ("escale", C.c_float), ("embed", C.c_void_p), ("norm", C.c_void_p), ("norms", C.c_void_p),
                ("lin", C.c_void_p), ("arch", C.c_int), ("bias", C.c_void_p), ("qk_norm", C.c_void_p),
                ("unembed", C.c_void_p), ("embed_dt", C.c_int), ("embed_scale", C.c_void_p)]


class Gemma:
    """The oracle's Gemma-2 (arch "gemma": Gemma::new, gemma.rs:52-60) or
    Llama / Qwen (arch "rope": Rope::new, rope.rs:56-64) over a bundle's
    arrays: config [n_layer, H, nkv, hd, d, ffn, vocab, tied]; config_f
    [theta, eps, attn_cap, final_cap, qscalar, escale] (gemma, window 4096)
    or [theta, eps] (rope).  Linears as Bundle::load keeps them: int4 / q4a
    packed + f32 scales (and mins), int8 transposed to (N, K)."""

    def __init__(self, manifest, arrs, nthreads: int = 8):
        L, H, KV, hd, d, ffn, vocab = (int(c) for c in manifest["config"][:7])
        rope = manifest["arch"] == "rope"
        if rope:
            theta, eps = (float(c) for c in manifest["config_f"][:2])
            cap, qscalar, escale = 0.0, float(hd), 1.0
        else:
            theta, eps, cap, _fcap, qscalar, escale = (float(c) for c in manifest["config_f"][:6])
        f32 = lambda n: np.ascontiguousarray(arrs[n], np.float32)
        self.keep = []
        norms = []
        lins = (_Lin * (7 * L))()
        names = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
                 "mlp.up_proj", "mlp.down_proj"]
        info = {e["name"]: e for e in manifest["arrays"]}
        biases, qkn = [], []
        for l in range(L):
            if rope:
                norms += [f32(f"l{l}.in_ln"), None, f32(f"l{l}.post_ln"), None]
                for nm in ("q_proj", "k_proj", "v_proj"):
                    bn = f"l{l}.self_attn.{nm}.bias"
                    biases.append(f32(bn) if bn in arrs else None)
                for nm in ("q_norm", "k_norm"):
                    qn = f"l{l}.self_attn.{nm}"
                    qkn.append(f32(qn) if qn in arrs else None)
            else:
                for nm in ("input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                           "post_feedforward_layernorm"):
                    norms.append(f32(f"l{l}.{nm}"))
            for j, nm in enumerate(names):
                a = arrs[f"l{l}.{nm}"]
                sc = f32(f"l{l}.{nm}__scale")
                ent = info[f"l{l}.{nm}"]
                if ent.get("dtype") == "i8":       # stored (in, out)
                    wt = np.ascontiguousarray(a.T)
                    lins[7 * l + j] = _Lin(1, wt.shape[0], wt.shape[1], 0, None, wt.ctypes.data, sc.ctypes.data,
                                           None)
                    self.keep.append(wt)
                else:                              # i4 / q4a stored (out, in) packed
                    n, k = ent["shape"]
                    q4a = ent.get("dtype") == "q4a"
                    g = ent.get("group") or (64 if q4a else 32)
                    pk = np.ascontiguousarray(a)
                    mn = f32(f"l{l}.{nm}__min") if q4a else None
                    lins[7 * l + j] = _Lin(3 if q4a else 2, n, k, g, pk.ctypes.data, None, sc.ctypes.data,
                                           None if mn is None else mn.ctypes.data)
                    self.keep += [pk, mn]
                self.keep.append(sc)
        self.keep.extend(norms + biases + qkn)
        ptrs = lambda lst: (C.c_void_p * max(len(lst), 1))(*[None if a is None else a.ctypes.data for a in lst])
        nptr, bptr, qptr = ptrs(norms), ptrs(biases), ptrs(qkn)
        self.keep += [lins, nptr, bptr, qptr]
        # the embed table as stored: f32, f16 or rowi8 (+ f32 per-row scales)
        edt = info["embed"].get("dtype", "f32")
        self.embed = np.ascontiguousarray(arrs["embed"])
        self.embed_scale = f32("embed__scale") if edt == "rowi8" else None
        edt = {"f32": 3, "f16": 4, "rowi8": 5}[edt]
        tied = int(manifest["config"][7]) != 0
        self.unembed = None if (not rope or tied) else np.ascontiguousarray(arrs["lm_head"]).view(np.uint16)
        self.norm = f32("norm")
        self.s = _GemmaW(L, H, KV, hd, d, ffn, vocab, 4096, np.float32(theta), np.float32(eps), np.float32(cap),
                         np.float32(np.float32(qscalar) ** np.float32(-0.5)), np.float32(escale),
                         self.embed.ctypes.data, self.norm.ctypes.data, C.cast(nptr, C.c_void_p),
                         C.cast(lins, C.c_void_p), int(rope), C.cast(bptr, C.c_void_p), C.cast(qptr, C.c_void_p),
                         None if self.unembed is None else self.unembed.ctypes.data, edt,
                         None if self.embed_scale is None else self.embed_scale.ctypes.data)
        self.vocab, self.nthreads = vocab, nthreads

    def generate(self, prompt, n_new: int, kv_int8: bool = False, with_logits: bool = False):
        prompt = _c(prompt, np.int64)
        out = np.empty(n_new, np.int64)
        lg = np.empty((n_new, self.vocab), np.float32) if with_logits else None
        rc = lib.fro_gemma_generate(C.byref(self.s), _p(prompt), len(prompt), n_new, int(kv_int8),
                                    self.nthreads, _p(out), _p(lg))
        if rc == 3:
            raise OracleNaN("NaN in activations or logits")
        if rc:
            raise IndexError("token beyond the vocabulary")
        return (out, lg) if with_logits else out


Rope = Gemma  # the Llama / Qwen family rides the same restatement (arch "rope")


def rmsnorm(x, w, eps: float):
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib.fro_rmsnorm(_p(x), x.shape[0], x.shape[1], _p(_c(w, np.float32)), eps, _p(out))
    return out
