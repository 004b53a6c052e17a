"""Pins the CPU oracle before anything is checked against it.

Each check is independent of the oracle's own code: the reference's unit-test
known answers (tests/golden/reference_kats.json, lifted from the Rust tests
cited there), numpy's IEEE binary16 conversions, int64 / float64 brute force,
and closed-form invariants chosen so that a dropped term, a wrong rounding
mode, a wrong nibble order or a transposed operand fails one of them.
"""
import json
import os

import numpy as np
import pytest

import oracle

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))
M64 = (1 << 64) - 1


def xorshift_i8(seed, n):
    """The PRNG of i8dot_simd_vs_scalar (src/bundle.rs:1364-1370)."""
    s = seed
    out = []
    for _ in range(n):
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        v = s >> 56
        out.append(v - 256 if v >= 128 else v)
    return out, s


def lcg_u32(seed, add, n):
    """The LCG of src/jit.rs tests: s = s*6364136223846793005 + add; s>>33."""
    s = seed
    out = []
    for _ in range(n):
        s = (s * 6364136223846793005 + add) & M64
        out.append(s >> 33)
    return out, s


def u32_to_unit(u):
    # Rust: (next() as f32 / u32::MAX as f32) * 2.0 - 1.0 in f32
    return np.float32(np.float32(u) / np.float32(4294967295.0))


def round_half_away(x):
    x = np.asarray(x, np.float32)
    r = np.trunc(x)
    frac = x - r  # exact
    return r + np.where(np.abs(frac) >= 0.5, np.sign(x), 0).astype(np.float32)


# ---------------------------------------------------------------- f16 ----
def test_f16_to_f32_exhaustive():
    """Every binary16 pattern (cf. f16_to_f32_simd_vs_scalar, bundle.rs:1384)."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_matches_ieee_rne():
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000).astype(np.float32),
        np.array([0.0, -0.0, 65504, 65520, 65519.99, 1e-8, 5.96e-8, 2.98e-8, 2.9802322e-8, 6.1e-5,
                  np.inf, -np.inf, 1e30, -1e30], np.float32),
        # exact ties between adjacent f16 values (RNE must pick even)
        (np.arange(1, 2048, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10),
    ]).astype(np.float32)
    got = np.array([oracle.f32_to_f16_bits(x) for x in xs], np.uint16)
    want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------- quantisers ----
def test_put_i8_closed_form_and_kat():
    rng = np.random.default_rng(2)
    src = rng.standard_normal((37, 53)).astype(np.float32)  # (out, in) nn.Linear
    w, s16 = oracle.put_i8(src, transpose=True)
    sc = np.maximum(np.abs(src).max(axis=1) / np.float32(127.0), np.float32(1e-8)).astype(np.float32)
    want = np.clip(np.rint(src / sc[:, None]), -127, 127).astype(np.int8).T
    assert np.array_equal(w, want)
    assert np.array_equal(s16, sc.astype(np.float16).view(np.uint16))
    assert w.min() >= -127  # never -128 (convert.rs:349-354)
    k = KATS["int8_quant_roundtrip"]
    w, s16 = oracle.put_i8(np.array(k["data"], np.float32).reshape(k["rows"], k["cols"]), k["transpose"])
    s = s16.view(np.float16).astype(np.float32)
    rows = w.astype(np.float32) * s[None, :]  # weight_row(m, r) = wt[j*k+r]*scale[j]
    assert np.allclose(rows, np.array(k["want_rows"]), atol=k["tol"])


def test_put_i4_closed_form():
    rng = np.random.default_rng(3)
    for out, inp in [(5, 64), (7, 37), (3, 32), (2, 1)]:
        src = rng.standard_normal((out, inp)).astype(np.float32)
        packed, s16, g = oracle.put_i4(src, transpose=True)
        assert g == min(32, inp)
        ng = (inp + g - 1) // g
        sc = np.zeros((out, ng), np.float32)
        for gi in range(ng):
            blk = src[:, gi * g:(gi + 1) * g]
            sc[:, gi] = np.maximum(np.abs(blk).max(axis=1) / np.float32(7.0), np.float32(1e-8))
        q = np.clip(np.rint(src / np.repeat(sc, g, axis=1)[:, :inp]), -7, 7).astype(np.int8)
        # unpack: even input index = low nibble
        lo = (packed & 0x0F).astype(np.int8)
        hi = (packed >> 4).astype(np.int8)
        nib = np.stack([lo, hi], axis=2).reshape(out, -1)[:, :inp]
        nib = np.where(nib >= 8, nib - 16, nib)
        assert np.array_equal(nib, q)
        assert np.array_equal(s16, sc.astype(np.float16).view(np.uint16))


def test_put_embed_i8_kat():
    k = KATS["rowi8_embed_roundtrip"]
    data = np.array(k["data"], np.float32).reshape(k["vocab"], k["d"])
    q, s16 = oracle.put_embed_i8(data)
    row = q[k["row"]].astype(np.float32) * s16.view(np.float16).astype(np.float32)[k["row"]]
    assert np.all(np.abs(row - data[k["row"]]) < k["tol"])


# ---------------------------------------------------------------- i8dot ----
def test_i8dot_kats():
    k = KATS["i8dot_matches_manual"]
    a, w = np.array(k["a"], np.int8), np.array(k["w"], np.int8)
    assert oracle.i8dot(a, w) == int(np.dot(a.astype(np.int64), w.astype(np.int64)))
    k = KATS["i8dot_simd_vs_scalar"]
    seed = int(k["xorshift_seed"], 16)
    state = seed
    for n in k["lengths"]:
        vals, state = xorshift_i8(state, 2 * n)
        a = np.array(vals[:n], np.int8)
        w = np.array(vals[n:], np.int8)
        # the Rust test draws a (n values) then w (n values) from one stream
        assert oracle.i8dot(a, w) == int(np.dot(a.astype(np.int64), w.astype(np.int64))), n
    wc = k["worst_case"]
    a = np.full(wc["len"], wc["a"], np.int8)
    w = np.full(wc["len"], wc["w"], np.int8)
    assert oracle.i8dot(a, w) == 127 * -128 * 4864


def test_i8dot_avx512bw_equals_scalar():
    """i8dot_avx512bw (src/bundle.rs:1107-1126) against the scalar dot on the
    reference test's xorshift vectors and lengths (1359-1382), the worst
    case, and random lengths around the 32-lane step; and the int8 linear
    gives the same bits with either dot."""
    if not oracle.set_i8dot("avx512bw"):
        pytest.skip("host without AVX-512BW")
    oracle.set_i8dot("scalar")
    k = KATS["i8dot_simd_vs_scalar"]
    state = int(k["xorshift_seed"], 16)
    for n in k["lengths"]:
        vals, state = xorshift_i8(state, 2 * n)
        a, w = np.array(vals[:n], np.int8), np.array(vals[n:], np.int8)
        assert oracle.i8dot_avx512bw(a, w) == oracle.i8dot(a, w), n
    wc = k["worst_case"]
    a, w = np.full(wc["len"], wc["a"], np.int8), np.full(wc["len"], wc["w"], np.int8)
    assert oracle.i8dot_avx512bw(a, w) == 127 * -128 * 4864
    rng = np.random.default_rng(12)
    for n in (0, 1, 31, 32, 33, 63, 64, 65, 4095, 18944):
        a = rng.integers(-128, 128, n, dtype=np.int8)
        w = rng.integers(-128, 128, n, dtype=np.int8)
        assert oracle.i8dot_avx512bw(a, w) == int(np.dot(a.astype(np.int64), w.astype(np.int64))), n
    x = (rng.standard_normal((3, 896)) * np.where(rng.random(896) < 0.01, 20.0, 1.0)).astype(np.float32)
    wt = rng.integers(-127, 128, (300, 896), dtype=np.int8)
    sc = rng.uniform(1e-4, 3e-4, 300).astype(np.float32)
    ref = oracle.mm_i8_mt(x, wt, sc, 3)
    try:
        assert oracle.set_i8dot("avx512bw")
        got = oracle.mm_i8_mt(x, wt, sc, 3)
    finally:
        oracle.set_i8dot("scalar")
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_i8_transpose():
    rng = np.random.default_rng(4)
    w = rng.integers(-127, 128, (13, 29), dtype=np.int8)
    assert np.array_equal(oracle.i8_transpose(w), w.T)


# ---------------------------------------------------------- quant_row ----
def brute_quant(a):
    """Closed-form restatement of src/bundle.rs:699-708 with sorted ties."""
    a = np.asarray(a, np.float32)
    k = a.size
    t = min(32, k)
    order = sorted(range(k), key=lambda i: (-abs(float(a[i])), i))
    bulk = np.float32(abs(a[order[t]])) if t < k else np.float32(0.0)
    sa = np.float32(bulk / np.float32(127.0)) if bulk > 0 else np.float32(1.0)
    q = round_half_away(a / sa)
    a8 = np.clip(np.nan_to_num(q, nan=0.0), -127, 127).astype(np.int8)
    out_idx = sorted(order[:t])
    a8[out_idx] = 0
    return a8, sa, np.array(out_idx, np.uint32), a[out_idx]


@pytest.mark.parametrize("k", [1, 5, 32, 33, 37, 64, 100, 896, 4096])
def test_quant_row_matches_brute_force(k):
    rng = np.random.default_rng(10 + k)
    for trial in range(4):
        a = rng.standard_normal(k).astype(np.float32)
        if trial == 1 and k > 10:
            a[rng.choice(k, max(1, k // 100), replace=False)] *= 20  # outlier channels
        if trial == 2:
            a = np.round(a * 4) / 4  # many exact ties in |a|
        if trial == 3:
            a[: k // 2] = 0.0
        got = oracle.quant_row(a)
        want = brute_quant(a)
        for g, w in zip(got, want):
            assert np.array_equal(np.asarray(g), np.asarray(w)), (k, trial)


def test_quant_row_invariants_and_rounding():
    rng = np.random.default_rng(11)
    a = rng.standard_normal(4864).astype(np.float32) * 3
    a8, sa, oi, ov = oracle.quant_row(a)
    absa = np.abs(a)
    srt = np.sort(absa)[::-1]
    assert sa == np.float32(srt[32] / np.float32(127.0))  # (t+1)-th largest / 127
    assert len(oi) == 32 and np.all(a8[oi] == 0) and np.array_equal(ov, a[oi])
    assert set(oi.tolist()) == set(np.argsort(-absa, kind="stable")[:32].tolist())
    assert np.all(np.abs(a8.astype(int)) <= 127)
    assert np.all(np.diff(oi.astype(np.int64)) > 0)  # ascending channel order
    # half-away-from-zero, not ties-to-even: a/sa == 2.5 -> 3, -2.5 -> -3
    b = np.zeros(40, np.float32)
    b[:33] = 127.0  # bulk_max 127 -> sa 1
    b[33], b[34], b[35], b[36] = 2.5, -2.5, 0.5, 3.5
    a8, sa, _, _ = oracle.quant_row(b)
    assert sa == 1.0 and list(a8[33:37]) == [3, -3, 1, 4]


def test_quant_row_special_cases():
    a8, sa, oi, ov = oracle.quant_row(np.array([1.0, -2.0, 3.0], np.float32))  # t == K
    assert sa == 1.0 and not a8.any() and list(oi) == [0, 1, 2]
    a8, sa, oi, ov = oracle.quant_row(np.zeros(100, np.float32))  # bulk_max == 0
    assert sa == 1.0 and not a8.any() and list(oi) == list(range(32))
    x = np.ones(100, np.float32)
    x[7] = np.nan
    with pytest.raises(oracle.OracleNaN):
        oracle.quant_row(x)
    y = np.array([np.nan, 1.0], np.float32)  # t == K: no select, no panic
    a8, sa, oi, ov = oracle.quant_row(y)
    assert sa == 1.0 and np.isnan(ov[0])


# ---------------------------------------------------------- I8 linear ----
def test_mm_i8_f64_brute_force():
    rng = np.random.default_rng(12)
    m, k, n = 5, 300, 41
    a = rng.standard_normal((m, k)).astype(np.float32)
    a[:, [3, 77, 150]] *= 20
    wt = rng.integers(-127, 128, (n, k)).astype(np.int8)
    scale = (rng.uniform(1e-4, 3e-4, n)).astype(np.float16).astype(np.float32)
    out, acc = oracle.mm_i8(a, wt, scale, with_acc=True)
    for i in range(m):
        a8, sa, oi, ov = brute_quant(a[i])
        acc64 = wt.astype(np.int64) @ a8.astype(np.int64)
        assert np.array_equal(acc[i], acc64)
        corr = (wt[:, oi].astype(np.float64) * ov.astype(np.float64)[None, :]).sum(axis=1)
        ref = scale.astype(np.float64) * (np.float64(sa) * acc64 + corr)
        mag = np.abs(scale) * (np.abs(np.float64(sa) * acc64) + np.abs(wt[:, oi] * ov[None, :]).sum(axis=1))
        assert np.all(np.abs(out[i] - ref) <= 1e-6 * mag + 1e-30)
    # rows are independent and the threaded variant uses the same arithmetic
    assert np.array_equal(oracle.mm_i8_mt(a, wt, scale, 3), out)
    assert np.array_equal(oracle.mm_i8_mt(a[:1], wt, scale, 4), out[:1])


def test_mm_i8_nan_raises_like_reference():
    wt = np.ones((4, 40), np.int8)
    a = np.ones((2, 40), np.float32)
    a[1, 5] = np.nan
    with pytest.raises(oracle.OracleNaN):
        oracle.mm_i8(a, wt, np.ones(4, np.float32))


# ------------------------------------------------------------------ i4 ----
def pack_nibbles(q):
    q = np.asarray(q, np.int64) & 0xF
    k = q.shape[-1]
    if k % 2:
        q = np.concatenate([q, np.zeros(q.shape[:-1] + (1,), np.int64)], axis=-1)
    return (q[..., 0::2] | (q[..., 1::2] << 4)).astype(np.uint8)


def test_i4_dot_kats():
    k = KATS["i4_q4a_dot_matches_manual"]
    for f in (oracle.i4_dot, oracle.i4_dot_avx2):
        assert f(np.array(k["prow"], np.uint8), np.array(k["a"], np.float32),
                 np.array(k["scale"], np.float32), k["g"], k["k"]) == k["want_i4"]
    k = KATS["i4_q4a_dot_simd_vs_reference"]
    kk, g = k["k"], k["g"]
    ng = (kk + g - 1) // g
    nibs = np.array([((i * 7 + 3) % 16) - 8 for i in range(kk)], np.int64)
    prow = pack_nibbles(nibs)
    a = np.sin(np.arange(kk, dtype=np.float32) * np.float32(0.13) - np.float32(2.0)).astype(np.float32)
    scale = (np.float32(0.1) + np.arange(ng, dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    want = float((a.astype(np.float64) * nibs * scale[np.arange(kk) // g]).sum())
    for f in (oracle.i4_dot, oracle.i4_dot_avx2):
        assert abs(f(prow, a, scale, g, kk) - want) < k["tol"]


@pytest.mark.parametrize("case", ["jit_i4_dot_matches_scalar", "jit_i4_dot_vec_matches_scalar"])
def test_i4_dot_jit_lcg_vectors(case):
    k = KATS[case]
    cases = [(k["k"], k["g"])] if "cases" not in k else [tuple(c) for c in k["cases"]]
    for kk, g in cases:
        nb, ng = (kk + 1) // 2, (kk + g - 1) // g
        vals, _ = lcg_u32(k["seed"], k["lcg_add"], nb + kk + ng)
        prow = np.array([v & 0xFF for v in vals[:nb]], np.uint8)
        a = np.array([u32_to_unit(v) * np.float32(2.0) - np.float32(1.0) for v in vals[nb:nb + kk]], np.float32)
        scale = np.array([np.float32(0.01) + u32_to_unit(v) * np.float32(0.03) for v in vals[nb + kk:]], np.float32)
        s = oracle.i4_dot(prow, a, scale, g, kk)
        v = oracle.i4_dot_avx2(prow, a, scale, g, kk)
        lo = (prow & 0xF).astype(np.int64)
        hi = (prow >> 4).astype(np.int64)
        nib = np.stack([lo, hi], 1).reshape(-1)[:kk]
        nib = np.where(nib >= 8, nib - 16, nib)
        want = float((a.astype(np.float64) * nib * scale[np.arange(kk) // g]).sum())
        assert abs(s - v) < k["tol"] and abs(s - want) < 1e-4 and abs(v - want) < 1e-4


def test_i4_avx2_order_is_the_documented_tree():
    """g=8, one chunk: gsum = ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7)), l_q = w_q*a_q."""
    a = np.array([1e8, 1.0, -1e8, 3.0, 0.5, 1.0, 0.25, 7.0], np.float32)
    nib = np.array([1, 1, 1, 1, 1, 1, 1, 1])
    prow = pack_nibbles(nib)
    got = oracle.i4_dot_avx2(prow, a, np.array([1.0], np.float32), 8, 8)
    l = a.astype(np.float32)
    f = np.float32
    want = f(f(f(l[0] + l[4]) + f(l[2] + l[6])) + f(f(l[1] + l[5]) + f(l[3] + l[7])))
    assert got == want
    seq = np.float32(0)
    for x in l:
        seq = np.float32(seq + x)
    assert oracle.i4_dot(prow, a, np.array([1.0], np.float32), 8, 8) == seq


def test_mm_i4_f64_brute_force():
    rng = np.random.default_rng(13)
    for m, k, n in [(1, 96, 7), (3, 96, 7), (4, 37, 5)]:
        src = rng.standard_normal((n, k)).astype(np.float32)
        packed, s16, g = oracle.put_i4(src, True)
        scale = s16.view(np.float16).astype(np.float32)
        a = rng.standard_normal((m, k)).astype(np.float32)
        out = oracle.mm_i4(a, packed, scale, k, g)
        lo = (packed & 0xF).astype(np.int64)
        hi = (packed >> 4).astype(np.int64)
        nib = np.stack([lo, hi], 2).reshape(n, -1)[:, :k]
        nib = np.where(nib >= 8, nib - 16, nib)
        w = nib * scale[:, np.arange(k) // g].astype(np.float64)  # (n, k)
        ref = a.astype(np.float64) @ w.T
        mag = np.abs(a.astype(np.float64)) @ np.abs(w.T)
        assert np.all(np.abs(out - ref) <= 1e-5 * mag + 1e-12)


# ------------------------------------------------------------ experts ----
def test_expert_mm_and_sgemm_f64():
    rng = np.random.default_rng(14)
    x = rng.standard_normal((6, 64)).astype(np.float32)
    raw = rng.integers(-127, 128, (64, 48)).astype(np.int8)
    sc = rng.uniform(1e-3, 3e-3, 48).astype(np.float16).astype(np.float32)
    y = oracle.expert_mm_i8(x, raw, sc)
    v = raw.astype(np.float64) * sc.astype(np.float64)[None, :]
    ref = x.astype(np.float64) @ v
    assert np.all(np.abs(y - ref) <= 1e-5 * (np.abs(x) @ np.abs(v)) + 1e-12)


def test_nonlinearities():
    xs = np.linspace(-8, 8, 101).astype(np.float32)
    s = np.array([oracle.silu(x) for x in xs])
    assert np.allclose(s, xs / (1 + np.exp(-xs.astype(np.float64))), rtol=1e-6, atol=1e-7)
    g = np.array([oracle.gelu_tanh(x) for x in xs])
    x64 = xs.astype(np.float64)
    want = 0.5 * x64 * (1 + np.tanh(np.sqrt(2 / np.pi) * (x64 + 0.044715 * x64 ** 3)))
    assert np.allclose(g, want, rtol=1e-5, atol=1e-6)


def test_moe_route_brute_force():
    rng = np.random.default_rng(15)
    T, E, k = 64, 128, 8
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[3, 10] = logits[3, 20] = 9.0  # an exact tie: lower expert first
    for norm in (True, False):
        sel, w, probs = oracle.moe_route(logits, k, norm)
        l64 = logits.astype(np.float64)
        p64 = np.exp(l64 - l64.max(1, keepdims=True))
        p64 /= p64.sum(1, keepdims=True)
        assert np.allclose(probs, p64, rtol=2e-6, atol=1e-9)
        for t in range(T):
            order = sorted(range(E), key=lambda e: (-float(probs[t, e]), e))[:k]
            assert list(sel[t]) == order
            den = np.float32(sum(probs[t, order])) if norm else np.float32(1.0)
            assert np.allclose(w[t], probs[t, order] / den, rtol=1e-6)
        assert sel[3, 0] == 10 and sel[3, 1] == 20
    pes = rng.uniform(0.5, 1.5, E).astype(np.float32)
    sel, w2, probs = oracle.moe_route(logits, k, True, pes)
    sel_n, w_n, _ = oracle.moe_route(logits, k, True)
    assert np.array_equal(sel, sel_n)
    assert np.allclose(w2, w_n * pes[sel], rtol=1e-6)


def make_experts(rng, E, d, mi, act):
    gw = mi if act == 0 else 2 * mi
    gate = [rng.integers(-127, 128, (d, gw)).astype(np.int8) for _ in range(E)]
    gs = [rng.uniform(1e-3, 2e-3, gw).astype(np.float32) for _ in range(E)]
    up = [rng.integers(-127, 128, (d, mi)).astype(np.int8) for _ in range(E)]
    us = [rng.uniform(1e-3, 2e-3, mi).astype(np.float32) for _ in range(E)]
    down = [rng.integers(-127, 128, (mi, d)).astype(np.int8) for _ in range(E)]
    ds = [rng.uniform(1e-3, 2e-3, d).astype(np.float32) for _ in range(E)]
    return gate, gs, up, us, down, ds


@pytest.mark.parametrize("act", [0, 1])
def test_moe_f64_brute_force(act):
    rng = np.random.default_rng(16 + act)
    T, E, d, mi, k = 24, 8, 64, 32, 3
    x = rng.standard_normal((T, d)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    gate, gs, up, us, down, ds = make_experts(rng, E, d, mi, act)
    pes = rng.uniform(0.5, 1.5, E).astype(np.float32) if act else None
    out = oracle.moe(x, logits, k, True, gate, gs, up, us, down, ds, act, pes)
    sel, w, _ = oracle.moe_route(logits, k, True, pes)
    ref = np.zeros((T, d))
    for t in range(T):
        for i in range(k):
            e = sel[t, i]
            x64 = x[t].astype(np.float64)
            g = x64 @ (gate[e] * gs[e][None, :].astype(np.float64))
            if act == 0:
                u = x64 @ (up[e] * us[e][None, :].astype(np.float64))
                h = g / (1 + np.exp(-g)) * u
            else:
                gg, uu = g[:mi], g[mi:]
                h = 0.5 * gg * (1 + np.tanh(np.sqrt(2 / np.pi) * (gg + 0.044715 * gg ** 3))) * uu
            ref[t] += w[t, i] * (h @ (down[e] * ds[e][None, :].astype(np.float64)))
    assert np.max(np.abs(out - ref)) <= 1e-5 * np.max(np.abs(ref))
    # the threaded restatement (experts in parallel, one ascending-id
    # combine) gives the same bits for any thread count
    for nt in (2, 3, 8):
        o2 = oracle.moe(x, logits, k, True, gate, gs, up, us, down, ds, act, pes, nthreads=nt)
        assert np.array_equal(o2.view(np.uint32), out.view(np.uint32))


# ------------------------------------------- package quantisers vs oracle ----
def test_package_quantisers_match_oracle():
    from fieldrun_amd import convert
    rng = np.random.default_rng(17)
    for shape, tr in [((37, 53), True), ((64, 33), False), ((5, 1), True), ((3, 96), True)]:
        src = (rng.standard_normal(shape) * 0.02).astype(np.float32)
        w1, s1 = convert.put_i8(src, tr)
        w2, s2 = oracle.put_i8(src, tr)
        assert np.array_equal(w1, w2) and np.array_equal(s1.view(np.uint16), s2)
        p1, t1, g1 = convert.put_i4(src, tr)
        p2, t2, g2 = oracle.put_i4(src, tr)
        assert g1 == g2 and np.array_equal(p1, p2) and np.array_equal(t1.view(np.uint16), t2)
        k = src.shape[1] if tr else src.shape[0]
        assert np.array_equal(convert.unpack_i4(p1, k).shape, (p1.shape[0], k))
    e = rng.standard_normal((9, 17)).astype(np.float32)
    q1, s1 = convert.put_embed_i8(e)
    q2, s2 = oracle.put_embed_i8(e)
    assert np.array_equal(q1, q2) and np.array_equal(s1.view(np.uint16), s2)


# ---- the unembed row dot (src/bundle.rs:958-1015) ----
# The reference has no test for rowdot_f32; the oracle is pinned by exact
# small-integer dots (every order gives the same sum), an f64 bound, and
# inputs whose f32 result follows by hand from the order.

@pytest.mark.parametrize("kind", ["f32", "f16", "rowi8"])
@pytest.mark.parametrize("d", [0, 1, 7, 8, 9, 64, 131])
def test_rowdot_exact_integer_dots(kind, d):
    rng = np.random.default_rng(100 + d)
    rows = 5
    wi = rng.integers(-8, 9, (rows, d))
    x = rng.integers(-8, 9, d).astype(np.float32)
    exact = (wi.astype(np.int64) @ x.astype(np.int64)).astype(np.float64)
    scale = np.full(rows, 0.5, np.float32)
    if kind == "f32":
        data, want = wi.astype(np.float32), exact
    elif kind == "f16":
        data, want = wi.astype(np.float16).view(np.uint16), exact
    else:
        data, want = wi.astype(np.int8), exact * 0.5
    got = oracle.rowdot_f32(kind, data, x, scale if kind == "rowi8" else None)
    assert np.array_equal(got.astype(np.float64), want)
    sub = oracle.rowdot_f32_subset(kind, data, x, [4, 0, -1, rows, 2], scale if kind == "rowi8" else None)
    assert np.array_equal(sub[[0, 1, 4]].astype(np.float64), want[[4, 0, 2]])
    assert np.isneginf(sub[2]) and np.isneginf(sub[3])


def test_rowdot_f64_bound():
    rng = np.random.default_rng(7)
    rows, d = 40, 777
    x = rng.standard_normal(d).astype(np.float32)
    w16 = (rng.standard_normal((rows, d)) * 0.02).astype(np.float16)
    w8 = rng.integers(-127, 128, (rows, d)).astype(np.int8)
    s8 = rng.uniform(1e-4, 3e-4, rows).astype(np.float32)
    for kind, data, sc, wf in [("f16", w16.view(np.uint16), None, w16.astype(np.float64)),
                               ("rowi8", w8, s8, w8.astype(np.float64) * s8[:, None].astype(np.float64))]:
        got = oracle.rowdot_f32(kind, data, x, sc).astype(np.float64)
        ref = wf @ x.astype(np.float64)
        bound = d * 2.0 ** -23 * (np.abs(wf) @ np.abs(x.astype(np.float64))) + 1e-30
        assert np.all(np.abs(got - ref) <= bound)


def test_rowdot_order_fold_vs_avx2_lanes():
    # x = [2^24, 1 x 8], w = 1: the fold (f32, f16, rowi8 subset) drops every
    # +1 (2^24 + 1 rounds to even 2^24): 2^24.  rowi8_dot_avx2: lane 0 holds
    # 2^24, lanes 1..7 one each; hsum: (2^24+1 -> 2^24) + (1+1) + ... =
    # 2^24 + 6, then the tail (k = 8) + 1 -> 2^24 + 7, rounded to even 2^24 + 8.
    x = np.array([2.0 ** 24] + [1.0] * 8, np.float32)
    one = np.ones((1, 9))
    sc = np.ones(1, np.float32)
    assert oracle.rowdot_f32("f32", one.astype(np.float32), x)[0] == 2.0 ** 24
    assert oracle.rowdot_f32("f16", one.astype(np.float16).view(np.uint16), x)[0] == 2.0 ** 24
    assert oracle.rowdot_f32("rowi8", one.astype(np.int8), x, sc)[0] == 2.0 ** 24 + 8
    assert oracle.rowdot_f32_subset("rowi8", one.astype(np.int8), x, [0], sc)[0] == 2.0 ** 24
    # eight full lanes, no tail: x = [2^24, 1 x 63]: lane 0 stays 2^24, lanes
    # 1..7 hold 8 each: ((2^24 + 8) + 16) + (16 + 16) = 2^24 + 56, exact
    x = np.array([2.0 ** 24] + [1.0] * 63, np.float32)
    assert oracle.rowdot_f32("rowi8", np.ones((1, 64), np.int8), x, sc)[0] == 2.0 ** 24 + 56
    assert oracle.rowdot_f32("f32", np.ones((1, 64), np.float32), x)[0] == 2.0 ** 24


def test_rowdot_empty_rows_keep_the_fold_sign():
    # Rust 1.89's f32 Sum folds from -0.0: an empty f32 / f16 / subset dot is
    # -0.0; the AVX2 lanes start at +0.0
    x = np.zeros(0, np.float32)
    for kind, data in [("f32", np.zeros((2, 0), np.float32)), ("f16", np.zeros((2, 0), np.uint16))]:
        got = oracle.rowdot_f32(kind, data, x)
        assert np.all(got == 0) and np.all(np.signbit(got))
    sc = np.ones(2, np.float32)
    got = oracle.rowdot_f32("rowi8", np.zeros((2, 0), np.int8), x, sc)
    assert np.all(got == 0) and not np.any(np.signbit(got))
    sub = oracle.rowdot_f32_subset("rowi8", np.zeros((2, 0), np.int8), x, [1], sc)
    assert sub[0] == 0 and np.signbit(sub[0])


# ---- affine int4 (q4a): src/bundle.rs:118-143, 231-258, 802-845; convert.rs:223-260 ----
def test_q4a_dot_kats():
    k = KATS["i4_q4a_dot_matches_manual"]   # unsigned nibbles [1, 14, 3, 15], w = 0.5 q - 1
    for f in (oracle.q4a_dot, oracle.q4a_dot_avx2):
        got = f(np.array(k["prow"], np.uint8), np.array(k["a"], np.float32), np.array(k["q4a_scale"], np.float32),
                np.array(k["q4a_min"], np.float32), k["g"], k["k"])
        assert abs(got - k["want_q4a"]) < k["q4a_tol"]
        assert got == 12.5   # every step is exact here
    k = KATS["i4_q4a_dot_simd_vs_reference"]
    kk, g = k["k"], k["g"]
    ng = (kk + g - 1) // g
    nibs = np.array([((i * 7 + 3) % 16) - 8 for i in range(kk)], np.int64)
    prow = pack_nibbles(nibs)
    a = np.sin(np.arange(kk, dtype=np.float32) * np.float32(0.13) - np.float32(2.0)).astype(np.float32)
    scale = (np.float32(0.1) + np.arange(ng, dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    mins = (np.float32(-0.3) + np.arange(ng, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    u = nibs & 0xF
    want = float((a.astype(np.float64) * (scale[np.arange(kk) // g] * u + mins[np.arange(kk) // g])).sum())
    for f in (oracle.q4a_dot, oracle.q4a_dot_avx2):
        assert abs(f(prow, a, scale, mins, g, kk) - want) < k["tol"]


def test_q4a_dot_avx2_lane_order():
    # one group of 16, every nibble 1, scale 1, min 0; a0 = 2^24, a1 = a5 = 1.
    # The AVX2 order puts a1 and a5 in lanes 1 and 5: (l1 + l5) = 2 and
    # 2^24 + 2 is exact.  The scalar fold adds them to 2^24 one at a time and
    # loses both (2^24 + 1 ties to even, 2^24).
    a = np.zeros(16, np.float32)
    a[0], a[1], a[5] = 2.0 ** 24, 1.0, 1.0
    prow = pack_nibbles(np.ones(16, np.int64))
    one, zero = np.ones(1, np.float32), np.zeros(1, np.float32)
    assert oracle.q4a_dot_avx2(prow, a, one, zero, 16, 16) == 2.0 ** 24 + 2
    assert oracle.q4a_dot(prow, a, one, zero, 16, 16) == 2.0 ** 24
    # a group of 13 starting at an odd k: the chunk reads nibbles from byte kk / 2
    # (so from k - 1), as unpack8_nibbles does; then a 5-element tail
    k, g = 26, 13
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, k)
    a = rng.integers(-4, 5, k).astype(np.float32)
    prow = pack_nibbles(q)
    s, m = np.array([0.5, 0.25], np.float32), np.array([1.0, -2.0], np.float32)
    # group 1 (k = 13..25): chunk k = 13..20 pairs a[13+i] with nibble 12+i
    qs = sum(a[13 + i] * q[12 + i] for i in range(8)) + sum(a[21 + i] * q[21 + i] for i in range(5))
    as_ = a[13:].sum()
    g0 = (a[:8] * q[:8]).sum() + (a[8:13] * q[8:13]).sum()
    want = np.float32(0.5 * g0 + 1.0 * a[:13].sum()) + np.float32(0.25 * qs - 2.0 * as_)
    assert oracle.q4a_dot_avx2(prow, a, s, m, g, k) == want     # small integers: every step exact


def test_q4a_exact_small_integers_and_gemm():
    rng = np.random.default_rng(7)
    n, k, g = 24, 96, 32
    q = rng.integers(0, 16, (n, k))
    packed = pack_nibbles(q)
    s = (2.0 ** rng.integers(-3, 2, (n, k // g))).astype(np.float32)
    m = rng.integers(-4, 4, (n, k // g)).astype(np.float32)
    a = rng.integers(-8, 9, (3, k)).astype(np.float32)
    w = s[:, np.arange(k) // g] * q + m[:, np.arange(k) // g]          # exact
    want = a.astype(np.float64) @ w.T.astype(np.float64)
    for mm in (1, 3):
        assert np.array_equal(oracle.mm_q4a(a[:mm], packed, s, m, k, g), want[:mm].astype(np.float32))


def test_put_q4a_closed_forms():
    from fieldrun_amd import convert
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((40, 70)) * 0.1).astype(np.float32)        # (out, in)
    packed, s16, m16, g = oracle.put_q4a(w, True)
    assert g == 32 and packed.shape == (40, 35) and s16.shape == (40, 3)
    q = np.stack([packed & 15, packed >> 4], axis=2).reshape(40, -1)[:, :70].astype(np.int64)
    for j in range(40):
        for gi in range(3):
            seg = w[j, gi * 32:(gi + 1) * 32]
            qs = q[j, gi * 32:(gi + 1) * 32]
            assert qs[np.argmin(seg)] == 0 and qs[np.argmax(seg)] == 15   # the ends map to 0 and 15
            sc = max((np.float32(seg.max()) - np.float32(seg.min())) / np.float32(15), np.float32(1e-8))
            assert s16.view(np.float16)[j, gi] == np.float16(sc)
            assert m16.view(np.float16)[j, gi] == np.float16(seg.min())
            assert np.abs(sc * qs + seg.min() - seg).max() <= sc * 0.5001
    # the package's numpy quantiser writes the same bytes
    p2, s2, m2, g2 = convert.put_q4a(w, True)
    assert g2 == g and np.array_equal(p2, packed)
    assert np.array_equal(s2.view(np.uint16), s16) and np.array_equal(m2.view(np.uint16), m16)
    p3, s3, m3, _ = convert.put_q4a(np.ascontiguousarray(w.T), False)
    assert np.array_equal(p3, packed) and np.array_equal(s3, s2) and np.array_equal(m3, m2)


# ---- a.dot's order (matrixmultiply 0.3.10 sgemm) and expert_f32's arms ----

def test_mm_dot_blocks_of_256():
    """matrixmultiply's gemm_loop: k in blocks of 256 (S_KC), each an FMA
    chain from +0, the block results added in order.  x = [2^24, 0 x 255,
    1 x 256] against ones: the sequential chain stays at 2^24 (each + 1 is
    a tie to even), the blocked sum is 2^24 + 256 (block two sums to 256
    exactly); a 128-long block, or a chain that carried on, gives 2^24."""
    x = np.zeros(512, np.float32)
    x[0] = 2.0 ** 24
    x[256:] = 1.0
    w = np.ones(512, np.float32)
    assert oracle.mm_dot(x, w) == 2.0 ** 24 + 256
    assert oracle.mm_dot(x[:256], w[:256]) == 2.0 ** 24  # one block: one chain
    x2 = x.copy()
    x2[256:384] = 0.0  # block two sums to 128
    assert oracle.mm_dot(x2, w) == 2.0 ** 24 + 128
    # exact small integers: any order gives the integer dot
    rng = np.random.default_rng(0)
    a = rng.integers(-50, 50, 1000).astype(np.float32)
    b = rng.integers(-50, 50, 1000).astype(np.float32)
    assert oracle.mm_dot(a, b) == float(np.dot(a.astype(np.int64), b.astype(np.int64)))


def _i4_dequant_closed_form(packed, scale16, k, g):
    from fieldrun_amd import convert
    s4 = convert.unpack_i4(packed, k).astype(np.float32)  # (out, k)
    sc = np.repeat(oracle.f16_to_f32(scale16), g, axis=1)[:, :k]
    return np.ascontiguousarray((s4 * sc).T)  # (in, out); s4 * f16 scale is exact in f32


@pytest.mark.parametrize("k,out", [(256, 48), (130, 9), (37, 5)])
def test_expert_f32_arms_closed_forms(k, out):
    """expert_f32 (src/bundle.rs:404-454) per arm against a closed form:
    i4 = sign-extended nibble * scale[j, i / g] transposed to (in, out)
    (even input in the low nibble); q4a = scale * u4 + min (one f32 mul,
    one f32 add); f16 = the IEEE upcast; f32 as stored; i8 = q * scale[j]."""
    from fieldrun_amd import convert
    rng = np.random.default_rng(k)
    src = (rng.standard_normal((out, k)) * 0.05).astype(np.float32)
    packed, s16, g = convert.put_i4(src, True)
    e = oracle.expert("i4", packed, oracle.f16_to_f32(s16.view(np.uint16)), None, g, k, out)
    assert np.array_equal(oracle.expert_f32(e), _i4_dequant_closed_form(packed, s16.view(np.uint16), k, g))
    qp, qs16, qm16, qg = convert.put_q4a(src, True)
    lo, hi = (qp & 0x0F).astype(np.float32), (qp >> 4).astype(np.float32)
    u4 = np.stack([lo, hi], axis=2).reshape(out, -1)[:, :k]
    sc = np.repeat(qs16.astype(np.float32), qg, axis=1)[:, :k]
    mn = np.repeat(qm16.astype(np.float32), qg, axis=1)[:, :k]
    want = np.ascontiguousarray(((sc * u4).astype(np.float32) + mn).astype(np.float32).T)
    e = oracle.expert("q4a", qp, qs16.astype(np.float32), qm16.astype(np.float32), qg, k, out)
    assert np.array_equal(oracle.expert_f32(e), want)
    t = np.ascontiguousarray(src.T)
    h = t.astype(np.float16)
    assert np.array_equal(oracle.expert_f32(oracle.expert("f16", h.view(np.uint16))), h.astype(np.float32))
    assert np.array_equal(oracle.expert_f32(oracle.expert("f32", t)), t)
    w8, s8 = convert.put_i8(src, True)
    s8f = s8.astype(np.float32)
    assert np.array_equal(oracle.expert_f32(oracle.expert("i8", w8, s8f)), (w8.astype(np.float32) * s8f).astype(np.float32))


def test_expert_mm_any_dtype_f64_and_exact_integers():
    """expert_mm = x . expert_f32: within f32 rounding of the f64 product,
    and exact for small-integer activations against integer-valued f32
    weights; the i8 arm equals fro_expert_mm_i8."""
    from fieldrun_amd import convert
    rng = np.random.default_rng(7)
    src = (rng.standard_normal((40, 300)) * 0.05).astype(np.float32)
    x = rng.standard_normal((6, 300)).astype(np.float32)
    packed, s16, g = convert.put_i4(src, True)
    e = oracle.expert("i4", packed, oracle.f16_to_f32(s16.view(np.uint16)), None, g, 300, 40)
    W = oracle.expert_f32(e).astype(np.float64)
    y = oracle.expert_mm(x, e)
    ref = x.astype(np.float64) @ W
    assert np.all(np.abs(y - ref) <= 1e-5 * (np.abs(x).astype(np.float64) @ np.abs(W)) + 1e-30)
    xi = rng.integers(-9, 9, (4, 300)).astype(np.float32)
    wi = rng.integers(-30, 30, (300, 17)).astype(np.float32)
    yi = oracle.expert_mm(xi, oracle.expert("f32", wi))
    assert np.array_equal(yi, (xi.astype(np.int64) @ wi.astype(np.int64)).astype(np.float32))
    w8, s8 = convert.put_i8(src, True)
    assert np.array_equal(oracle.expert_mm(x, oracle.expert("i8", w8, s8.astype(np.float32))),
                          oracle.expert_mm_i8(x, w8, s8.astype(np.float32)))


@pytest.mark.parametrize("act", [0, 1])
def test_moe_ex_reduces_to_the_int8_bank(act):
    """The layer over f32 experts that hold exactly the int8 bank's
    dequantised values (q * s) is the int8 layer bit for bit: the generic
    expert path adds nothing of its own to routing, gating or combine."""
    from fieldrun_amd import synth
    E, d, mi, k, T = 8, 96, 40, 3, 11
    gate, gs, up, us, down, ds = synth.moe_layer(E, d, mi, 21 + act, act)
    rng = np.random.default_rng(act)
    x = rng.standard_normal((T, d)).astype(np.float32)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    pes = rng.uniform(0.5, 1.5, E).astype(np.float32) if act else None
    f32 = lambda W, S: [oracle.expert("f32", (w.astype(np.float32) * s[None, :]).astype(np.float32))  # noqa: E731
                        for w, s in zip(W, S)]
    r8 = oracle.moe(x, lg, k, True, gate, gs, up, us, down, ds, act, pes)
    rx = oracle.moe_ex(x, lg, k, True, f32(gate, gs), f32(up, us) if act == 0 else [], f32(down, ds), act, pes)
    assert np.array_equal(r8.view(np.uint32), rx.view(np.uint32))
