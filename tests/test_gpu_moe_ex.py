"""Parity of expert banks stored as int4, q4a, f16 and f32 (the other arms of
expert_f32, /root/reference/src/bundle.rs:404-454) against the CPU oracle.

expert_mm: bit-exact to the oracle (each weight formed as expert_f32 forms
it, then a.dot's order: matrixmultiply 0.3.10's 256-long k blocks, each an
FMA chain from +0, added in order).  The routed layer: q4a / f16 / f32
banks run the same order on the device, so the whole layer is bit-exact;
int4 banks with g % 32 == 0 run the int8 MFMA on 24-bit activation digits,
so every element is within 1e-5 of the sum of the magnitudes of its terms
(the bound below), with every token's expert set identical to the oracle's.
"""
import os
import tempfile

import numpy as np
import pytest

import oracle
from fieldrun_amd import synth
import fieldrun_amd as fa

pytestmark = pytest.mark.gpu

DTYPES = {"int4": "i4", "q4a": "q4a", "f16": "f16", "f32": "f32"}


def _silu(g):
    return g / (1.0 + np.exp(-g))


def _gelu(g):
    return 0.5 * g * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g + 0.044715 * g ** 3)))


def _ex(m, dtype):
    """synth.moe_layer_ex's dict -> the oracle's expert description."""
    sc = None if m["scale"] is None else oracle.f16_to_f32(m["scale"])
    mn = None if m["min"] is None else oracle.f16_to_f32(m["min"])
    return oracle.expert(DTYPES[dtype], m["raw"], sc, mn, m["g"], m["inp"], m["out"])


def _upload(ctx, dtype, d, mi, gate, up, down, act):
    pick = lambda lst, key: None if not lst or lst[0][key] is None else [m[key] for m in lst]  # noqa: E731
    return ctx.upload_moe(DTYPES[dtype], d, mi, [m["raw"] for m in gate], [m["raw"] for m in down],
                          [m["raw"] for m in up] if act == 0 else None, pick(gate, "scale"),
                          pick(up, "scale") if act == 0 else None, pick(down, "scale"), pick(gate, "min"),
                          pick(up, "min") if act == 0 else None, pick(down, "min"), act,
                          gate[0]["g"] if dtype in ("int4", "q4a") else 0)


def term_bound(x, sel, w, G, U, D, act):
    """f64 bound per output element (t, c): sum over t's experts of |w| *
    sum_j (|h_j| + dh_j) * |down[j, c]|, dh_j bounding how far an error of
    the gate / up sums (relative to the magnitudes of their terms) moves
    h_j = act(g_j) * u_j.  G, U, D: the experts' f64 weights (in, out) as
    expert_f32 forms them."""
    T, d = x.shape
    B = np.zeros((T, d))
    X = x.astype(np.float64)
    for e in range(len(G)):
        tok, slot = np.nonzero(sel == e)
        if not len(tok):
            continue
        Xe, Ae = X[tok], np.abs(X[tok])
        g, Sg = Xe @ G[e], Ae @ np.abs(G[e])
        if act == 0:
            u, Su = Xe @ U[e], Ae @ np.abs(U[e])
            a = _silu(g)
            h = a * u
            dh = 1.1 * np.abs(u) * Sg + np.abs(a) * Su
        else:
            mi = G[e].shape[1] // 2
            a = _gelu(g[:, :mi])
            h = a * g[:, mi:]
            dh = 1.2 * np.abs(g[:, mi:]) * Sg[:, :mi] + np.abs(a) * Sg[:, mi:]
        np.add.at(B, tok, np.abs(w[tok, slot])[:, None] * ((np.abs(h) + dh) @ np.abs(D[e])))
    return B


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("d,mi,act", [(256, 96, 0), (130, 40, 1), (2048, 768, 0)])
def test_expert_mm_bit_exact(ctx, dtype, d, mi, act):
    E = 3
    gate, up, down = synth.moe_layer_ex(E, d, mi, 60 + d + act, dtype, act)
    bank = _upload(ctx, dtype, d, mi, gate, up, down, act)
    assert bank.dtype == {"int4": fa.FRQ_DT_I4, "q4a": fa.FRQ_DT_Q4A, "f16": fa.FRQ_DT_F16,
                          "f32": fa.FRQ_DT_F32}[dtype]
    rng = np.random.default_rng(d + act)
    for e in range(E):
        x = rng.standard_normal((5, d)).astype(np.float32)
        y = bank.expert_mm(0, e, x)
        r = oracle.expert_mm(x, _ex(gate[e], dtype))
        assert np.array_equal(y.view(np.uint32), r.view(np.uint32)), (dtype, e, "gate")
        if act == 0:
            y = bank.expert_mm(1, e, x)
            r = oracle.expert_mm(x, _ex(up[e], dtype))
            assert np.array_equal(y.view(np.uint32), r.view(np.uint32)), (dtype, e, "up")
        h = rng.standard_normal((3, mi)).astype(np.float32)
        y = bank.expert_mm(2, e, h)
        r = oracle.expert_mm(h, _ex(down[e], dtype))
        assert np.array_equal(y.view(np.uint32), r.view(np.uint32)), (dtype, e, "down")


CASES = [(1, 16, 256, 64, 4, 0), (40, 16, 256, 64, 4, 0), (7, 8, 130, 40, 8, 1), (1, 8, 128, 32, 8, 1),
         (300, 8, 256, 64, 4, 0), (1, 128, 2048, 768, 8, 0), (512, 128, 2048, 768, 8, 0), (64, 32, 2048, 768, 8, 0)]


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("T,E,d,mi,k,act", CASES)
def test_moe_ex_layer_parity(ctx, dtype, T, E, d, mi, k, act):
    """configs[3]'s dims (E 128, d 2048, mi 768, top-8) at T = 1 and 512
    among the cases.  q4a / f16 / f32 layers bit-exact; int4 within the
    term bound, routing identical in every case."""
    if dtype != "int4" and T == 512:
        pytest.skip("the exact-order banks at T = 512 are covered by T = 300 and 64 (oracle time)")
    gate, up, down = synth.moe_layer_ex(E, d, mi, synth.seed(3) + T + act + E, dtype, act)
    bank = _upload(ctx, dtype, d, mi, gate, up, down, act)
    rng = np.random.default_rng(T + E + d)
    x = rng.standard_normal((T, d)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    pes = rng.uniform(0.5, 1.5, E).astype(np.float32) if act else None
    out = bank.forward(x, logits, k, True, pes)
    G = [_ex(m, dtype) for m in gate]
    U = [_ex(m, dtype) for m in up]
    D = [_ex(m, dtype) for m in down]
    ref = oracle.moe_ex(x, logits, k, True, G, U, D, act, pes, nthreads=16)
    sel, w = ctx.moe_route(logits, k, True, pes)
    rsel, rw, _ = oracle.moe_route(logits, k, True, pes)
    assert np.array_equal(sel, rsel)
    if dtype != "int4":
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
        return
    f64 = lambda lst: [oracle.expert_f32(m).astype(np.float64) for m in lst]  # noqa: E731
    B = term_bound(x, rsel, rw, f64(G), f64(U), f64(D), act)
    err = np.abs(out.astype(np.float64) - ref)
    assert np.all(err <= 1e-5 * B), float((err / np.maximum(B, 1e-300)).max())


def test_moe_int4_decode_matches_batched_row(ctx):
    """T == 1 (4-row tiles) and the same token inside a batch (32-row
    tiles) run the same digit MFMAs and the same ascending-expert combine:
    the row is bit-identical."""
    E, d, mi, k = 32, 512, 128, 8
    gate, up, down = synth.moe_layer_ex(E, d, mi, 77, "int4", 0)
    bank = _upload(ctx, "int4", d, mi, gate, up, down, 0)
    rng = np.random.default_rng(9)
    x = rng.standard_normal((40, d)).astype(np.float32)
    logits = rng.standard_normal((40, E)).astype(np.float32)
    one = bank.forward(x[:1], logits[:1], k, True)
    many = bank.forward(x, logits, k, True)
    assert np.array_equal(one[0].view(np.uint32), many[0].view(np.uint32))


@pytest.mark.parametrize("T", [1, 3])
def test_moe_int4_extreme_row_takes_exact_path(ctx, T):
    """A token row the 24-bit digits cannot carry (one |x| of 1e35) takes
    expert_mm's own order over the stored nibbles.  Input channel 7 has zero
    weights in every gate / up matrix, so the row stays finite."""
    E, d, mi, k = 16, 256, 64, 4
    gate, up, down = synth.moe_layer_ex(E, d, mi, 91, "int4", 0)
    for m in gate + up:  # nibbles of input 7 (high nibble of byte 3) to zero
        m["raw"][:, 3] &= 0x0F
    bank = _upload(ctx, "int4", d, mi, gate, up, down, 0)
    rng = np.random.default_rng(11)
    x = rng.standard_normal((T, d)).astype(np.float32)
    x[0, 7] = np.float32(1.0e35)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    out = bank.forward(x, logits, k, True)
    G, U, D = ([_ex(m, "int4") for m in lst] for lst in (gate, up, down))
    ref = oracle.moe_ex(x, logits, k, True, G, U, D, 0, None)
    assert np.all(np.isfinite(ref)) and np.all(np.isfinite(out))
    rsel, rw, _ = oracle.moe_route(logits, k, True)
    f64 = lambda lst: [oracle.expert_f32(m).astype(np.float64) for m in lst]  # noqa: E731
    B = term_bound(np.where(np.abs(x) > 1e30, 0, x), rsel, rw, f64(G), f64(U), f64(D), 0)
    err = np.abs(out.astype(np.float64) - ref)
    assert np.all(err <= 1e-5 * B), float((err / np.maximum(B, 1e-300)).max())


@pytest.mark.parametrize("dtype", list(DTYPES))
def test_bundle_moe_ex_chain(ctx, dtype):
    """A Qwen3-MoE layer written at `dtype` (router and experts, as
    convert_qwen3moe with --dtype): the bank from frq_bundle_moe equals a
    direct upload bit for bit, and the chain router mm (int4 / q4a) ->
    route -> experts routes as the oracle and matches it (bit-exact, or the
    term bound for int4)."""
    E, d, mi, k, T = 16, 256, 64, 4, 24
    with tempfile.TemporaryDirectory() as tmp:
        stem = os.path.join(tmp, "moe")
        synth.write_qwen3moe_layer_bundle(stem, 5, n_exp=E, d=d, mi=mi, topk=k, dtype=dtype)
        b = fa.Bundle(stem, ctx)
        bank = b.moe("l0.", E)
        assert (bank.d, bank.mi) == (d, mi)
        m, arrs = oracle.read_bundle(stem)
        spec = {a["name"]: a for a in m["arrays"]}

        def mat(name):
            raw = arrs[name]
            if dtype == "f16":
                raw = raw.view(np.uint16)
            sc = arrs.get(name + "__scale")
            mn = arrs.get(name + "__min")
            return {"raw": raw, "scale": None if sc is None else sc.view(np.uint16),
                    "min": None if mn is None else mn.view(np.uint16), "g": int(spec[name].get("group") or 0),
                    "inp": spec[name]["shape"][1 if dtype in ("int4", "q4a") else 0],
                    "out": spec[name]["shape"][0 if dtype in ("int4", "q4a") else 1]}
        gate = [mat(f"l0.experts.{e}.gate") for e in range(E)]
        up = [mat(f"l0.experts.{e}.up") for e in range(E)]
        down = [mat(f"l0.experts.{e}.down") for e in range(E)]
        direct = _upload(ctx, dtype, d, mi, gate, up, down, 0)
        rng = np.random.default_rng(3)
        x = rng.standard_normal((T, d)).astype(np.float32)
        # the router is a Bundle::mm linear in the quantised dtypes; the
        # f16 / f32 dense arms of Bundle::mm are not this library's, so
        # those banks are routed from seeded logits
        logits = (b.mm(x, "l0.gate") if dtype in ("int4", "q4a")
                  else rng.standard_normal((T, E)).astype(np.float32))
        out = bank.forward(x, logits, k, True)
        assert np.array_equal(out.view(np.uint32), direct.forward(x, logits, k, True).view(np.uint32))
        G, U, D = ([_ex(mm_, dtype) for mm_ in lst] for lst in (gate, up, down))
        ref = oracle.moe_ex(x, logits, k, True, G, U, D, 0, None)
        rsel, rw, _ = oracle.moe_route(logits, k, True)
        sel, _ = ctx.moe_route(logits, k, True)
        assert np.array_equal(sel, rsel)
        if dtype != "int4":
            assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
        else:
            f64 = lambda lst: [oracle.expert_f32(mm_).astype(np.float64) for mm_ in lst]  # noqa: E731
            B = term_bound(x, rsel, rw, f64(G), f64(U), f64(D), 0)
            assert np.all(np.abs(out.astype(np.float64) - ref) <= 1e-5 * B)
        bank.free()
        direct.free()
        b.close()
