"""Parity of the gfx950 routed-expert layer against the CPU oracle.

Routing: selected experts identical and combine weights bit-identical (the
device runs the restated glibc expf, as Rust's f32::exp reaches it; ties ->
lower expert id, as the stable sort in src/qwen3moe.rs:129).  expert_mm:
bit-exact (same sequential-k FMA order).  Layer output: every element within
1e-5 of the sum of the magnitudes of its terms (moe_term_bound), for every
token, with every token's expert set identical to the oracle's.
"""
import numpy as np
import pytest

import oracle
from fieldrun_amd import synth
import fieldrun_amd as fa

pytestmark = pytest.mark.gpu


def _silu(g):
    return g / (1.0 + np.exp(-g))


def _gelu(g):
    return 0.5 * g * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g + 0.044715 * g ** 3)))


def moe_term_bound(x, sel, w, gate, gs, up, us, down, ds, act):
    """f64 bound per output element (t, c): sum over t's experts of |w| *
    sum_j (|h_j| + dh_j) * |down[j, c]|, where dh_j bounds how far an
    error of the gate / up sums (relative to the magnitudes of their terms)
    moves h_j = act(g_j) * u_j.  The device rounds each row to 24 bits
    before its exact integer products; the reference sums in f32."""
    T, d = x.shape
    B = np.zeros((T, d))
    X = x.astype(np.float64)
    for e in range(len(gate)):
        tok, slot = np.nonzero(sel == e)
        if not len(tok):
            continue
        Xe, Ae = X[tok], np.abs(X[tok])
        G = gate[e].astype(np.float64) * gs[e]
        g, Sg = Xe @ G, Ae @ np.abs(G)
        if act == 0:
            U = up[e].astype(np.float64) * us[e]
            u, Su = Xe @ U, Ae @ np.abs(U)
            a = _silu(g)
            h = a * u
            dh = 1.1 * np.abs(u) * Sg + np.abs(a) * Su
        else:
            mi = G.shape[1] // 2
            a = _gelu(g[:, :mi])
            h = a * g[:, mi:]
            dh = 1.2 * np.abs(g[:, mi:]) * Sg[:, :mi] + np.abs(a) * Sg[:, mi:]
        D = np.abs(down[e].astype(np.float64) * ds[e])
        np.add.at(B, tok, np.abs(w[tok, slot])[:, None] * ((np.abs(h) + dh) @ D))
    return B


@pytest.mark.parametrize("T,E,k,norm", [(1, 128, 8, True), (512, 128, 8, True), (37, 60, 4, False),
                                        (5, 8, 8, True), (64, 128, 1, True), (9, 300, 5, True),
                                        (6, 200, 12, False)])
def test_route_parity(ctx, T, E, k, norm):
    rng = np.random.default_rng(T * 31 + E)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    if T > 3:
        logits[2, 1] = logits[2, E - 2] = 7.0  # exact tie: the lower expert first
    sel, w = ctx.moe_route(logits, k, norm)
    rsel, rw, _ = oracle.moe_route(logits, k, norm)
    assert np.array_equal(sel, rsel)
    assert np.array_equal(w.view(np.uint32), rw.view(np.uint32))
    pes = rng.uniform(0.5, 1.5, E).astype(np.float32)
    sel2, w2 = ctx.moe_route(logits, k, True, pes)
    rsel2, rw2, _ = oracle.moe_route(logits, k, True, pes)
    assert np.array_equal(sel2, rsel2)
    assert np.array_equal(w2.view(np.uint32), rw2.view(np.uint32))


def test_route_nan_is_an_error(ctx):
    logits = np.zeros((3, 16), np.float32)
    logits[1, 3] = np.nan
    with pytest.raises(fa.FrqError) as ei:
        ctx.moe_route(logits, 2)
    assert ei.value.code == fa.FRQ_ERR_NAN


@pytest.mark.parametrize("E", [16, 100, 300])
def test_route_infinite_max_is_an_error(ctx, E):
    """A +inf logit (inf - inf in its exponent) or a row of -inf makes the
    reference's probabilities NaN, and its sort's partial_cmp().unwrap()
    panics (src/qwen3moe.rs:47-51, 129): an error, as for a NaN logit."""
    logits = np.zeros((3, E), np.float32)
    logits[1, E - 1] = np.inf
    with pytest.raises(fa.FrqError) as ei:
        ctx.moe_route(logits, 2)
    assert ei.value.code == fa.FRQ_ERR_NAN
    logits = np.zeros((2, E), np.float32)
    logits[0, :] = -np.inf
    with pytest.raises(fa.FrqError) as ei:
        ctx.moe_route(logits, 2)
    assert ei.value.code == fa.FRQ_ERR_NAN


@pytest.mark.parametrize("act", [0, 1])
def test_expert_mm_bit_exact(ctx, act):
    E, d, mi = 4, 256, 96
    gate, gs, up, us, down, ds = synth.moe_layer(E, d, mi, 50 + act, act)
    bank = ctx.upload_moe_i8(gate, gs, up, us, down, ds, act)
    rng = np.random.default_rng(act)
    x = rng.standard_normal((5, d)).astype(np.float32)
    for e in range(E):
        y = bank.expert_mm(0, e, x)
        assert np.array_equal(y.view(np.uint32), oracle.expert_mm_i8(x, gate[e], gs[e]).view(np.uint32))
        h = rng.standard_normal((3, mi)).astype(np.float32)
        y = bank.expert_mm(2, e, h)
        assert np.array_equal(y.view(np.uint32), oracle.expert_mm_i8(h, down[e], ds[e]).view(np.uint32))


@pytest.mark.parametrize("T,E,d,mi,k,act", [(1, 16, 256, 64, 4, 0), (40, 16, 256, 64, 4, 0),
                                            (7, 8, 128, 32, 8, 1), (1, 128, 2048, 768, 8, 0),
                                            (64, 128, 2048, 768, 8, 0), (1, 8, 128, 32, 8, 1),
                                            (1, 60, 256, 64, 4, 0), (1, 32, 320, 96, 16, 1),
                                            (512, 128, 2048, 768, 8, 0), (1, 16, 256, 40, 4, 1),
                                            (1, 300, 256, 64, 6, 0), (300, 8, 256, 64, 4, 0),
                                            (90, 12, 320, 48, 3, 1)])
def test_moe_layer_parity(ctx, T, E, d, mi, k, act):
    gate, gs, up, us, down, ds = synth.moe_layer(E, d, mi, synth.seed(3) + T + act, act)
    bank = ctx.upload_moe_i8(gate, gs, up, us, down, ds, act)
    rng = np.random.default_rng(T + E)
    x = rng.standard_normal((T, d)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    pes = rng.uniform(0.5, 1.5, E).astype(np.float32) if act else None
    out = bank.forward(x, logits, k, True, pes)
    ref = oracle.moe(x, logits, k, True, gate, gs, up, us, down, ds, act, pes, nthreads=16)
    sel, w = ctx.moe_route(logits, k, True, pes)
    rsel, rw, _ = oracle.moe_route(logits, k, True, pes)
    assert np.array_equal(sel, rsel)
    B = moe_term_bound(x, rsel, rw, gate, gs, up, us, down, ds, act)
    err = np.abs(out.astype(np.float64) - ref)
    assert np.all(err <= 1e-5 * B), float((err / np.maximum(B, 1e-300)).max())


@pytest.mark.parametrize("act", [0, 1])
def test_moe_decode_matches_batched_row(ctx, act):
    """T == 1 runs the two-launch decode path; the same token inside a
    batch runs the general pipeline.  Both compute the same digit GEMMs and
    the same ascending-expert combine, so the row is bit-identical."""
    E, d, mi, k = 32, 512, 128, 8
    gate, gs, up, us, down, ds = synth.moe_layer(E, d, mi, synth.seed(3) + 77 + act, act)
    bank = ctx.upload_moe_i8(gate, gs, up, us, down, ds, act)
    rng = np.random.default_rng(5 + act)
    x = rng.standard_normal((3, d)).astype(np.float32)
    logits = rng.standard_normal((3, E)).astype(np.float32)
    pes = rng.uniform(0.5, 1.5, E).astype(np.float32) if act else None
    one = bank.forward(x[:1], logits[:1], k, True, pes)
    many = bank.forward(x, logits, k, True, pes)
    assert np.array_equal(one[0].view(np.uint32), many[0].view(np.uint32))


@pytest.mark.parametrize("T", [1, 3])
def test_moe_extreme_row_takes_exact_path(ctx, T):
    """A token row whose digit scale leaves the exact range (one |x| of
    1e35) takes the reference's sequential expert sum, in the decode
    kernels (T == 1) and in the batched pipeline.  Input channel 7 has zero
    weights in every gate / up matrix, so the row's outputs stay finite and
    the exact path's arithmetic is compared value by value."""
    E, d, mi, k = 16, 256, 64, 4
    gate, gs, up, us, down, ds = synth.moe_layer(E, d, mi, synth.seed(3) + 91, 0)
    for e in range(E):
        gate[e][7, :] = 0
        up[e][7, :] = 0
    bank = ctx.upload_moe_i8(gate, gs, up, us, down, ds, 0)
    rng = np.random.default_rng(11)
    x = rng.standard_normal((T, d)).astype(np.float32)
    x[0, 7] = np.float32(1.0e35)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    out = bank.forward(x, logits, k, True)
    ref = oracle.moe(x, logits, k, True, gate, gs, up, us, down, ds, 0, None)
    assert np.all(np.isfinite(ref)) and np.all(np.isfinite(out))
    rsel, rw, _ = oracle.moe_route(logits, k, True)
    B = moe_term_bound(np.where(np.abs(x) > 1e30, 0, x), rsel, rw, gate, gs, up, us, down, ds, 0)
    err = np.abs(out.astype(np.float64) - ref)
    assert np.all(err <= 1e-5 * B), float((err / np.maximum(B, 1e-300)).max())


def test_moe_decode_nan_logits_is_an_error(ctx):
    E, d, mi, k = 16, 256, 64, 4
    gate, gs, up, us, down, ds = synth.moe_layer(E, d, mi, synth.seed(3) + 92, 0)
    bank = ctx.upload_moe_i8(gate, gs, up, us, down, ds, 0)
    x = np.ones((1, d), np.float32)
    logits = np.zeros((1, E), np.float32)
    logits[0, 2] = np.nan
    with pytest.raises(Exception):
        bank.forward(x, logits, k, True)
    logits[0, 2] = np.inf
    with pytest.raises(Exception):
        bank.forward(x, logits, k, True)
