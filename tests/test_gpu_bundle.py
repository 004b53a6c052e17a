"""A written bundle read back by the library and run on the device: each
weight's device copy computes what the same stored arrays give through the
direct uploads and the oracle (src/bundle.rs:314-376 then mm / rowdot_f32 /
the routed experts)."""
import numpy as np
import pytest

import fieldrun_amd as fa
import oracle
from fieldrun_amd import convert, synth
from fieldrun_amd.bundle import BundleWriter, manifest
from test_gpu_moe import moe_term_bound

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def stem(tmp_path_factory):
    rng = np.random.default_rng(21)
    s = str(tmp_path_factory.mktemp("bundle") / "tiny")
    w = BundleWriter(s)
    w.put_embed("wte", (rng.standard_normal((300, 64)) * 0.02).astype(np.float32), "int8")
    w.put_small("lm_head", (rng.standard_normal((200, 64)) * 0.02).astype(np.float32), None, "f16")
    w.put_lin("q", (rng.standard_normal((96, 64)) * 0.02).astype(np.float32), "int8")     # (out, in)
    w.put_lin("g4", (rng.standard_normal((80, 128)) * 0.02).astype(np.float32), "int4")
    E, d, mi = 4, 64, 32
    for e in range(E):
        w.put_i8(f"l0.experts.{e}.gate", (rng.standard_normal((mi, d)) * 0.02).astype(np.float32), True)
        w.put_i8(f"l0.experts.{e}.up", (rng.standard_normal((mi, d)) * 0.02).astype(np.float32), True)
        w.put_i8(f"l0.experts.{e}.down", (rng.standard_normal((d, mi)) * 0.02).astype(np.float32), True)
    w.put_i8("broken", rng.standard_normal((8, 8)), True)
    w.finish(manifest("rope", [1, 2, 1, 32, 64, 32, 300, 0], [1e6, 1e-6]))
    # drop broken's scale from the manifest: an i8 array without its sibling
    import json
    m = json.load(open(s + ".fieldrun.json"))
    m["arrays"] = [a for a in m["arrays"] if a["name"] != "broken__scale"]
    json.dump(m, open(s + ".fieldrun.json", "w"))
    return s


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_bundle_linears_on_device(ctx, stem):
    b = fa.Bundle(stem, ctx)
    assert b.config_f == [1e6, 1e-6]
    w_kn, s16 = b.arr("q"), b.arr("q__scale")
    wt = np.ascontiguousarray(w_kn.T)
    sc = s16.astype(np.float32)
    for m in (1, 5, 40):
        a = synth.activations(m, 64, 300 + m)
        assert same_bits(b.mm(a, "q"), ctx.upload_i8(wt, sc).mm(a))
        if m <= 16:
            assert same_bits(b.mm(a, "q"), oracle.mm_i8(a, wt, sc))
    # int4: the stored packed bytes and scales, as the direct upload
    packed, s4 = b.arr("g4"), b.arr("g4__scale")
    _, shape, g, _ = b.info("g4")
    a = synth.activations(1, 128, 7, 1.0)
    assert same_bits(b.mm(a, "g4"), ctx.upload_i4(packed, s4, shape[1], g).mm(a))
    b.close()


def test_bundle_row_tables_on_device(ctx, stem):
    b = fa.Bundle(stem, ctx)
    x = np.random.default_rng(5).standard_normal(64).astype(np.float32)
    q, s16 = b.arr("wte"), b.arr("wte__scale")
    assert same_bits(b.rowdot_f32("wte", x), oracle.rowdot_f32("rowi8", q, x, s16.astype(np.float32)))
    h = b.arr("lm_head")
    assert same_bits(b.rowdot_f32("lm_head", x), oracle.rowdot_f32("f16", h.view(np.uint16), x))
    cand = [3, 199, 200, -1]
    assert same_bits(b.rowdot_f32_subset("lm_head", x, cand),
                     oracle.rowdot_f32_subset("f16", h.view(np.uint16), x, cand))
    b.close()


def test_bundle_expert_bank_on_device(ctx, stem):
    b = fa.Bundle(stem, ctx)
    bank = b.moe("l0.", 4, fa.FRQ_ACT_SILU)
    arr = lambda n: b.arr(n)
    sc = lambda n: b.arr(n + "__scale").astype(np.float32)
    direct = ctx.upload_moe_i8([arr(f"l0.experts.{e}.gate") for e in range(4)],
                               [sc(f"l0.experts.{e}.gate") for e in range(4)],
                               [arr(f"l0.experts.{e}.up") for e in range(4)],
                               [sc(f"l0.experts.{e}.up") for e in range(4)],
                               [arr(f"l0.experts.{e}.down") for e in range(4)],
                               [sc(f"l0.experts.{e}.down") for e in range(4)])
    rng = np.random.default_rng(9)
    for T in (1, 6):
        x = rng.standard_normal((T, 64)).astype(np.float32)
        logits = rng.standard_normal((T, 4)).astype(np.float32)
        assert same_bits(bank.forward(x, logits, 2), direct.forward(x, logits, 2))
    b.close()


def test_bundle_upload_errors(ctx, stem):
    b = fa.Bundle(stem, ctx)
    with pytest.raises(fa.FrqError) as e:
        b.weight("broken")
    assert e.value.code == fa.FRQ_ERR_MISSING and "broken__scale" in str(e.value)
    with pytest.raises(fa.FrqError) as e:
        b.weight("absent")
    assert e.value.code == fa.FRQ_ERR_MISSING
    with pytest.raises(fa.FrqError) as e:
        b.moe("l9.", 2)
    assert e.value.code == fa.FRQ_ERR_MISSING
    b.close()


def test_gpt2_config_bundle_on_device(ctx, tmp_path):
    """configs[0]'s shapes (GPT-2 small, one layer): each Conv1D linear read
    from the bundle and run on the device gives the oracle's bits, and the
    tied f16 wte unembed is the reference's rowdot_f32."""
    stem = str(tmp_path / "gpt2")
    synth.write_gpt2_bundle(stem, 5, n_layer=1)
    b = fa.Bundle(stem, ctx)
    for name in ("attn.c_attn", "attn.c_proj", "mlp.c_fc", "mlp.c_proj"):
        w = f"h0.{name}.weight"
        k, n = b.dims(w)
        wt = np.ascontiguousarray(b.arr(w).T)
        sc = b.arr(w + "__scale").astype(np.float32)
        for m in (1, 8):
            a = synth.activations(m, k, 17 * m + n)
            assert same_bits(b.mm(a, w), oracle.mm_i8(a, wt, sc)), (name, m)
    x = np.random.default_rng(6).standard_normal(768).astype(np.float32)
    assert same_bits(b.rowdot_f32("wte", x), oracle.rowdot_f32("f16", b.arr("wte").view(np.uint16), x))
    b.close()


def test_qwen3moe_config_bundle_on_device(ctx, tmp_path):
    """configs[3]'s expert shapes (Qwen3-30B-A3B: d 2048, moe_inter 768, top
    8) with 16 experts: the router is the bundle's int8 l0.gate through mm,
    and the routed layer from the bundle's expert bank matches the oracle
    (the call-site chain of src/qwen3moe.rs:120-158: router mm, softmax,
    top-k, experts, combine)."""
    E, d, mi, k = 16, 2048, 768, 8
    stem = str(tmp_path / "q")
    synth.write_qwen3moe_layer_bundle(stem, 6, n_exp=E, d=d, mi=mi, topk=k)
    b = fa.Bundle(stem, ctx)
    x = np.random.default_rng(8).standard_normal((6, d)).astype(np.float32)
    rt = np.ascontiguousarray(b.arr("l0.gate").T)
    logits = b.mm(x, "l0.gate")
    assert same_bits(logits, oracle.mm_i8(x, rt, b.arr("l0.gate__scale").astype(np.float32)))
    bank = b.moe("l0.", E, fa.FRQ_ACT_SILU)
    lst = lambda fr: [b.arr(f"l0.experts.{e}.{fr}") for e in range(E)]
    scs = lambda fr: [b.arr(f"l0.experts.{e}.{fr}__scale").astype(np.float32) for e in range(E)]
    out = bank.forward(x, logits, k, True)
    ref = oracle.moe(x, logits, k, True, lst("gate"), scs("gate"), lst("up"), scs("up"),
                     lst("down"), scs("down"), 0, None)
    # the logits are the oracle's bits, so the routing is too: every row's
    # experts and weights, and every output within 1e-5 of its terms' bound
    sel, w = ctx.moe_route(logits, k, True)
    rsel, rw, _ = oracle.moe_route(logits, k, True)
    assert np.array_equal(sel, rsel)
    assert np.array_equal(w.view(np.uint32), rw.view(np.uint32))
    B = moe_term_bound(x, rsel, rw, lst("gate"), scs("gate"), lst("up"), scs("up"), lst("down"), scs("down"), 0)
    err = np.abs(out.astype(np.float64) - ref)
    assert np.all(err <= 1e-5 * B), float((err / np.maximum(B, 1e-300)).max())
    b.close()


@pytest.mark.parametrize("dtype,shape", [("i8", [1 << 33, 1 << 31]), ("i4", [1 << 32, 1 << 36]),
                                         ("q4a", [1 << 32, 1 << 36])])
def test_bundle_shape_overflow_is_a_format_error(ctx, tmp_path, dtype, shape):
    """A manifest whose shape products wrap around 2^64 onto the arrays'
    byte counts (0 here: for int4, 2^32 * 2^35 packed bytes and 2^32 * 2^31
    * 2 scale bytes) is refused before any upload reads the blob."""
    import json
    stem = str(tmp_path / "o")
    with open(stem + ".fieldrun.bin", "wb") as f:
        f.write(b"\0" * 64)
    arrays = [{"name": "w", "dtype": dtype, "shape": shape, "offset": 0, "bytes": 0},
              {"name": "w__scale", "dtype": "f16", "shape": [shape[1] if dtype == "i8" else shape[0], 1 << 31],
               "offset": 0, "bytes": 0},
              {"name": "w__min", "dtype": "f16", "shape": [shape[0], 1 << 31], "offset": 0, "bytes": 0}]
    if dtype != "i8":
        arrays[0]["group"] = 32
    m = {"format": "fieldrun-bundle", "version": 1, "arch": "rope", "config": [1], "arrays": arrays}
    with open(stem + ".fieldrun.json", "w") as f:
        json.dump(m, f)
    b = fa.Bundle(stem, ctx)
    with pytest.raises(fa.FrqError) as e:
        b.weight("w")
    assert e.value.code == fa.FRQ_ERR_FORMAT
    b.close()
