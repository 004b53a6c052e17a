"""GPT-2 greedy decode on the device (Gpt2::generate / predict,
src/composition.rs:175-341) against the oracle's restatement on the same
bundle: identical greedy tokens and bit-identical logits, for the f32 and
the int8 KV cache, prompts of 1 row, 2..16 rows and more (chunked), the
captured-graph decode equal to the eager one, and configs[0] (GPT-2 small,
random init) at full size."""
import numpy as np
import pytest

import fieldrun_amd as fa
import oracle
from fieldrun_amd import synth

pytestmark = pytest.mark.gpu


def bundle(tmp_path_factory, name, s, **kw):
    stem = str(tmp_path_factory.mktemp("gpt2") / name)
    synth.write_gpt2_bundle(stem, s, **kw)
    return stem


@pytest.fixture(scope="module")
def lively(tmp_path_factory):
    # std 0.2: the layers move the residual stream, so the tokens vary
    return bundle(tmp_path_factory, "lively", 31, n_layer=3, n_head=4, d=128, n_pos=96, vocab=700, std=0.2)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def first_diff(lg, rlg):
    """(step, max |diff|) of the first step whose logits differ, for the
    failure message."""
    for s in range(len(rlg)):
        if not same_bits(lg[s], rlg[s]):
            return s, float(np.abs(lg[s] - rlg[s]).max())
    return None


@pytest.mark.parametrize("kv_int8", [False, True])
@pytest.mark.parametrize("P", [1, 5, 16, 40])
def test_generate_matches_oracle(ctx, lively, kv_int8, P):
    m, arrs = oracle.read_bundle(lively)
    ref = oracle.Gpt2(m, arrs, nthreads=8)
    b = fa.Bundle(lively, ctx)
    g = fa.Gpt2(b, kv_int8)
    prompt = np.random.default_rng(P).integers(0, 700, P)
    n_new = 24
    toks, lg = g.generate(prompt, n_new, with_logits=True)
    rt, rlg = ref.generate(prompt, n_new, kv_int8=kv_int8, with_logits=True)
    assert np.array_equal(toks, rt)
    assert same_bits(lg, rlg), first_diff(lg, rlg)
    assert len(set(toks.tolist())) > 3
    g.free()
    b.close()


@pytest.mark.parametrize("kv_int8", [False, True])
def test_graph_decode_equals_eager(ctx, lively, kv_int8):
    b = fa.Bundle(lively, ctx)
    g = fa.Gpt2(b, kv_int8)
    prompt = np.random.default_rng(9).integers(0, 700, 12)
    eager, _ = g.generate(prompt, 40, with_logits=True)   # eager path (logits kept)
    g.set_graphs(False)
    eager2 = g.generate(prompt, 40)
    g.set_graphs(True)
    graph = g.generate(prompt, 40)
    again = g.generate(prompt, 40)      # a fresh capture on a used model
    short = g.generate(prompt[:3], 7)   # another shape in between
    graph3 = g.generate(prompt, 40)
    assert np.array_equal(eager, eager2)
    assert np.array_equal(eager, graph) and np.array_equal(graph, again) and np.array_equal(graph, graph3)
    g.set_graphs(False)
    assert np.array_equal(short, g.generate(prompt[:3], 7))
    g.free()
    b.close()


def test_predict_matches_oracle(ctx, lively):
    m, arrs = oracle.read_bundle(lively)
    ref = oracle.Gpt2(m, arrs, nthreads=8)
    b = fa.Bundle(lively, ctx)
    g = fa.Gpt2(b)
    for n in (1, 9, 33):
        ids = np.random.default_rng(50 + n).integers(0, 700, n)
        t, lg = g.predict(ids, with_logits=True)
        rt, rlg = ref.predict(ids, with_logits=True)
        assert t == rt
        assert same_bits(lg, rlg)
    g.free()
    b.close()


def test_gpt2_errors(ctx, lively, tmp_path):
    b = fa.Bundle(lively, ctx)
    g = fa.Gpt2(b)
    with pytest.raises(fa.FrqError) as e:
        g.generate([1, 700], 3)
    assert e.value.code == fa.FRQ_ERR_ARG
    with pytest.raises(fa.FrqError) as e:
        g.generate(np.zeros(90, np.int64), 8)    # position 96 past n_positions
    assert e.value.code == fa.FRQ_ERR_ARG and "n_positions" in str(e.value)
    with pytest.raises(fa.FrqError) as e:
        g.generate([], 3)
    assert e.value.code == fa.FRQ_ERR_ARG
    # the longest generate that fits: positions up to n_pos - 1
    assert len(g.generate(np.zeros(90, np.int64), 7)) == 7
    g.free()
    b.close()
    # a bundle that is not gpt2
    stem = str(tmp_path / "q")
    synth.write_qwen3moe_layer_bundle(stem, 1, n_exp=2, d=64, mi=16, topk=1)
    bq = fa.Bundle(stem, ctx)
    with pytest.raises(fa.FrqError) as e:
        fa.Gpt2(bq)
    assert e.value.code == fa.FRQ_ERR_FORMAT
    bq.close()


@pytest.mark.parametrize("kv_int8", [False, True])
def test_config0_gpt2_small_greedy_tokens(ctx, tmp_path_factory, kv_int8):
    """GPT-2 small int8, random init (std 0.02), 32-token seeded
    prompt, 128 greedy tokens: identical to the oracle, logits bit for bit."""
    stem = bundle(tmp_path_factory, "config0", 1234)
    m, arrs = oracle.read_bundle(stem)
    ref = oracle.Gpt2(m, arrs, nthreads=16)
    b = fa.Bundle(stem, ctx)
    g = fa.Gpt2(b, kv_int8)
    prompt = synth.gpt2_prompt(32, 50257, 7)
    toks, lg = g.generate(prompt, 128, with_logits=True)
    rt, rlg = ref.generate(prompt, 128, kv_int8=kv_int8, with_logits=True)
    assert np.array_equal(toks, rt)
    assert same_bits(lg, rlg), first_diff(lg, rlg)
    assert np.array_equal(g.generate(prompt, 128), toks)   # the graph path
    g.free()
    b.close()
