"""Gemma-2 greedy decode on the device (Gemma::generate / predict,
src/gemma.rs:242-441) against the oracle's restatement of the same bundle:
tokens and logits bit for bit, for int4 / int8 / q4a linears, the f32 and
int8 caches, prompts of 1, 5, 20 rows, the captured-graph decode equal to
the eager one, the sliding window (a prompt past 4096 positions), and
configs[2] (Gemma-2-2b, int4) at full size on a short sample."""
import numpy as np
import pytest

import fieldrun_amd as fa
import oracle
from fieldrun_amd import synth

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def first_diff(lg, rlg):
    for s in range(len(rlg)):
        if not same_bits(lg[s], rlg[s]):
            return s, float(np.abs(lg[s] - rlg[s]).max())
    return None


@pytest.fixture(scope="module", params=["int4", "int8", "q4a"])
def small(request, tmp_path_factory):
    stem = str(tmp_path_factory.mktemp("gemma") / request.param)
    synth.write_gemma2_bundle(stem, 7, n_layer=2, n_head=4, n_kv=2, hd=32, d=128, ffn=256, vocab=500, std=0.05,
                              dtype=request.param, norm_std=0.1)
    return stem


@pytest.mark.parametrize("kv_int8", [False, True])
@pytest.mark.parametrize("P", [1, 5, 20])
def test_gemma_generate_matches_oracle(ctx, small, kv_int8, P):
    m, arrs = oracle.read_bundle(small)
    ref = oracle.Gemma(m, arrs, nthreads=8)
    b = fa.Bundle(small, ctx)
    g = fa.Gemma(b, kv_int8)
    prompt = synth.gpt2_prompt(P, 500, P + 3)
    toks, lg = g.generate(prompt, 12, with_logits=True)
    rt, rlg = ref.generate(prompt, 12, kv_int8=kv_int8, with_logits=True)
    assert np.array_equal(toks, rt)
    assert same_bits(lg, rlg), first_diff(lg, rlg)
    g.set_graphs(True)
    assert np.array_equal(g.generate(prompt, 12), toks)       # the captured-graph decode
    t1, l1 = g.predict(prompt, with_logits=True)
    assert t1 == toks[0] and same_bits(l1, lg[0])
    g.free()
    b.close()


def test_gemma_sliding_window(ctx, tmp_path):
    """Layer 0 (even) attends over the last 4096 positions only: a prompt of
    4100 rows puts the window's lower edge inside the cache."""
    stem = str(tmp_path / "w")
    synth.write_gemma2_bundle(stem, 8, n_layer=2, n_head=2, n_kv=1, hd=16, d=32, ffn=64, vocab=300, std=0.1,
                              norm_std=0.1)
    m, arrs = oracle.read_bundle(stem)
    ref = oracle.Gemma(m, arrs, nthreads=16)
    b = fa.Bundle(stem, ctx)
    g = fa.Gemma(b)
    prompt = synth.gpt2_prompt(4100, 300, 5)
    toks, lg = g.generate(prompt, 3, with_logits=True)
    rt, rlg = ref.generate(prompt, 3, with_logits=True)
    assert np.array_equal(toks, rt)
    assert same_bits(lg, rlg), first_diff(lg, rlg)
    g.free()
    b.close()


def test_gemma_errors(ctx, small, tmp_path):
    b = fa.Bundle(small, ctx)
    g = fa.Gemma(b)
    with pytest.raises(fa.FrqError) as e:
        g.generate([1, 500], 2)
    assert e.value.code == fa.FRQ_ERR_ARG
    g.free()
    b.close()
    stem = str(tmp_path / "gpt2")
    synth.write_gpt2_bundle(stem, 1, n_layer=1, n_head=2, d=32, n_pos=8, vocab=40)
    b2 = fa.Bundle(stem, ctx)
    with pytest.raises(fa.FrqError) as e:
        fa.Gemma(b2)
    assert e.value.code == fa.FRQ_ERR_FORMAT
    b2.close()


def test_config2_gemma2_2b_int4(ctx, tmp_path):
    """Gemma-2-2b shapes (26 layers, d 2304, 8 / 4 heads of 256,
    ffn 9216, vocab 256000, int4 g=32, f16 embed), a seeded prompt: tokens
    and logits bit for bit on a short sample (the oracle is a CPU restatement)."""
    stem = str(tmp_path / "g2")
    synth.write_gemma2_bundle(stem, 2, raw=True)
    m, arrs = oracle.read_bundle(stem)
    ref = oracle.Gemma(m, arrs, nthreads=16)
    b = fa.Bundle(stem, ctx)
    g = fa.Gemma(b)
    prompt = synth.gpt2_prompt(8, 256000, 3)
    toks, lg = g.generate(prompt, 4, with_logits=True)
    rt, rlg = ref.generate(prompt, 4, with_logits=True)
    assert np.array_equal(toks, rt)
    assert same_bits(lg, rlg), first_diff(lg, rlg)
    g.free()
    b.close()


@pytest.mark.parametrize("kv_int8", [False, True])
def test_gemma_long_cache_decode(ctx, tmp_path, kv_int8):
    """The three-launch decode attention (caches past 512 positions) with
    Gemma's soft-cap: the same bits as the oracle."""
    stem = str(tmp_path / "g")
    synth.write_gemma2_bundle(stem, 13, n_layer=2, n_head=4, n_kv=2, hd=32, d=128, ffn=256, vocab=500, std=0.05,
                              norm_std=0.1)
    m, arrs = oracle.read_bundle(stem)
    ref = oracle.Gemma(m, arrs, nthreads=16)
    b = fa.Bundle(stem, ctx)
    g = fa.Gemma(b, kv_int8)
    prompt = synth.gpt2_prompt(600, 500, 14)
    toks, lg = g.generate(prompt, 6, with_logits=True)
    rt, rlg = ref.generate(prompt, 6, kv_int8=kv_int8, with_logits=True)
    assert np.array_equal(toks, rt)
    assert same_bits(lg, rlg), first_diff(lg, rlg)
    assert np.array_equal(g.generate(prompt, 6), toks)
    g.free()
    b.close()


def test_gemma_refused_length_leaves_model_usable(ctx, small):
    """A generate whose cache the attention cannot hold is refused with
    FRQ_ERR_ARG before anything changes; the same handle then still decodes
    bit for bit (before and after a successful call)."""
    m, arrs = oracle.read_bundle(small)
    ref = oracle.Gemma(m, arrs, nthreads=8)
    prompt = synth.gpt2_prompt(5, 500, 21)
    rt, rlg = ref.generate(prompt, 4, with_logits=True)
    b = fa.Bundle(small, ctx)
    g = fa.Gemma(b)
    for first in (True, False):
        if not first:
            toks, lg = g.generate(prompt, 4, with_logits=True)
            assert np.array_equal(toks, rt) and same_bits(lg, rlg)
        with pytest.raises(fa.FrqError) as e:
            g.generate(prompt, 40000)
        assert e.value.code == fa.FRQ_ERR_ARG
        toks, lg = g.generate(prompt, 4, with_logits=True)
        assert np.array_equal(toks, rt)
        assert same_bits(lg, rlg), first_diff(lg, rlg)
    g.free()
    b.close()


def test_gemma_cache_past_64k_of_scores(ctx, tmp_path):
    """A cache of 8300 positions (Gemma-2's 8192-token context and more):
    the one-launch prefill attention (one query head per kv head, so not the
    grouped kernel) and the long-cache decode split hold more than 64 KB of
    scores in LDS; tokens and logits bit for bit."""
    stem = str(tmp_path / "l")
    synth.write_gemma2_bundle(stem, 17, n_layer=2, n_head=2, n_kv=2, hd=16, d=32, ffn=64, vocab=300, std=0.1,
                              norm_std=0.1)
    m, arrs = oracle.read_bundle(stem)
    ref = oracle.Gemma(m, arrs, nthreads=16)
    b = fa.Bundle(stem, ctx)
    g = fa.Gemma(b)
    prompt = synth.gpt2_prompt(8300, 300, 6)
    toks, lg = g.generate(prompt, 3, with_logits=True)
    rt, rlg = ref.generate(prompt, 3, with_logits=True)
    assert np.array_equal(toks, rt)
    assert same_bits(lg, rlg), first_diff(lg, rlg)
    g.free()
    b.close()


@pytest.mark.parametrize("kv_int8", [False, True])
def test_gemma_batch_matches_single_sequences(ctx, small, kv_int8):
    """configs[2]'s batch decode: each row of a batch is its own
    Gemma::generate (the reference has no batched generate), so the batch
    gives, bit for bit, the tokens and logits of one call a sequence, and of
    the oracle (int4 rows in i4_dot_avx2's order, q4a / int8 rows as at
    M == 1); the captured-graph batch decode gives the same tokens."""
    m, arrs = oracle.read_bundle(small)
    ref = oracle.Gemma(m, arrs, nthreads=8)
    b = fa.Bundle(small, ctx)
    g = fa.Gemma(b, kv_int8)
    prompts = np.stack([synth.gpt2_prompt(5, 500, 40 + i) for i in range(5)])
    toks, lg = g.generate_batch(prompts, 12, with_logits=True)
    for i in range(len(prompts)):
        t1, l1 = g.generate(prompts[i], 12, with_logits=True)
        assert np.array_equal(toks[i], t1), i
        assert same_bits(lg[i], l1), (i, first_diff(lg[i], l1))
        rt, rlg = ref.generate(prompts[i], 12, kv_int8=kv_int8, with_logits=True)
        assert np.array_equal(toks[i], rt) and same_bits(lg[i], rlg), i
    g.set_graphs(True)
    assert np.array_equal(g.generate_batch(prompts, 12), toks)
    g.free()
    b.close()


def test_gemma_batch_long_cache_and_sixteen_rows(ctx, tmp_path):
    """A batch of 16 sequences (the int4 linears' widest batch in one pass)
    past 512 positions (the long-cache attention, a sequence at a time)."""
    stem = str(tmp_path / "g")
    synth.write_gemma2_bundle(stem, 23, n_layer=2, n_head=4, n_kv=2, hd=32, d=128, ffn=256, vocab=500, std=0.05,
                              norm_std=0.1)
    b = fa.Bundle(stem, ctx)
    g = fa.Gemma(b)
    prompts = np.stack([synth.gpt2_prompt(520, 500, 60 + i) for i in range(16)])
    toks, lg = g.generate_batch(prompts, 3, with_logits=True)
    for i in (0, 7, 15):
        t1, l1 = g.generate(prompts[i], 3, with_logits=True)
        assert np.array_equal(toks[i], t1) and same_bits(lg[i], l1), i
    g.set_graphs(True)
    assert np.array_equal(g.generate_batch(prompts, 3), toks)
    g.free()
    b.close()


@pytest.mark.parametrize("embed,d", [("f32", 132), ("int8", 132), ("f16", 132), ("f16", 196)])
def test_gemma_batch_head_table_types(ctx, tmp_path, embed, d):
    """The batched head (the tied table's row dot and argmax for every
    sequence in one pass, the vectors zero-padded to 4, 8 or 16) on f32, f16
    and rowi8 tables, rows ending inside a 128-byte chunk: bit for bit the
    one-sequence head, and the oracle."""
    stem = str(tmp_path / "g")
    synth.write_gemma2_bundle(stem, 29, n_layer=2, n_head=4, n_kv=2, hd=32, d=d, ffn=256, vocab=700, std=0.05,
                              norm_std=0.1, embed=embed)
    m, arrs = oracle.read_bundle(stem)
    ref = oracle.Gemma(m, arrs, nthreads=8)
    b = fa.Bundle(stem, ctx)
    g = fa.Gemma(b)
    for nb in (3, 9):
        prompts = np.stack([synth.gpt2_prompt(4, 700, 90 + nb + i) for i in range(nb)])
        toks, lg = g.generate_batch(prompts, 4, with_logits=True)
        for i in range(nb):
            t1, l1 = g.generate(prompts[i], 4, with_logits=True)
            assert np.array_equal(toks[i], t1) and same_bits(lg[i], l1), (nb, i, first_diff(lg[i], l1))
        rt, rlg = ref.generate(prompts[nb - 1], 4, with_logits=True)
        assert np.array_equal(toks[nb - 1], rt) and same_bits(lg[nb - 1], rlg), nb
    g.free()
    b.close()


def test_gemma_batch_errors(ctx, small):
    b = fa.Bundle(small, ctx)
    g = fa.Gemma(b)
    with pytest.raises(fa.FrqError) as e:
        g.generate_batch(np.array([[1, 2], [3, 500]]), 2)
    assert e.value.code == fa.FRQ_ERR_ARG
    g.free()
    b.close()
