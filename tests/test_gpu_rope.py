"""Llama / Qwen greedy decode on the device (Rope::generate / predict,
src/rope.rs:391-437, 1147-1170) against the oracle's restatement of the
same bundle, tokens and logits bit for bit: Qwen2.5-style (q/k/v biases,
untied lm_head) int8, Qwen3-style (per-head q/k norms, tied) int4, q4a,
the f32 and int8 caches, prompts of 1, 5 and 20 rows (the int8 prefill in
bit-exact chunks), the captured-graph decode equal to the eager one; and
configs[4]'s width (d 3584, 28 / 4 heads of 128, ffn 18944, vocab 152064)
on two layers."""
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


VARIANTS = {
    "qwen25_int8": dict(dtype="int8", qkv_bias=True),
    "qwen3_int4": dict(dtype="int4", qkv_bias=False, qk_norm=True, tied=True),
    "llama_q4a": dict(dtype="q4a", qkv_bias=False),
}


@pytest.fixture(scope="module", params=list(VARIANTS))
def small(request, tmp_path_factory):
    stem = str(tmp_path_factory.mktemp("rope") / request.param)
    synth.write_rope_bundle(stem, 4, n_layer=2, n_head=4, n_kv=2, hd=32, d=128, ffn=256, vocab=500, std=0.1,
                            norm_std=0.1, **VARIANTS[request.param])
    return stem


@pytest.mark.parametrize("kv_int8", [False, True])
@pytest.mark.parametrize("P", [1, 5, 20])
def test_rope_generate_matches_oracle(ctx, small, kv_int8, P):
    m, arrs = oracle.read_bundle(small)
    ref = oracle.Rope(m, arrs, nthreads=8)
    b = fa.Bundle(small, ctx)
    g = fa.Rope(b, kv_int8)
    prompt = synth.gpt2_prompt(P, 500, P + 11)
    toks, lg = g.generate(prompt, 12, with_logits=True)
    rt, rlg = ref.generate(prompt, 12, kv_int8=kv_int8, with_logits=True)
    assert np.array_equal(toks, rt)
    assert same_bits(lg, rlg), first_diff(lg, rlg)
    assert np.array_equal(g.generate(prompt, 12), toks)       # the captured-graph decode
    t1, l1 = g.predict(prompt, with_logits=True)
    assert t1 == toks[0] and same_bits(l1, lg[0])
    g.free()
    b.close()


def test_rope_rejects_other_archs(ctx, tmp_path):
    stem = str(tmp_path / "g")
    synth.write_gemma2_bundle(stem, 1, n_layer=1, n_head=2, n_kv=1, hd=16, d=32, ffn=64, vocab=50)
    b = fa.Bundle(stem, ctx)
    with pytest.raises(fa.FrqError) as e:
        fa.Rope(b)
    assert e.value.code == fa.FRQ_ERR_FORMAT
    b.close()


def test_config4_width_two_layers(ctx, tmp_path):
    """configs[4]'s layer width (Qwen2.5-7B: d 3584, 28 / 4 heads of 128,
    ffn 18944, vocab 152064, int8 with q/k/v biases, untied head) on two
    layers: a 20-token prompt through the chunked bit-exact int8 prefill,
    then decode, bit for bit."""
    stem = str(tmp_path / "q7")
    synth.write_rope_bundle(stem, 6, n_layer=2, raw=True)
    m, arrs = oracle.read_bundle(stem)
    ref = oracle.Rope(m, arrs, nthreads=16)
    b = fa.Bundle(stem, ctx)
    g = fa.Rope(b)
    prompt = synth.gpt2_prompt(20, 152064, 9)
    toks, lg = g.generate(prompt, 5, with_logits=True)
    rt, rlg = ref.generate(prompt, 5, with_logits=True)
    assert np.array_equal(toks, rt)
    assert same_bits(lg, rlg), first_diff(lg, rlg)
    g.free()
    b.close()


@pytest.mark.parametrize("hd", [32, 128])
@pytest.mark.parametrize("kv_int8", [False, True])
def test_rope_long_cache_decode(ctx, tmp_path, kv_int8, hd):
    """Caches past 512 positions take the three-launch decode attention
    (scores over many blocks, then the key-order softmax and value chains):
    the same bits as the oracle."""
    stem = str(tmp_path / "r")
    synth.write_rope_bundle(stem, 12, n_layer=2, n_head=4, n_kv=2, hd=hd, d=4 * hd, ffn=256, vocab=500, std=0.1,
                            norm_std=0.1, dtype="int8", qk_norm=True)
    m, arrs = oracle.read_bundle(stem)
    ref = oracle.Rope(m, arrs, nthreads=16)
    b = fa.Bundle(stem, ctx)
    g = fa.Rope(b, kv_int8)
    prompt = synth.gpt2_prompt(600, 500, 13)
    toks, lg = g.generate(prompt, 6, with_logits=True)
    rt, rlg = ref.generate(prompt, 6, kv_int8=kv_int8, with_logits=True)
    assert np.array_equal(toks, rt)
    assert same_bits(lg, rlg), first_diff(lg, rlg)
    assert np.array_equal(g.generate(prompt, 6), toks)
    g.free()
    b.close()


def test_rope_batch_matches_single_sequences(ctx, small):
    """The batch decode on the Llama / Qwen family: every row its own
    Rope::generate, bit for bit."""
    b = fa.Bundle(small, ctx)
    g = fa.Rope(b)
    prompts = np.stack([synth.gpt2_prompt(6, 500, 70 + i) for i in range(4)])
    toks, lg = g.generate_batch(prompts, 9, with_logits=True)
    for i in range(len(prompts)):
        t1, l1 = g.generate(prompts[i], 9, with_logits=True)
        assert np.array_equal(toks[i], t1), i
        assert same_bits(lg[i], l1), (i, first_diff(lg[i], l1))
    g.free()
    b.close()


@pytest.mark.parametrize("n_head,n_kv,hd", [(8, 2, 64), (20, 4, 32)])
def test_rope_long_prompt_two_launch_attention(ctx, tmp_path, n_head, n_kv, hd):
    """Prompts of 1024 rows and more take the two-launch prefill attention
    (scores tiled over blocks of rows and 128-key tiles, then the exps,
    key-order sums and value chains per block of rows): tokens and logits
    bit for bit against the oracle, at 4 and 5 query heads a kv head."""
    stem = str(tmp_path / "r")
    synth.write_rope_bundle(stem, 21, n_layer=2, n_head=n_head, n_kv=n_kv, hd=hd, d=n_head * hd, ffn=256,
                            vocab=500, std=0.1, norm_std=0.1, dtype="int8")
    m, arrs = oracle.read_bundle(stem)
    ref = oracle.Rope(m, arrs, nthreads=16)
    b = fa.Bundle(stem, ctx)
    g = fa.Rope(b)
    prompt = synth.gpt2_prompt(1100, 500, 23)
    toks, lg = g.generate(prompt, 4, with_logits=True)
    rt, rlg = ref.generate(prompt, 4, with_logits=True)
    assert np.array_equal(toks, rt)
    assert same_bits(lg, rlg), first_diff(lg, rlg)
    g.free()
    b.close()
