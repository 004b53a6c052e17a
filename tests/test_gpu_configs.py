"""The benchmark configs end to end at their full size and length on the
device, against the oracle's golden fixtures (tests/golden, written by
make_config_fixtures.py with the C restatement of Gemma::generate /
Rope::generate on the same seeded bundles and prompts): the greedy tokens,
and every generated token's f32 logits row bit for bit (its SHA-256).

Qwen2.5-7B-shaped int8, all 28 layers, the 2048-token prompt
(the engine's MFMA prefill with the exact epilogue, grouped prefill
attention over 2048 rows) and 128 greedy tokens (long-cache decode to 2175
positions).  configs[2]: Gemma-2-2b-shaped int4, the 64-token prompt and
256 greedy tokens, batch 1, and batch 16 (sixteen prompts decoded together,
each sequence against its own oracle generate)."""
import os
import sys
import tempfile

import numpy as np
import pytest

import fieldrun_amd as fa

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import config_fixtures as cfx  # noqa: E402

pytestmark = pytest.mark.gpu


def shm():
    return "/dev/shm" if os.path.isdir("/dev/shm") else None


@pytest.mark.parametrize("name,engine", [("config4", fa.Rope), ("config2", fa.Gemma), ("config2_b16", fa.Gemma)])
def test_config_full_length_vs_fixture(ctx, name, engine):
    fx = cfx.load_fixture(name)
    assert fx is not None, f"tests/golden/{name}.json missing: run tests/golden/make_config_fixtures.py"
    wl = cfx.WORKLOADS[name]
    with tempfile.TemporaryDirectory(dir=shm()) as tmp:
        stem = os.path.join(tmp, name)
        wl["write"](stem)
        b = fa.Bundle(stem, ctx)
        g = engine(b)
        prompts = wl["prompts"]()
        if len(prompts) == 1:
            toks, lg = g.generate(prompts[0], fx["n_new"], with_logits=True)
            toks, lg = toks[None], lg[None]
        else:  # the batch decode: every sequence its own generate
            toks, lg = g.generate_batch(np.stack(prompts), fx["n_new"], with_logits=True)
            g.set_graphs(True)
            assert np.array_equal(g.generate_batch(np.stack(prompts), fx["n_new"]), toks)
        for i, seq in enumerate(fx["sequences"]):
            same_tok, bad = cfx.compare(seq, toks[i], lg[i])
            assert same_tok, f"sequence {i}: tokens differ"
            assert bad is None, f"sequence {i}: logits row {bad} differs"
        g.free()
        b.close()
