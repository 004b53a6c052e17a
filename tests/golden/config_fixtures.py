"""The end-to-end workloads behind the golden fixtures (written by
make_config_fixtures.py through the CPU oracle) and the checks against
them, shared by the GPU tests and bench.py: the same seeded bundle, the same
prompts, the tokens and the SHA-256 of every logits row."""
import hashlib
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def _synth():
    from fieldrun_amd import synth
    return synth


WORKLOADS = {
    "config4": {
        "what": "configs[4]: Qwen2.5-7B-shaped int8 bundle (write_rope_bundle(stem, 6, raw=True)), "
                "prompt gpt2_prompt(2048, 152064, 9), 128 greedy tokens, f32 KV cache",
        "write": lambda stem: _synth().write_rope_bundle(stem, 6, raw=True),
        "prompts": lambda: [_synth().gpt2_prompt(2048, 152064, 9)],
        "n_new": 128, "arch": "rope",
    },
    "config2": {
        "what": "configs[2]: Gemma-2-2b-shaped int4 bundle (write_gemma2_bundle(stem, 2, raw=True)), "
                "prompt gpt2_prompt(64, 256000, 7), 256 greedy tokens, batch 1, f32 KV cache",
        "write": lambda stem: _synth().write_gemma2_bundle(stem, 2, raw=True),
        "prompts": lambda: [_synth().gpt2_prompt(64, 256000, 7)],
        "n_new": 256, "arch": "gemma",
    },
    "config2_b16": {
        "what": "configs[2] batch 16: the configs[2] bundle, prompts gpt2_prompt(64, 256000, 100 + i) for "
                "i < 16, 256 greedy tokens each, every sequence its own batch-1 generate",
        "write": lambda stem: _synth().write_gemma2_bundle(stem, 2, raw=True),
        "prompts": lambda: [_synth().gpt2_prompt(64, 256000, 100 + i) for i in range(16)],
        "n_new": 256, "arch": "gemma",
    },
}


def fixture_path(name: str) -> str:
    return os.path.join(HERE, f"{name}.json")


def load_fixture(name: str):
    """The fixture's dict, or None when it has not been generated."""
    try:
        with open(fixture_path(name)) as f:
            return json.load(f)
    except OSError:
        return None


def logits_sha256(lg) -> list:
    return [hashlib.sha256(np.ascontiguousarray(r, "<f4").tobytes()).hexdigest() for r in np.asarray(lg)]


def compare(seq: dict, tokens, logits=None):
    """(tokens identical, index of the first logits row whose bits differ or
    None).  logits may be None (tokens only)."""
    same_tok = [int(t) for t in tokens] == seq["tokens"]
    bad = None
    if logits is not None:
        for i, h in enumerate(logits_sha256(logits)):
            if h != seq["logits_sha256"][i]:
                bad = i
                break
    return same_tok, bad
