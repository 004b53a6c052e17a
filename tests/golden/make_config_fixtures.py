#!/usr/bin/env python3
"""Writes the end-to-end golden fixtures of the BASELINE configs by running
the CPU oracle (oracle/frq_oracle.c, the C restatement of the reference's
Gemma::generate / Rope::generate, src/gemma.rs:403-431 and
src/rope.rs:1147-1170) on the same synthetic bundles and prompts that the
GPU tests and bench.py build (fieldrun_amd/synth.py, seeded).

Each fixture holds the greedy tokens and, per generated token, the SHA-256
of the f32 logits row it was chosen from (little-endian bytes), so the GPU
test can compare the device's logits bit for bit without shipping them.

  python tests/golden/make_config_fixtures.py config4 config2 config2_b16

config4     configs[4]: Qwen2.5-7B-shaped int8 bundle (28 layers), a 2048-token
            prompt, 128 greedy tokens
config2     configs[2]: Gemma-2-2b-shaped int4 bundle, a 64-token prompt,
            256 greedy tokens (batch 1)
config2_b16 configs[2] at batch 16: sixteen 64-token prompts, 256 tokens
            each; the reference has no batched generate, so each sequence is
            its own batch-1 Gemma::generate

Runs in minutes (config4's 2048-token prefill through the oracle's scalar
int8 path is the longest); the bundles go to a temporary directory in
/dev/shm when it exists.
"""
import json
import os
import sys
import tempfile
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

# the workloads, shared with the tests and bench.py (config_fixtures.WORKLOADS)
sys.path.insert(0, HERE)
from config_fixtures import WORKLOADS, fixture_path, logits_sha256  # noqa: E402


def run(name, nthreads):
    wl = WORKLOADS[name]
    tmpdir = "/dev/shm" if os.path.isdir("/dev/shm") else None
    with tempfile.TemporaryDirectory(dir=tmpdir) as tmp:
        stem = os.path.join(tmp, name)
        t0 = time.time()
        wl["write"](stem)
        m, arrs = oracle.read_bundle(stem)
        ref = oracle.Gemma(m, arrs, nthreads=nthreads)
        seqs = []
        for prompt in wl["prompts"]():
            t1 = time.time()
            toks, lg = ref.generate(prompt, wl["n_new"], with_logits=True)
            seqs.append({"tokens": [int(t) for t in toks], "logits_sha256": logits_sha256(lg),
                         "logits_first": [float(v) for v in lg[0, :4]]})
            print(f"{name}: sequence {len(seqs)} in {time.time() - t1:.1f}s", flush=True)
            del lg
        fx = {"workload": name, "what": wl["what"], "n_new": wl["n_new"], "kv_int8": False,
              "oracle_threads": nthreads, "seconds": round(time.time() - t0, 1), "sequences": seqs}
    with open(fixture_path(name), "w") as f:
        json.dump(fx, f, indent=1)
    print(f"wrote {fixture_path(name)}", flush=True)


if __name__ == "__main__":
    names = sys.argv[1:] or list(WORKLOADS)
    for n in names:
        run(n, os.cpu_count() or 8)
