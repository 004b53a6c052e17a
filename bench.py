#!/usr/bin/env python3
"""Benchmark of the quantised-linear hot path on one MI355X.

Headline (BASELINE.json metric "decode tok/s & GEMV HBM GB/s (int8/int4);
prefill int8 TOPS vs MFMA peak") on configs[4], the largest single-GPU
configuration: a Qwen2.5-7B-shaped int8 bundle (28 layers, d 3584, 28 / 4
heads of 128, ffn 18944, vocab 152064; seeded random int8 linears, per-token
outlier-aware int8 activations), a 2048-token seeded prompt prefilled, then
128 greedy tokens, batch 1 (Rope::generate, src/rope.rs:1147-1170, through
Bundle::mm at every linear).

One step is one such generate call (prefill + 128 decode tokens), weights
and KV cache resident in HBM.  `value` is the decode rate, 127 tokens over
(step time - the time of the same call with 1 new token, i.e. the prefill
and the first token), in tok/s; `ms_per_step` the whole call.

`roofline`: the decode's HBM-bound kernel, the fused M=1 int8 linear
(linear_m1_kernel: activation quant + GEMV + epilogue), over one layer's
four launches at the engine's shapes (q|k|v 3584->4608, o 3584->3584,
gate|up 3584->37888, down 18944->3584): algorithmic bytes (N*K + 4N + 4K + 4N
each) over the launches' summed average durations, HIP events on the
library's stream, weights rotated over at least 4 sets of more than 640 MB
in all for each shape (beyond the 256 MB MALL).
`roofline_prefill`: the prefill's dominant kernel, the int8 MFMA GEMM the
engine's prefill runs (its exact int32 sums), at the gate|up shape (M=2048,
K=3584, N=37888) on pre-quantised rows, 2*M*N*K ops over its average
duration, against the dense int8 peak; beside it the whole exact linear
(quant + GEMM + exact epilogue) and the union-correction GEMM.
`cpu_baseline`: the oracle's restatement of Rope::generate (the reference's
scalar int8 path, the `_scalar_i8_bench` build, -O3 -march=x86-64) on the
same bundle, decode tok/s over a bounded sample; `cpu_baseline_avx512` the
same with the AVX-512BW dot the production x86 build dispatches to.
`parity`: the timed generate's tokens (and, in an untimed call, every
logits row's SHA-256) against the oracle's fixture (tests/golden).

`detail` holds the other configs and legs: configs[1]'s isolated int8
sweep (M = 1, 4, 16, 128, 2048), int4 / q4a GEMVs at Gemma-2 shapes, the
unembed row dot, configs[3]'s MoE layer, configs[0] GPT-2 decode and
configs[2] Gemma-2-2b int4 decode, each with its oracle check.
"""
import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))

METRIC = "decode tok/s & GEMV HBM GB/s (int8/int4); prefill int8 TOPS vs MFMA peak"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
# configs[4]
C4 = dict(L=28, H=28, KV=4, hd=128, d=3584, ffn=18944, vocab=152064, prompt=2048, n_new=128)
C4_SHAPES = [(3584, 4608), (3584, 3584), (3584, 2 * 18944), (18944, 3584)]  # (K, N) of one layer's linears
PMC_COPY_BYTES = 256 << 20


def int8_linear_bytes(m, k, n):
    return n * k + 4 * n + 4 * m * k + 4 * m * n


def gemv_kernel_bytes(m, k, n):
    # weights + scale + a8 + sa + 32 outliers (idx, val) per row + f32 out
    return n * k + 4 * n + m * k + m * (4 + 32 * 8) + 4 * m * n


def int4_bytes(m, k, n, g=32):
    return n * k // 2 + 2 * n * ((k + g - 1) // g) + 4 * m * k + 4 * m * n


def q4a_bytes(m, k, n, g=32):
    # packed nibbles + the f16 scale and min of each group + f32 in / out
    return n * ((k + 1) // 2) + 4 * n * ((k + g - 1) // g) + 4 * m * k + 4 * m * n


def moe_bytes(T, E, d, mi, active):
    # the MoE layer's bytes: active experts' int8 gate/up/down + f32 scales, x, out, logits
    return active * (3 * d * mi + 4 * (mi + mi + d)) + 4 * T * d + 4 * T * d + 4 * T * E


def moe_i4_bytes(T, E, d, mi, active, g=32):
    # int4 experts: packed nibbles + f16 group scales of gate / up / down, x, out, logits
    return active * (3 * d * mi // 2 + 2 * 3 * d * mi // g) + 4 * T * d + 4 * T * d + 4 * T * E


ROT_BYTES = 640 << 20  # weight bytes a timed shape rotates over (beyond the 256 MB MALL)


def n_rot(bytes_each):
    """Weight sets a timed shape rotates over: at least 4, together more
    than ROT_BYTES, so no repeat can be served from the MALL."""
    return max(4, -(-ROT_BYTES // bytes_each))


def host_threads():
    """Threads for the CPU baseline: the cores this process may run on (what
    rayon's default pool uses), at most 16 (the GPU box's CPU share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16)), n


def shm_dir():
    return "/dev/shm" if os.path.isdir("/dev/shm") else None


def traffic_from(summary):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE scaled by a copy of known size); None if absent."""
    try:
        with open(os.path.join(ROOT, "profiles", summary)) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3, help="timed configs[4] generate calls")
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-detail", action="store_true")
    ap.add_argument("--no-graphs", action="store_true",
                    help="decode steps launched eagerly rather than from a captured graph (the same kernels; "
                         "rocprofv3's kernel trace does not survive graph capture on this image)")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="only the counter-collection workload (run under rocprofv3 --pmc)")
    ap.add_argument("--vendor", action="store_true",
                    help="also time hipBLASLt's int8 GEMM (torch._int_mm) at the prefill GEMM shapes, a speed "
                         "reference for roofline_prefill (imports torch: not in the default run)")
    ap.add_argument("--only-gemma2", action="store_true",
                    help="only configs[2]'s Gemma-2 decode (batch 1 and batch 16) and print its detail entry "
                         "(for profiling those runs; combine with --no-graphs under rocprofv3)")
    ap.add_argument("--pmc-what", default="layer", choices=["layer", "int4", "m128", "moe", "moe4"],
                    help="counter workload: the configs[4] layer's four decode linears (default), the int4 "
                         "M=1 GEMV at the Gemma-2 shapes, the int8 linear at M=128, or configs[3]'s MoE "
                         "layer at T=1 and T=512")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(collectives are out of scope); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import fieldrun_amd as fa
    from fieldrun_amd import convert, hip, synth

    ctx = fa.Context(0)
    stream = fa.lib.frq_get_stream(ctx.h)
    log = lambda *a: print("[bench]", *a, file=sys.stderr, flush=True)

    def time_loop(fn, iters, warm=3):
        for i in range(warm):
            fn(i)
        hip.synchronize()
        e0, e1 = hip.Event(), hip.Event()
        e0.record(stream)
        for i in range(iters):
            fn(i)
        e1.record(stream)
        e1.synchronize()
        ctx.sync()
        return e0.elapsed_ms(e1) / iters

    def decode_linears():
        """The configs[4] layer's four linear shapes at M=1 (the engine's
        kernel), each rotated over n_rot sets: per-launch us and algorithmic
        bytes."""
        rows = []
        for si, (k, n) in enumerate(C4_SHAPES):
            reps = []
            nr = n_rot(n * k)
            for r in range(nr):
                wt, scale = synth.int8_weight(n, k, synth.seed(4, r) + si)
                reps.append(ctx.upload_i8(wt, scale))
                del wt
            a = synth.activations(1, k, synth.seed(4) + si)
            da, do = hip.DeviceArray.from_numpy(a), hip.DeviceArray((1, n), np.float32)
            us = time_loop(lambda i: reps[i % nr].mm_dev(da.ptr, 1, do.ptr), max(60, 2 * nr)) * 1e3
            rows.append({"K": k, "N": n, "us": round(us, 2), "bytes": int8_linear_bytes(1, k, n),
                         "GBps": round(int8_linear_bytes(1, k, n) / (us * 1e-6) / 1e9, 1),
                         "rotation": {"sets": nr, "bytes": nr * n * k}})
            for w in reps:
                w.free()
        return rows

    if args.pmc_pass:
        # counter workload: 3 device copies of known size (the calibration),
        # then 9 launches of each of the layer's four decode linears
        src, dst = hip.DeviceArray((PMC_COPY_BYTES,), np.uint8), hip.DeviceArray((PMC_COPY_BYTES,), np.uint8)
        src.zero()
        hip.synchronize()
        for _ in range(3):
            hip.copy_d2d(dst.ptr, src.ptr, PMC_COPY_BYTES)
        hip.synchronize()
        log(f"pmc: 3 copies of {PMC_COPY_BYTES} bytes")
        if args.pmc_what == "int4":
            for (k, n) in [(2304, 9216), (9216, 2304)]:
                reps = []
                for r in range(3):
                    packed, s16, g = synth.int4_weight(n, k, synth.seed(2, r))
                    reps.append(ctx.upload_i4(packed, s16, k, g))
                a = hip.DeviceArray.from_numpy(synth.activations(1, k, synth.seed(2, 9), outlier_scale=1.0))
                o = hip.DeviceArray((1, n), np.float32)
                for i in range(9):
                    reps[i % 3].mm_dev(a.ptr, 1, o.ptr)
                ctx.sync()
                log(f"pmc: 9 int4 M=1 launches at K={k} N={n}, {int4_bytes(1, k, n)} algorithmic bytes each")
                for w in reps:
                    w.free()
            return
        if args.pmc_what in ("moe", "moe4"):
            # the Qwen3-MoE routed layer at T=1 and T=512, 9 calls each (moe4: int4 experts, g 32)
            E, d, mi, topk = 128, 2048, 768, 8
            if args.pmc_what == "moe":
                gate, gs, up, us_, down, ds = synth.moe_layer(E, d, mi, synth.seed(3))
                bank = ctx.upload_moe_i8(gate, gs, up, us_, down, ds)
            else:
                gate, up, down = synth.moe_layer_ex(E, d, mi, synth.seed(3), "int4")
                pick = lambda lst, key: [m[key] for m in lst]  # noqa: E731
                bank = ctx.upload_moe("i4", d, mi, pick(gate, "raw"), pick(down, "raw"), pick(up, "raw"),
                                      pick(gate, "scale"), pick(up, "scale"), pick(down, "scale"), g=32)
                del gate, up, down
            for T in (1, 512):
                rng = np.random.default_rng(synth.seed(3, T))
                x = hip.DeviceArray.from_numpy(rng.standard_normal((T, d), dtype=np.float32))
                lg = hip.DeviceArray.from_numpy(rng.standard_normal((T, E), dtype=np.float32))
                o = hip.DeviceArray((T, d), np.float32)
                for i in range(9):
                    bank.forward_dev(x.ptr, T, lg.ptr, topk, True, None, o.ptr)
                ctx.sync()
                log(f"pmc: 9 MoE layer calls at T={T} (E={E}, d={d}, mi={mi}, k={topk})")
            bank.free()
            return
        if args.pmc_what == "m128":
            for (k, n) in [(896, 151936), (4096, 14336)]:
                reps = [ctx.upload_i8(*synth.int8_weight(n, k, synth.seed(1, r) + k)) for r in range(3)]
                a = hip.DeviceArray.from_numpy(synth.activations(128, k, synth.seed(1) + k))
                o = hip.DeviceArray((128, n), np.float32)
                for i in range(9):
                    reps[i % 3].mm_dev(a.ptr, 128, o.ptr)
                ctx.sync()
                log(f"pmc: 9 int8 M=128 linears at K={k} N={n}, {int8_linear_bytes(128, k, n)} algorithmic bytes each")
                for w in reps:
                    w.free()
            return
        for si, (k, n) in enumerate(C4_SHAPES):
            reps = [ctx.upload_i8(*synth.int8_weight(n, k, synth.seed(4, r) + si)) for r in range(3)]
            a = hip.DeviceArray.from_numpy(synth.activations(1, k, synth.seed(4) + si))
            o = hip.DeviceArray((1, n), np.float32)
            for i in range(9):
                reps[i % 3].mm_dev(a.ptr, 1, o.ptr)
            ctx.sync()
            log(f"pmc: 9 launches at K={k} N={n}, {int8_linear_bytes(1, k, n)} algorithmic bytes each")
            for w in reps:
                w.free()
        return

    threads, visible = host_threads()
    detail = {}
    import config_fixtures as cfx

    if args.only_gemma2:
        print(json.dumps({"gemma2_decode": gemma2_detail(args, ctx, fa, cfx, log)}))
        return

    # ======================= headline: configs[4] =======================
    with tempfile.TemporaryDirectory(dir=shm_dir()) as tmp:
        stem = os.path.join(tmp, "qwen25_7b")
        t0 = time.time()
        cfx.WORKLOADS["config4"]["write"](stem)
        prompt = cfx.WORKLOADS["config4"]["prompts"]()[0]
        log(f"configs[4] bundle written in {time.time() - t0:.1f}s")
        b = fa.Bundle(stem, ctx)
        g = fa.Rope(b)
        g.set_graphs(not args.no_graphs)
        n_new = C4["n_new"]
        # untimed: the parity call (tokens and every logits row against the fixture)
        toks, lg = g.generate(prompt, n_new, with_logits=True)
        fx = cfx.load_fixture("config4")
        parity = {"fixture": "tests/golden/config4.json", "present": fx is not None}
        if fx is not None:
            same_tok, bad = cfx.compare(fx["sequences"][0], toks, lg)
            parity.update(tokens_identical=same_tok, logits_bit_identical=bad is None,
                          first_logits_mismatch=bad)
        del lg
        for _ in range(max(0, args.warmup - 1)):
            g.generate(prompt, n_new)
        # prefill + the first token (median of 3)
        tp = []
        for _ in range(3):
            t0 = time.perf_counter()
            g.generate(prompt, 1)
            tp.append(time.perf_counter() - t0)
        t_prefill = float(np.median(tp))
        # the timed steps
        steps = []
        timed_toks = None
        for _ in range(args.steps):
            t0 = time.perf_counter()
            timed_toks = g.generate(prompt, n_new)
            steps.append(time.perf_counter() - t0)
        t_step = float(np.median(steps))
        if fx is not None:
            parity["timed_tokens_identical"] = [int(t) for t in timed_toks] == fx["sequences"][0]["tokens"]
        dec_s = (t_step - t_prefill) / (n_new - 1)
        value = 1.0 / dec_s
        lin_params = C4["L"] * sum(k * n for k, n in C4_SHAPES)
        prefill_tops = 2.0 * lin_params * C4["prompt"] / t_prefill / 1e12
        log(f"configs[4]: step {t_step * 1e3:.1f} ms, prefill+first {t_prefill * 1e3:.1f} ms, "
            f"decode {dec_s * 1e3:.3f} ms/token ({value:.1f} tok/s), parity {parity}")
        g.free()
        b.close()

        # ---- CPU baseline: the oracle's Rope::generate on the same bundle ----
        cpu = cpu512 = None
        if not args.no_cpu:
            import oracle  # the CPU baseline leg: the reference's decode restated in C

            m_, arrs = oracle.read_bundle(stem)
            ref = oracle.Rope(m_, arrs, nthreads=threads)
            sp = prompt[:8]

            def oracle_rate():
                t0 = time.perf_counter()
                r1 = ref.generate(sp, 1)
                t1 = time.perf_counter()
                r5 = ref.generate(sp, 5)
                t5 = time.perf_counter()
                return 4.0 / ((t5 - t1) - (t1 - t0)), r1, r5

            rate, _, r5 = oracle_rate()
            cpu = {"value": round(rate, 3), "unit": "tok/s", "cores": threads, "kind": "port",
                   "sample": "configs[4] bundle, 8-token prompt: decode rate 4 / (t(5 new) - t(1 new)) of the "
                             "oracle's Rope::generate (scalar i8dot, -O3 -march=x86-64, rayon-style splits), "
                             f"{threads} threads ({visible} visible to the process)"}
            if oracle.set_i8dot("avx512bw"):
                try:
                    rate2, _, r5b = oracle_rate()
                finally:
                    oracle.set_i8dot("scalar")
                cpu512 = {"value": round(rate2, 3), "unit": "tok/s", "cores": threads, "kind": "port",
                          "sample": "as cpu_baseline with i8dot_avx512bw (src/bundle.rs:1107-1126), the dot the "
                                    "production x86 build dispatches to",
                          "tokens_identical_to_scalar": bool(np.array_equal(r5, r5b))}
            else:
                cpu512 = {"value": None, "note": "the host lacks AVX-512BW"}
            log(f"CPU baseline {cpu}; avx512 {cpu512}")
            del ref, arrs

    # decode GEMV roofline at the engine's shapes
    lin = decode_linears()
    lay_bytes = sum(r["bytes"] for r in lin)
    lay_us = sum(r["us"] for r in lin)
    gbs = lay_bytes / (lay_us * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from("linear_m1_config4_pmc.md"),
                "traffic_per": "one launch of each of the layer's four shapes (FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
                "kernel": "linear_m1_kernel (fused quant + GEMV, M=1), one configs[4] layer's four launches",
                "bytes_per_layer": lay_bytes, "us_per_layer": round(lay_us, 2), "launches": lin}
    log(f"decode linears: {lin}")

    # prefill GEMM roofline: M=2048 at the gate|up shape, pre-quantised rows,
    # the GEMM the engine's prefill runs (int32 sums for the exact epilogue)
    k, n, M = 3584, 2 * 18944, C4["prompt"]
    nr = max(2, n_rot(n * k))  # weight sets rotated (each 136 MB)
    ws_ = []
    for r in range(nr):
        wt, scale = synth.int8_weight(n, k, synth.seed(4, 9) + r)
        ws_.append(ctx.upload_i8(wt, scale))
        del wt
    a = synth.activations(M, k, synth.seed(4, 10))
    da, do = hip.DeviceArray.from_numpy(a), hip.DeviceArray((M, n), np.float32)
    dacc = hip.DeviceArray((M, n), np.int32)
    kp = fa.quant_pitch(k)
    a8, sa = hip.DeviceArray((M, kp), np.int8), hip.DeviceArray((M,), np.float32)
    oi, ov = hip.DeviceArray((M, 32), np.uint32), hip.DeviceArray((M, 32), np.float32)
    ctx.quant_dev(da.ptr, M, k, a8.ptr, sa.ptr, oi.ptr, ov.ptr)
    gus = float(np.median([time_loop(lambda i: ws_[i % nr].mm_acc_dev(a8.ptr, M, dacc.ptr), 2 * nr,
                                     warm=2 if r == 0 else 0) for r in range(3)])) * 1e3
    fus = float(np.median([time_loop(lambda i: ws_[i % nr].mm_exact_dev(da.ptr, M, do.ptr), 2 * nr, warm=1)
                           for _ in range(3)])) * 1e3
    uus = float(np.median([time_loop(lambda i: ws_[i % nr].mm_q_dev(a8.ptr, sa.ptr, oi.ptr, ov.ptr, M, do.ptr),
                                     2 * nr, warm=1) for _ in range(3)])) * 1e3
    ops = 2.0 * M * n * k
    tops = ops / (gus * 1e-6) / 1e12
    roofline_prefill = {"bound": "mfma", "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
                        "frac": round(tops / INT8_PEAK_TOPS, 4), "traffic": None,
                        "kernel": "gemm_i8_kernel, the int32-sum MFMA GEMM the engine's prefill runs "
                                  f"(frq_mm_i8_acc_dev: blockify + GEMM on pre-quantised rows), M={M} K={k} N={n}",
                        "us_per_launch": round(gus, 1),
                        "rotation": {"sets": nr, "bytes": nr * n * k},
                        "exact_linear_us": round(fus, 1),
                        "exact_linear_TOPS": round(ops / (fus * 1e-6) / 1e12, 1),
                        "exact_linear_note": "frq_mm_exact_dev: quant, this GEMM, the exact sequential outlier "
                                             "epilogue (the engine's prefill linear, bit-exact)",
                        "union_gemm_us": round(uus, 1),
                        "union_gemm_note": "frq_mm_i8_q_dev at M > 16: the GEMM with the outlier correction as "
                                           "f16 hi/lo MFMAs (within 1e-6 of the exact sum)"}
    for w in ws_:
        w.free()
    del a, da, do, dacc, a8, sa, oi, ov
    log(f"prefill GEMM: {roofline_prefill}")
    if args.vendor:  # in a child process: torch's own HIP runtime does not start beside libfrq's
        import subprocess
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--vendor-child"], capture_output=True,
                           text=True, timeout=600)
        lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
        roofline_prefill["vendor"] = json.loads(lines[-1]) if r.returncode == 0 and lines else {
            "error": (r.stderr or "")[-400:]}
        log(f"vendor int8 GEMM: {roofline_prefill['vendor']}")

    if not args.no_detail:
        detail.update(run_detail(args, ctx, fa, hip, synth, convert, time_loop, log, threads, cfx))

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(t_step * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded random-init weights of the config's shapes, written in the reference's "
                "bundle format; seeded prompt)",
        "config": {"workload": "configs[4]: Qwen2.5-7B-shaped int8 (28 layers, d 3584, 28/4 heads of 128, "
                               "ffn 18944, vocab 152064), 2048-token prompt prefill then 128 greedy tokens, "
                               "batch 1; value = decode tok/s",
                   "prompt_tokens": C4["prompt"], "new_tokens": n_new, "batch": 1},
        "prefill": {"ms_prefill_plus_first": round(t_prefill * 1e3, 2),
                    "tok_s": round(C4["prompt"] / t_prefill, 1),
                    "linear_TOPS": round(prefill_tops, 1),
                    "linear_frac_int8_peak": round(prefill_tops / INT8_PEAK_TOPS, 4)},
        "decode_ms_per_token": round(dec_s * 1e3, 4),
        "parity": parity,
        "roofline": roofline,
        "roofline_prefill": roofline_prefill,
        "cpu_baseline": cpu,
        "cpu_baseline_avx512": cpu512,
        "detail": detail,
    }
    print(json.dumps(line))


def vendor_int8_gemm(log=lambda *a: None):
    """hipBLASLt's int8 GEMM through torch._int_mm (A (M,K) i8 row-major, B
    (K,N) the transpose of an (N,K) row-major i8 weight, i32 out) at the
    configs[4] prefill shapes, weights rotated over >= 4 sets: a speed
    reference for the MFMA GEMM, not a parity path."""
    import torch
    res = {}
    for (m, k, n) in [(2048, 3584, 37888), (2048, 3584, 4608), (2048, 18944, 3584), (2048, 4096, 14336)]:
        a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device="cuda:0")
        nr = n_rot(n * k)
        bs = [torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda:0").t() for _ in range(nr)]
        for i in range(3):
            torch._int_mm(a, bs[i % nr])
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        it = 4 * nr
        e0.record()
        for i in range(it):
            torch._int_mm(a, bs[i % nr])
        e1.record()
        e1.synchronize()
        us = e0.elapsed_time(e1) / it * 1e3
        tops = 2.0 * m * n * k / (us * 1e-6) / 1e12
        res[f"M{m}_K{k}_N{n}"] = {"us": round(us, 1), "TOPS": round(tops, 1),
                                  "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        del a, bs
        torch.cuda.empty_cache()
    log(f"vendor int8 GEMM (torch._int_mm / hipBLASLt): {res}")
    return {"library": "hipBLASLt via torch._int_mm", "shapes": res}


def run_detail(args, ctx, fa, hip, synth, convert, time_loop, log, threads, cfx):
    detail = {}
    # ---------------- the isolated int8 sweep ----------------
    shapes = list(synth.SWEEP_KN)
    weights, acts = [], []
    for si, (k, n) in enumerate(shapes):
        weights.append([ctx.upload_i8(*synth.int8_weight(n, k, synth.seed(1, r) + si)) for r in range(n_rot(n * k))])
        a = synth.activations(1, k, synth.seed(1) + si)
        acts.append((a, hip.DeviceArray.from_numpy(a)))
    detail["int8_sweep_m1"] = {"full_linear": {}, "gemv_kernel": {},
                               "rotation": {f"K{k}_N{n}": {"sets": len(weights[si]), "bytes": len(weights[si]) * n * k}
                                            for si, (k, n) in enumerate(shapes)}}
    for si, (k, n) in enumerate(shapes):
        R = len(weights[si])
        o = hip.DeviceArray((1, n), np.float32)
        us = time_loop(lambda i, si=si: weights[si][i % R].mm_dev(acts[si][1].ptr, 1, o.ptr), max(60, 2 * R)) * 1e3
        gb = int8_linear_bytes(1, k, n) / (us * 1e-6) / 1e9
        detail["int8_sweep_m1"]["full_linear"][f"K{k}_N{n}"] = {"us": round(us, 2), "GBps": round(gb, 1),
                                                                "frac": round(gb / HBM_PEAK_GBS, 3)}
        kp = fa.quant_pitch(k)
        a8, sa = hip.DeviceArray((1, kp), np.int8), hip.DeviceArray((1,), np.float32)
        oi, ov = hip.DeviceArray((1, 32), np.uint32), hip.DeviceArray((1, 32), np.float32)
        ctx.quant_dev(acts[si][1].ptr, 1, k, a8.ptr, sa.ptr, oi.ptr, ov.ptr)
        gus = time_loop(lambda i, si=si: weights[si][i % R].mm_q_dev(a8.ptr, sa.ptr, oi.ptr, ov.ptr, 1, o.ptr),
                        max(60, 2 * R)) * 1e3
        qus = time_loop(lambda i, si=si: ctx.quant_dev(acts[si][1].ptr, 1, k, a8.ptr, sa.ptr, oi.ptr, ov.ptr),
                        60) * 1e3
        detail["int8_sweep_m1"]["gemv_kernel"][f"K{k}_N{n}"] = {
            "us": round(gus, 2), "GBps": round(gemv_kernel_bytes(1, k, n) / (gus * 1e-6) / 1e9, 1),
            "quant_us": round(qus, 2)}
    log(f"configs[1] M=1: {detail['int8_sweep_m1']}")
    # the sweep's other M: decode batches (HBM-bound) and M=128
    detail["int8_sweep_m"] = {}
    for m in (4, 16, 128):
        row = {}
        for si, (k, n) in enumerate(shapes):
            R = len(weights[si])
            a = synth.activations(m, k, synth.seed(1, 20 + m) + si)
            da, do = hip.DeviceArray.from_numpy(a), hip.DeviceArray((m, n), np.float32)
            us = time_loop(lambda i, si=si: weights[si][i % R].mm_dev(da.ptr, m, do.ptr), max(30, 2 * R)) * 1e3
            row[f"K{k}_N{n}"] = {"full_linear_us": round(us, 2),
                                 "full_linear_GBps": round(int8_linear_bytes(m, k, n) / (us * 1e-6) / 1e9, 1)}
        detail["int8_sweep_m"][f"M{m}"] = row
        log(f"configs[1] M={m}: {row}")
    for reps in weights:
        for w in reps:
            w.free()
    # M=2048, the MFMA-bound shapes
    detail["int8_m2048_gemm"] = {}
    for (k, n) in [(4096, 14336), (14336, 4096)]:
        wt, scale = synth.int8_weight(n, k, synth.seed(1, 7))
        w = ctx.upload_i8(wt, scale)
        del wt
        a = synth.activations(2048, k, synth.seed(1, 8))
        da, do = hip.DeviceArray.from_numpy(a), hip.DeviceArray((2048, n), np.float32)

        def med3(fn):
            return float(np.median([time_loop(fn, 20, warm=10 if r == 0 else 0) for r in range(3)])) * 1e3
        us = med3(lambda i: w.mm_dev(da.ptr, 2048, do.ptr))
        kp = fa.quant_pitch(k)
        a8, sa = hip.DeviceArray((2048, kp), np.int8), hip.DeviceArray((2048,), np.float32)
        oi, ov = hip.DeviceArray((2048, 32), np.uint32), hip.DeviceArray((2048, 32), np.float32)
        ctx.quant_dev(da.ptr, 2048, k, a8.ptr, sa.ptr, oi.ptr, ov.ptr)
        gus = med3(lambda i: w.mm_q_dev(a8.ptr, sa.ptr, oi.ptr, ov.ptr, 2048, do.ptr))
        ops = 2.0 * 2048 * n * k
        detail["int8_m2048_gemm"][f"K{k}_N{n}"] = {
            "full_linear_us": round(us, 1), "full_linear_TOPS": round(ops / (us * 1e-6) / 1e12, 1),
            "gemm_us": round(gus, 1), "gemm_TOPS": round(ops / (gus * 1e-6) / 1e12, 1),
            "gemm_frac_int8_peak": round(ops / (gus * 1e-6) / 1e12 / INT8_PEAK_TOPS, 3)}
        log(f"M=2048 K={k} N={n}: {detail['int8_m2048_gemm'][f'K{k}_N{n}']}")
        w.free()
    # ---------------- int4 / q4a decode GEMV (Gemma-2-2b shapes) ----------------
    detail["int4_m1_gemv"], detail["q4a_m1_gemv"] = {}, {}
    for (k, n) in [(2304, 9216), (9216, 2304), (2304, 2048)]:
        # the rotation: distinct weight buffers over the same few seeded
        # sets (the bytes, not the values, decide what the MALL can serve)
        nr = n_rot(int4_bytes(0, k, n))
        base = [synth.int4_weight(n, k, synth.seed(2, r)) for r in range(3)]
        reps = [ctx.upload_i4(base[r % 3][0], base[r % 3][1], k, base[r % 3][2]) for r in range(nr)]
        a = synth.activations(1, k, synth.seed(2, 9), outlier_scale=1.0)
        da, do = hip.DeviceArray.from_numpy(a), hip.DeviceArray((1, n), np.float32)
        us = time_loop(lambda i: reps[i % nr].mm_dev(da.ptr, 1, do.ptr), max(60, 2 * nr)) * 1e3
        gb = int4_bytes(1, k, n) / (us * 1e-6) / 1e9
        detail["int4_m1_gemv"][f"K{k}_N{n}"] = {"us": round(us, 2), "GBps": round(gb, 1),
                                                "frac": round(gb / HBM_PEAK_GBS, 3),
                                                "rotation": {"sets": nr, "bytes": nr * int4_bytes(0, k, n)}}
        for w in reps:
            w.free()
        base = []
        for r in range(3):
            rng = np.random.default_rng(synth.seed(5, r))
            base.append(convert.put_q4a(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02), True))
        g = base[0][3]
        nr = n_rot(q4a_bytes(0, k, n, g))
        reps = [ctx.upload_q4a(base[r % 3][0], base[r % 3][1], base[r % 3][2], k, g) for r in range(nr)]
        us = time_loop(lambda i: reps[i % nr].mm_dev(da.ptr, 1, do.ptr), max(60, 2 * nr)) * 1e3
        gb = q4a_bytes(1, k, n, g) / (us * 1e-6) / 1e9
        detail["q4a_m1_gemv"][f"K{k}_N{n}"] = {"us": round(us, 2), "GBps": round(gb, 1),
                                               "frac": round(gb / HBM_PEAK_GBS, 3),
                                               "rotation": {"sets": nr, "bytes": nr * q4a_bytes(0, k, n, g)}}
        for w in reps:
            w.free()
    log(f"int4 {detail['int4_m1_gemv']}; q4a {detail['q4a_m1_gemv']}")
    # ---------------- unembed row dot (Bundle::rowdot_f32) ----------------
    detail["unembed_rowdot"] = {}
    for name, rows, d, kind in [("gemma2_f16", 256000, 2304, "f16"), ("gemma2_rowi8", 256000, 2304, "rowi8"),
                                ("qwen25_f16", 152064, 3584, "f16"), ("gpt2_f16", 50257, 768, "f16")]:
        rng = np.random.default_rng(synth.seed(2, 30))
        if kind == "f16":
            data = (rng.standard_normal((rows, d), dtype=np.float32) * np.float32(0.02)).astype(np.float16)
            sc, es = None, 2
        else:
            data = rng.integers(-127, 128, (rows, d), dtype=np.int8)
            sc, es = rng.uniform(1e-4, 3e-4, rows).astype(np.float16).astype(np.float32), 1
        t = ctx.upload_rows(kind, data, sc)
        del data
        x = hip.DeviceArray.from_numpy(rng.standard_normal(d).astype(np.float32))
        o = hip.DeviceArray((rows,), np.float32)
        us = time_loop(lambda i: t.rowdot_f32_dev(x.ptr, o.ptr), 30) * 1e3
        nbytes = rows * d * es + (4 * rows if kind == "rowi8" else 0) + 4 * d + 4 * rows
        gb = nbytes / (us * 1e-6) / 1e9
        detail["unembed_rowdot"][name] = {"us": round(us, 2), "GBps": round(gb, 1),
                                          "frac": round(gb / HBM_PEAK_GBS, 3)}
        t.free()
    log(f"rowdot {detail['unembed_rowdot']}")
    # ---------------- the Qwen3-MoE routed layer ----------------
    detail["moe_qwen3_layer"] = {}
    E, d, mi, topk = 128, 2048, 768, 8
    gate, gs, up, us_, down, ds = synth.moe_layer(E, d, mi, synth.seed(3))
    bank = ctx.upload_moe_i8(gate, gs, up, us_, down, ds)
    for T in (1, 512):
        rng = np.random.default_rng(synth.seed(3, T))
        xh = rng.standard_normal((T, d), dtype=np.float32)
        lgh = rng.standard_normal((T, E), dtype=np.float32)
        x, lg = hip.DeviceArray.from_numpy(xh), hip.DeviceArray.from_numpy(lgh)
        o = hip.DeviceArray((T, d), np.float32)
        us = time_loop(lambda i: bank.forward_dev(x.ptr, T, lg.ptr, topk, True, None, o.ptr), 10) * 1e3
        sel, _ = ctx.moe_route(lgh, topk, True)
        active = len(np.unique(sel))
        nb = moe_bytes(T, E, d, mi, active)
        gb = nb / (us * 1e-6) / 1e9
        detail["moe_qwen3_layer"][f"T{T}"] = {"us": round(us, 1), "active_experts": active, "bytes": nb,
                                              "GBps": round(gb, 1), "frac_hbm": round(gb / HBM_PEAK_GBS, 3),
                                              "TFLOPs": round(2 * T * topk * 3 * d * mi / (us * 1e-6) / 1e12, 2)}
    bank.free()
    log(f"moe {detail['moe_qwen3_layer']}")
    # the same layer with int4 experts (convert --dtype int4: put_i4, g = 32)
    detail["moe_qwen3_layer_int4"] = {}
    gate, up, down = synth.moe_layer_ex(E, d, mi, synth.seed(3), "int4")
    pick = lambda lst, key: [m[key] for m in lst]  # noqa: E731
    bank = ctx.upload_moe("i4", d, mi, pick(gate, "raw"), pick(down, "raw"), pick(up, "raw"), pick(gate, "scale"),
                          pick(up, "scale"), pick(down, "scale"), g=32)
    del gate, up, down
    for T in (1, 512):
        rng = np.random.default_rng(synth.seed(3, T))
        xh = rng.standard_normal((T, d), dtype=np.float32)
        lgh = rng.standard_normal((T, E), dtype=np.float32)
        x, lg = hip.DeviceArray.from_numpy(xh), hip.DeviceArray.from_numpy(lgh)
        o = hip.DeviceArray((T, d), np.float32)
        us = time_loop(lambda i: bank.forward_dev(x.ptr, T, lg.ptr, topk, True, None, o.ptr), 10) * 1e3
        sel, _ = ctx.moe_route(lgh, topk, True)
        active = len(np.unique(sel))
        nb = moe_i4_bytes(T, E, d, mi, active)
        gb = nb / (us * 1e-6) / 1e9
        detail["moe_qwen3_layer_int4"][f"T{T}"] = {"us": round(us, 1), "active_experts": active, "bytes": nb,
                                                   "GBps": round(gb, 1), "frac_hbm": round(gb / HBM_PEAK_GBS, 3),
                                                   "TFLOPs": round(2 * T * topk * 3 * d * mi / (us * 1e-6) / 1e12, 2)}
    bank.free()
    log(f"moe int4 {detail['moe_qwen3_layer_int4']}")
    # ---------------- GPT-2 small greedy decode ----------------
    detail["gpt2_decode"] = {}
    with tempfile.TemporaryDirectory(dir=shm_dir()) as tmp:
        stem = os.path.join(tmp, "gpt2")
        synth.write_gpt2_bundle(stem, 1234)
        b = fa.Bundle(stem, ctx)
        prompt = synth.gpt2_prompt(32, 50257, 7)
        for kv8 in (False, True):
            g = fa.Gpt2(b, kv8)
            g.set_graphs(not args.no_graphs)
            g.generate(prompt, 128)
            runs = {}
            for n_new in (1, 128):
                ts = []
                for _ in range(3):
                    t0 = time.perf_counter()
                    g.generate(prompt, n_new)
                    ts.append(time.perf_counter() - t0)
                runs[n_new] = sorted(ts)[1]
            dec_ms = (runs[128] - runs[1]) / 127 * 1e3
            detail["gpt2_decode"]["kv_int8" if kv8 else "kv_f32"] = {
                "tok_s": round(128 / runs[128], 1), "decode_ms_per_token": round(dec_ms, 4),
                "decode_tok_s": round(1e3 / dec_ms, 1), "prefill_plus_first_ms": round(runs[1] * 1e3, 3)}
            g.free()
        if not args.no_cpu:
            import oracle  # configs[0]'s CPU rate: the reference's GPT-2 decode restated in C

            m_, arrs = oracle.read_bundle(stem)
            ref = oracle.Gpt2(m_, arrs, nthreads=threads)
            g = fa.Gpt2(b)
            t0 = time.perf_counter()
            rt = ref.generate(prompt, 16)
            el = time.perf_counter() - t0
            detail["gpt2_decode"]["cpu_oracle"] = {"tok_s": round(16 / el, 2), "threads": threads,
                                                   "sample": "16 tokens after the 32-token prompt",
                                                   "tokens_identical": bool(np.array_equal(rt, g.generate(prompt, 16)))}
            g.free()
        b.close()
    log(f"gpt2 {detail['gpt2_decode']}")
    detail["gemma2_decode"] = gemma2_detail(args, ctx, fa, cfx, log)
    return detail


def gemma2_detail(args, ctx, fa, cfx, log):
    """Gemma-2-2b int4 greedy decode, batch 1 and batch 16."""
    out = {}
    with tempfile.TemporaryDirectory(dir=shm_dir()) as tmp:
        stem = os.path.join(tmp, "gemma2")
        cfx.WORKLOADS["config2"]["write"](stem)
        b = fa.Bundle(stem, ctx)
        g = fa.Gemma(b)
        g.set_graphs(not args.no_graphs)
        prompt = cfx.WORKLOADS["config2"]["prompts"]()[0]
        toks = g.generate(prompt, 256)
        fx = cfx.load_fixture("config2")
        runs = {}
        for n_new in (1, 256):
            t0 = time.perf_counter()
            g.generate(prompt, n_new)
            runs[n_new] = time.perf_counter() - t0
        dec_ms = (runs[256] - runs[1]) / 255 * 1e3
        out["int4_kv_f32_batch1"] = {
            "tok_s": round(256 / runs[256], 1), "decode_ms_per_token": round(dec_ms, 3),
            "decode_tok_s": round(1e3 / dec_ms, 1), "prefill_plus_first_ms": round(runs[1] * 1e3, 1),
            "tokens_identical_to_fixture": None if fx is None else cfx.compare(fx["sequences"][0], toks)[0]}
        # batch 16: sixteen 64-token prompts decoded together (every sequence
        # its own generate); decode tok/s over all sequences, and the step's
        # weight stream (int4 linears + f16 scales + the f16 unembed) per step
        pb = np.stack(cfx.WORKLOADS["config2_b16"]["prompts"]())
        tb = g.generate_batch(pb, 256)
        fxb = cfx.load_fixture("config2_b16")
        runs = {}
        for n_new in (1, 256):
            t0 = time.perf_counter()
            g.generate_batch(pb, n_new)
            runs[n_new] = time.perf_counter() - t0
        step_s = (runs[256] - runs[1]) / 255
        L_, d_, ffn_, V_ = 26, 2304, 9216, 256000
        lin = L_ * (d_ * (2048 + 1024 + 1024) + 2048 * d_ + d_ * 2 * ffn_ + ffn_ * d_)
        step_bytes = lin // 2 + 2 * (lin // 32) + V_ * d_ * 2
        out["int4_kv_f32_batch16"] = {
            "decode_tok_s": round(16 / step_s, 1), "step_ms": round(step_s * 1e3, 3),
            "prefill_plus_first_ms": round(runs[1] * 1e3, 1),
            "weight_GBps": round(step_bytes / step_s / 1e9, 1),
            "weight_frac_hbm": round(step_bytes / step_s / 1e9 / HBM_PEAK_GBS, 3),
            # the exact per-sequence orders make the batch step VALU-bound:
            # one f32 FMA (linears) or mul + add (the f16 head) per weight
            # element and sequence
            "fma_per_step": 16 * (lin + V_ * d_),
            "fma_T_per_s": round(16 * (lin + V_ * d_) / step_s / 1e12, 2),
            "tokens_identical_to_fixture": None if fxb is None else all(
                cfx.compare(fxb["sequences"][i], tb[i])[0] for i in range(len(pb)))}
        log(f"gemma2 {out}")
        g.free()
        b.close()
    return out


if __name__ == "__main__":
    if "--vendor-child" in sys.argv:
        print(json.dumps(vendor_int8_gemm()))
    else:
        main()
