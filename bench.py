#!/usr/bin/env python3
"""Benchmark of the quantised-linear hot path on one MI355X.

Headline (BASELINE.json metric "decode tok/s & GEMV HBM GB/s (int8/int4);
prefill int8 TOPS vs MFMA peak", workload configs[1]): one step is one pass
of the full int8 linear (outlier-aware activation quant + i8 dot + epilogue,
Bundle::mm's I8 arm) at M=1 over the five (K,N) shapes of the isolated
int8 sweep, inputs already resident in HBM.  `value` is the step's
algorithmic bytes (N*K + 4N + 4K + 4N per shape) over its wall time on the
GPU stream, in GB/s.  Weights are rotated over 3 replica sets (786 MB, over
the 256 MB MALL) so repeats are served from HBM.

At M=1 the full linear is one kernel (linear_m1_kernel: the activation quant
fused into the GEMV); `roofline` is that kernel at the step's dominant shape
(K=896, N=151936, 136 MB of weights), its algorithmic bytes (weights, scales,
f32 activation row, f32 outputs) over its average launch time on the
library's stream.  Also reported (in "detail"): the GEMV kernel alone on
pre-quantised input, the M=2048 MFMA-bound shapes in TOPS, the int4 decode
GEMV and the affine-int4 (q4a) GEMV on Gemma-2 shapes, the unembed row dot, the config-4 MoE layer, and
config 0 end to end: GPT-2 small greedy decode (tok/s, f32 and int8 KV
caches) with the oracle's CPU rate and token check beside it, and config 2:
Gemma-2-2b int4 greedy decode (256 tokens after a 64-token prompt), and
config 4: Qwen2.5-7B int8, a 2048-token prefill then 128 greedy tokens.  The CPU
baseline is the
oracle's restatement of the reference's scalar int8 path (the
`_scalar_i8_bench` build) on the host's cores, on a bounded sample.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

METRIC = "decode tok/s & GEMV HBM GB/s (int8/int4); prefill int8 TOPS vs MFMA peak"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0


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


DOM_SHAPE = (896, 151936)  # the headline's dominant launch (136 MB of weights)
DOM_KERNEL = "linear_m1_kernel<8,8,true,1,256>"
PMC_COPY_BYTES = 256 << 20
PMC_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                           "linear_m1_K896_N151936_pmc.md")


def measured_traffic():
    """HBM bytes per launch of the dominant kernel, from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, each scaled by the
    same counter's reading on a copy of known size); None if absent."""
    try:
        with open(PMC_SUMMARY) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def pmc_pass(fa, hip, synth, ctx, log):
    """Counter-collection workload, run under `rocprofv3 --pmc`: 3 device
    copies of PMC_COPY_BYTES (the calibration kernel), then 9 launches of
    the dominant kernel, the fused M=1 linear (3 weight replicas)."""
    src = hip.DeviceArray((PMC_COPY_BYTES,), np.uint8)
    dst = hip.DeviceArray((PMC_COPY_BYTES,), np.uint8)
    src.zero()
    hip.synchronize()
    for _ in range(3):
        hip.copy_d2d(dst.ptr, src.ptr, PMC_COPY_BYTES)
    hip.synchronize()
    log(f"pmc: 3 copies of {PMC_COPY_BYTES} bytes")
    k, n = DOM_SHAPE
    reps = []
    for r in range(3):
        wt, scale = synth.int8_weight(n, k, synth.seed(1, r) + 2)
        reps.append(ctx.upload_i8(wt, scale))
    a = synth.activations(1, k, synth.seed(1) + 2)
    da = hip.DeviceArray.from_numpy(a)
    out = hip.DeviceArray((1, n), np.float32)
    for i in range(9):
        reps[i % 3].mm_dev(da.ptr, 1, out.ptr)
    ctx.sync()
    log(f"pmc: 9 launches of {DOM_KERNEL} at K={k} N={n}, "
        f"{int8_linear_bytes(1, k, n)} algorithmic bytes each")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--replicas", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-detail", action="store_true")
    ap.add_argument("--no-graphs", action="store_true",
                    help="GPT-2 decode steps launched eagerly rather than from a captured graph (the same "
                         "kernels; rocprofv3's kernel trace does not survive graph capture on this image)")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="only the counter-collection workload (run under rocprofv3 --pmc)")
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
    if args.pmc_pass:
        pmc_pass(fa, hip, synth, ctx, log)
        return

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

    # ---------------- headline: M=1 int8 sweep, full linear ----------------
    R = args.replicas
    shapes = list(synth.SWEEP_KN)
    weights, host_w0, acts, outs = [], [], [], []
    t0 = time.time()
    for si, (k, n) in enumerate(shapes):
        reps = []
        for r in range(R):
            wt, scale = synth.int8_weight(n, k, synth.seed(1, r) + si)
            reps.append(ctx.upload_i8(wt, scale))
            if r == 0:
                host_w0.append((wt, scale))
        weights.append(reps)
        a = synth.activations(1, k, synth.seed(1) + si)
        acts.append((a, hip.DeviceArray.from_numpy(a)))
        outs.append(hip.DeviceArray((1, n), np.float32))
    log(f"uploaded {R} replicas of {len(shapes)} shapes in {time.time() - t0:.1f}s")

    def step(i):
        for si in range(len(shapes)):
            w = weights[si][i % R]
            w.mm_dev(acts[si][1].ptr, 1, outs[si].ptr)

    for i in range(args.warmup):
        step(i)
    hip.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    e1.synchronize()
    ctx.sync()
    ms_total = e0.elapsed_ms(e1)
    ms_step = ms_total / args.steps
    step_bytes = sum(int8_linear_bytes(1, k, n) for k, n in shapes)
    value = step_bytes / (ms_step * 1e-3) / 1e9
    log(f"M=1 sweep: {ms_step * 1e3:.1f} us/step, {value:.0f} GB/s")

    # correctness spot check of the timed outputs against the oracle-free
    # path: the host entry point (same kernels) on replica (steps-1) % R
    detail = {"int8_m1_full_linear": {}, "int8_m1_gemv_kernel": {}}
    for si, (k, n) in enumerate(shapes):
        w = weights[si][0]
        us = time_loop(lambda i, w=w, si=si: weights[si][i % R].mm_dev(acts[si][1].ptr, 1, outs[si].ptr), 30) * 1e3
        detail["int8_m1_full_linear"][f"K{k}_N{n}"] = {
            "us": round(us, 2), "GBps": round(int8_linear_bytes(1, k, n) / (us * 1e-6) / 1e9, 1)}

    # ---------------- the GEMV kernel alone on pre-quantised input -------------
    gemv_rows = {}
    for si, (k, n) in enumerate(shapes):
        kp = fa.quant_pitch(k)
        a8 = hip.DeviceArray((1, kp), np.int8)
        sa = hip.DeviceArray((1,), np.float32)
        oi = hip.DeviceArray((1, 32), np.uint32)
        ov = hip.DeviceArray((1, 32), np.float32)
        ctx.quant_dev(acts[si][1].ptr, 1, k, a8.ptr, sa.ptr, oi.ptr, ov.ptr)
        us = time_loop(lambda i, si=si: weights[si][i % R].mm_q_dev(a8.ptr, sa.ptr, oi.ptr, ov.ptr, 1,
                                                                   outs[si].ptr), 60) * 1e3
        gb = gemv_kernel_bytes(1, k, n) / (us * 1e-6) / 1e9
        gemv_rows[(k, n)] = (us, gb)
        detail["int8_m1_gemv_kernel"][f"K{k}_N{n}"] = {"us": round(us, 2), "GBps": round(gb, 1),
                                                       "frac": round(gb / HBM_PEAK_GBS, 3)}
        qus = time_loop(lambda i, si=si: ctx.quant_dev(acts[si][1].ptr, 1, k, a8.ptr, sa.ptr, oi.ptr,
                                                       ov.ptr), 60) * 1e3
        detail["int8_m1_gemv_kernel"][f"K{k}_N{n}"]["quant_us"] = round(qus, 2)
    # ---------------- roofline: the dominant launch of the step -------------
    # at M=1 the full linear is the single fused kernel: time it alone, 60
    # launches over the weight replicas, HIP events on the library's stream
    dom = DOM_SHAPE
    dsi = shapes.index(dom)
    us_dom = time_loop(lambda i: weights[dsi][i % R].mm_dev(acts[dsi][1].ptr, 1, outs[dsi].ptr), 60) * 1e3
    gb_dom = int8_linear_bytes(1, *dom) / (us_dom * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(gb_dom, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gb_dom / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                "kernel": f"{DOM_KERNEL} (M=1, K={dom[0]}, N={dom[1]})",
                "bytes_per_launch": int8_linear_bytes(1, *dom), "us_per_launch": round(us_dom, 2)}

    if not args.no_detail:
        # ---------------- the sweep's other M (full linear and GEMM-only) ----------------
        # decode batches (M=4, 16: HBM-bound, GB/s) and M=128 (HBM-bound at
        # these K, N); weights rotated over the same replicas
        detail["int8_sweep_m"] = {}
        for m in (4, 16, 128):
            row = {}
            for si, (k, n) in enumerate(shapes):
                a = synth.activations(m, k, synth.seed(1, 20 + m) + si)
                da = hip.DeviceArray.from_numpy(a)
                do = hip.DeviceArray((m, n), np.float32)
                us = time_loop(lambda i, si=si: weights[si][i % R].mm_dev(da.ptr, m, do.ptr), 30) * 1e3
                kp = fa.quant_pitch(k)
                a8 = hip.DeviceArray((m, kp), np.int8)
                sa = hip.DeviceArray((m,), np.float32)
                oi = hip.DeviceArray((m, 32), np.uint32)
                ov = hip.DeviceArray((m, 32), np.float32)
                ctx.quant_dev(da.ptr, m, k, a8.ptr, sa.ptr, oi.ptr, ov.ptr)
                gus = time_loop(lambda i, si=si: weights[si][i % R].mm_q_dev(a8.ptr, sa.ptr, oi.ptr, ov.ptr, m,
                                                                            do.ptr), 30) * 1e3
                row[f"K{k}_N{n}"] = {"full_linear_us": round(us, 2),
                                     "full_linear_GBps": round(int8_linear_bytes(m, k, n) / (us * 1e-6) / 1e9, 1),
                                     "gemm_only_us": round(gus, 2),
                                     "gemm_only_GBps": round(gemv_kernel_bytes(m, k, n) / (gus * 1e-6) / 1e9, 1)}
            detail["int8_sweep_m"][f"M{m}"] = row
            log(f"M={m}: {row}")
        # ---------------- prefill: M=2048 MFMA-bound shapes ----------------
        detail["int8_m2048_gemm"] = {}
        for (k, n) in [(4096, 14336), (14336, 4096)]:
            wt, scale = synth.int8_weight(n, k, synth.seed(1, 7))
            w = ctx.upload_i8(wt, scale)
            del wt
            a = synth.activations(2048, k, synth.seed(1, 8))
            da = hip.DeviceArray.from_numpy(a)
            do = hip.DeviceArray((2048, n), np.float32)
            # ~150 us launches: 10 warm-up launches, then the median of three
            # trials of 20 (single trials of 10 vary by ~15% on the clock)
            def med3(fn):
                return float(np.median([time_loop(fn, 20, warm=10 if r == 0 else 0) for r in range(3)])) * 1e3
            us = med3(lambda i: w.mm_dev(da.ptr, 2048, do.ptr))
            kp = fa.quant_pitch(k)
            a8 = hip.DeviceArray((2048, kp), np.int8)
            sa = hip.DeviceArray((2048,), np.float32)
            oi = hip.DeviceArray((2048, 32), np.uint32)
            ov = hip.DeviceArray((2048, 32), np.float32)
            ctx.quant_dev(da.ptr, 2048, k, a8.ptr, sa.ptr, oi.ptr, ov.ptr)
            gus = med3(lambda i: w.mm_q_dev(a8.ptr, sa.ptr, oi.ptr, ov.ptr, 2048, do.ptr))
            ops = 2.0 * 2048 * n * k
            detail["int8_m2048_gemm"][f"K{k}_N{n}"] = {
                "full_linear_us": round(us, 1), "full_linear_TOPS": round(ops / (us * 1e-6) / 1e12, 1),
                "gemm_us": round(gus, 1), "gemm_TOPS": round(ops / (gus * 1e-6) / 1e12, 1),
                "gemm_frac_int8_peak": round(ops / (gus * 1e-6) / 1e12 / INT8_PEAK_TOPS, 3)}
            log(f"M=2048 K={k} N={n}: {detail['int8_m2048_gemm'][f'K{k}_N{n}']}")
            w.free()
        # ---------------- int4 decode GEMV (Gemma-2-2b shapes) ----------------
        detail["int4_m1_gemv"] = {}
        for (k, n) in [(2304, 9216), (9216, 2304), (2304, 2048)]:
            reps = []
            for r in range(3):
                packed, s16, g = synth.int4_weight(n, k, synth.seed(2, r))
                reps.append(ctx.upload_i4(packed, s16, k, g))
            a = synth.activations(1, k, synth.seed(2, 9), outlier_scale=1.0)
            da = hip.DeviceArray.from_numpy(a)
            do = hip.DeviceArray((1, n), np.float32)
            us = time_loop(lambda i: reps[i % 3].mm_dev(da.ptr, 1, do.ptr), 60) * 1e3
            gb = int4_bytes(1, k, n) / (us * 1e-6) / 1e9
            detail["int4_m1_gemv"][f"K{k}_N{n}"] = {"us": round(us, 2), "GBps": round(gb, 1),
                                                    "frac": round(gb / HBM_PEAK_GBS, 3)}
            for w in reps:
                w.free()
        # ---------------- affine int4 (q4a) decode GEMV, same shapes ----------------
        detail["q4a_m1_gemv"] = {}
        for (k, n) in [(2304, 9216), (9216, 2304), (2304, 2048)]:
            reps = []
            for r in range(3):
                rng = np.random.default_rng(synth.seed(5, r))
                wsrc = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
                packed, s16, m16, g = convert.put_q4a(wsrc, True)
                del wsrc
                reps.append(ctx.upload_q4a(packed, s16, m16, k, g))
            a = synth.activations(1, k, synth.seed(5, 9), outlier_scale=1.0)
            da = hip.DeviceArray.from_numpy(a)
            do = hip.DeviceArray((1, n), np.float32)
            us = time_loop(lambda i: reps[i % 3].mm_dev(da.ptr, 1, do.ptr), 60) * 1e3
            gb = q4a_bytes(1, k, n, g) / (us * 1e-6) / 1e9
            detail["q4a_m1_gemv"][f"K{k}_N{n}"] = {"us": round(us, 2), "GBps": round(gb, 1),
                                                   "frac": round(gb / HBM_PEAK_GBS, 3)}
            for w in reps:
                w.free()
        # ---------------- unembed row dot (Bundle::rowdot_f32) ----------------
        # the tied f16 unembed of Gemma-2 (256000 x 2304, 1.18 GB: beyond the
        # MALL, one table suffices) and its rowi8 form, the GPT-2 f16 head
        detail["unembed_rowdot"] = {}
        for name, rows, d, kind in [("gemma2_f16", 256000, 2304, "f16"), ("gemma2_rowi8", 256000, 2304, "rowi8"),
                                    ("gpt2_f16", 50257, 768, "f16")]:
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
            log(f"rowdot {name}: {detail['unembed_rowdot'][name]}")
            t.free()
        # ---------------- MoE layer (config 4) ----------------
        detail["moe_qwen3_layer"] = {}
        E, d, mi, topk = 128, 2048, 768, 8
        gate, gs, up, us_, down, ds = synth.moe_layer(E, d, mi, synth.seed(3))
        bank = ctx.upload_moe_i8(gate, gs, up, us_, down, ds)
        for T in (1, 512):
            rng = np.random.default_rng(synth.seed(3, T))
            x = hip.DeviceArray.from_numpy(rng.standard_normal((T, d), dtype=np.float32))
            lg = hip.DeviceArray.from_numpy(rng.standard_normal((T, E), dtype=np.float32))
            o = hip.DeviceArray((T, d), np.float32)
            us = time_loop(lambda i: bank.forward_dev(x.ptr, T, lg.ptr, topk, True, None, o.ptr), 10) * 1e3
            detail["moe_qwen3_layer"][f"T{T}"] = {"us": round(us, 1),
                                                  "flops_TF": round(2 * T * topk * 3 * d * mi / (us * 1e-6) / 1e12, 2)}
        bank.free()
        # ---------------- GPT-2 greedy decode (config 0) ----------------
        # GPT-2 small int8, random init, 32-token seeded prompt, 128 greedy
        # tokens (Gpt2::generate), whole call timed on the host clock; the
        # decode rate excludes the prefill (generate(128) - generate(1))
        import tempfile
        detail["gpt2_decode"] = {}
        with tempfile.TemporaryDirectory() as tmp:
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
                log(f"gpt2 decode kv_int8={kv8}: {detail['gpt2_decode']['kv_int8' if kv8 else 'kv_f32']}")
                g.free()
            if not args.no_cpu:
                import oracle  # the reference's GPT-2 restated in C (the CPU rate beside the device's)

                m_, arrs = oracle.read_bundle(stem)
                threads = min(os.cpu_count() or 1, 16)
                ref = oracle.Gpt2(m_, arrs, nthreads=threads)
                g = fa.Gpt2(b)
                t0 = time.perf_counter()
                rt = ref.generate(prompt, 16)
                el = time.perf_counter() - t0
                same = bool(np.array_equal(rt, g.generate(prompt, 16)))
                detail["gpt2_decode"]["cpu_oracle"] = {"tok_s": round(16 / el, 2), "threads": threads,
                                                       "sample": "16 tokens after the 32-token prompt",
                                                       "tokens_identical": same}
                log(f"gpt2 oracle: {detail['gpt2_decode']['cpu_oracle']}")
                g.free()
            b.close()
        # ---------------- Gemma-2-2b int4 greedy decode (config 2) ----------------
        # 26 layers, int4 g=32 (seeded random nibbles and f16 scales), f16 embed
        # and tied unembed, 64-token seeded prompt, 256 greedy tokens, batch 1
        detail["gemma2_decode"] = {}
        with tempfile.TemporaryDirectory() as tmp:
            stem = os.path.join(tmp, "gemma2")
            synth.write_gemma2_bundle(stem, 2, raw=True)
            b = fa.Bundle(stem, ctx)
            g = fa.Gemma(b)
            g.set_graphs(not args.no_graphs)
            prompt = synth.gpt2_prompt(64, 256000, 7)
            g.generate(prompt, 8)
            runs = {}
            for n_new in (1, 256):
                t0 = time.perf_counter()
                g.generate(prompt, n_new)
                runs[n_new] = time.perf_counter() - t0
            dec_ms = (runs[256] - runs[1]) / 255 * 1e3
            detail["gemma2_decode"]["int4_kv_f32"] = {
                "tok_s": round(256 / runs[256], 1), "decode_ms_per_token": round(dec_ms, 3),
                "decode_tok_s": round(1e3 / dec_ms, 1), "prefill_plus_first_ms": round(runs[1] * 1e3, 1)}
            log(f"gemma2 decode: {detail['gemma2_decode']['int4_kv_f32']}")
            if not args.no_cpu:
                import oracle  # the reference's Gemma restated in C (the CPU rate beside the device's)

                m_, arrs = oracle.read_bundle(stem)
                threads = min(os.cpu_count() or 1, 16)
                ref = oracle.Gemma(m_, arrs, nthreads=threads)
                t0 = time.perf_counter()
                rt = ref.generate(prompt[:8], 4)
                el = time.perf_counter() - t0
                same = bool(np.array_equal(rt, g.generate(prompt[:8], 4)))
                detail["gemma2_decode"]["cpu_oracle"] = {"seconds": round(el, 2), "threads": threads,
                                                         "sample": "8-token prompt, 4 tokens (prefill-dominated)",
                                                         "tokens_identical": same}
                log(f"gemma2 oracle: {detail['gemma2_decode']['cpu_oracle']}")
            g.free()
            b.close()

        # ---------------- Qwen2.5-7B int8 prefill + greedy decode (config 4) ----------------
        # 28 layers, d 3584, 28 / 4 heads of 128, ffn 18944, vocab 152064, int8
        # per-column scales (seeded random bytes), q/k/v biases, untied f16
        # head; 2048-token seeded prompt, then 128 greedy tokens, batch 1
        detail["rope_decode"] = {}
        with tempfile.TemporaryDirectory() as tmp:
            stem = os.path.join(tmp, "qwen25")
            synth.write_rope_bundle(stem, 6, raw=True)
            b = fa.Bundle(stem, ctx)
            g = fa.Rope(b)
            g.set_graphs(not args.no_graphs)
            prompt = synth.gpt2_prompt(2048, 152064, 9)
            g.generate(prompt[:16], 4)
            runs = {}
            for n_new in (1, 128):
                t0 = time.perf_counter()
                g.generate(prompt, n_new)
                runs[n_new] = time.perf_counter() - t0
            dec_ms = (runs[128] - runs[1]) / 127 * 1e3
            detail["rope_decode"]["qwen25_7b_int8"] = {
                "prefill_tok_s": round(2048 / runs[1], 1), "prefill_plus_first_ms": round(runs[1] * 1e3, 1),
                "decode_ms_per_token": round(dec_ms, 3), "decode_tok_s": round(1e3 / dec_ms, 1),
                "total_s_2048_plus_128": round(runs[128], 3)}
            log(f"qwen2.5-7b: {detail['rope_decode']['qwen25_7b_int8']}")
            g.free()
            b.close()

    # ---------------- CPU baseline (the oracle's scalar restatement) ----------------
    cpu = None
    if not args.no_cpu:
        import oracle  # the CPU baseline leg: the reference's scalar i8 path restated in C

        threads = min(os.cpu_count() or 1, 16)
        t_end = time.time() + args.cpu_seconds
        iters, t_start = 0, time.time()
        while True:
            for si, (k, n) in enumerate(shapes):
                wt, scale = host_w0[si]
                oracle.mm_i8_mt(acts[si][0], wt, scale, threads)
            iters += 1
            if time.time() >= t_end:
                break
        el = time.time() - t_start
        cpu_gbs = iters * step_bytes / el / 1e9
        cpu = {"value": round(cpu_gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"{iters} passes of the M=1 int8 sweep (5 shapes, replica 0) in {el:.1f}s; "
                         f"oracle fro_mm_i8_mt: scalar i8dot built -O3 -march=x86-64, rayon-style split over N"}
        log(f"CPU baseline {cpu_gbs:.2f} GB/s on {threads} threads")

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "configs[1] isolated int8 linear sweep at M=1 (decode): full linear "
                               "(outlier-aware per-token quant + i8 dot + scale epilogue) over "
                               "(K,N) in " + str(shapes) + f", {R} weight replicas rotated",
                   "m": 1, "shapes": [list(s) for s in shapes]},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "detail": detail,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
