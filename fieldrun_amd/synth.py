"""Seeded synthetic workloads of the benchmark configs (host-side numpy).

Seeds are 0xF1E1D000 + config_index*1000 + replica.  Generated once on the
host; the same arrays feed the HIP path and the CPU oracle.
"""
from __future__ import annotations

import numpy as np

from . import convert

SEED0 = 0xF1E1D000

# the isolated int8 linear sweep
SWEEP_M = (1, 4, 16, 128, 2048)
SWEEP_KN = ((896, 4864), (4864, 896), (896, 151936), (4096, 14336), (14336, 4096))


def seed(config: int, replica: int = 0) -> int:
    return SEED0 + config * 1000 + replica


def outlier_channels(k: int, rng: np.random.Generator) -> np.ndarray:
    """round(0.01 K) fixed channels (the same for every row)."""
    n = max(1, int(round(0.01 * k)))
    return np.sort(rng.choice(k, n, replace=False))


def activations(m: int, k: int, s: int, outlier_scale: float = 20.0) -> np.ndarray:
    """A ~ N(0,1) (M,K) f32 with 1% of the channels multiplied by 20."""
    rng = np.random.default_rng(s)
    chans = outlier_channels(k, np.random.default_rng(s ^ 0x5A5A))
    a = rng.standard_normal((m, k), dtype=np.float32)
    a[:, chans] *= np.float32(outlier_scale)
    return a


def int8_weight(n: int, k: int, s: int):
    """W (N,K) int8 uniform in [-127,127]; f32 row scales that are
    f16-representable values in [1e-4, 3e-4]."""
    rng = np.random.default_rng(s + 1)
    wt = rng.integers(-127, 128, (n, k), dtype=np.int8)
    scale = rng.uniform(1e-4, 3e-4, n).astype(np.float16).astype(np.float32)
    return wt, scale


def int4_weight(n: int, k: int, s: int, std: float = 0.02):
    """put_i4 of N(0, std) weights, shape (out=N, in=K): packed, f16 scales, g."""
    rng = np.random.default_rng(s + 2)
    src = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(std)).astype(np.float32)
    return convert.put_i4(src, transpose=True)


def moe_layer(E: int, d: int, mi: int, s: int, act: int = 0, std: float = 0.02):
    """Experts as put_i8 stores them: (in,out) int8 + f32 scales (from f16)."""
    rng = np.random.default_rng(s + 3)
    gw = mi if act == 0 else 2 * mi

    def lin(out, inp):
        src = (rng.standard_normal((out, inp), dtype=np.float32) * np.float32(std)).astype(np.float32)
        w, s16 = convert.put_i8(src, transpose=True)
        return w, s16.astype(np.float32)

    gate, gs, up, us, down, ds = [], [], [], [], [], []
    for _ in range(E):
        w, sc = lin(gw, d); gate.append(w); gs.append(sc)
        if act == 0:
            w, sc = lin(mi, d); up.append(w); us.append(sc)
        w, sc = lin(d, mi); down.append(w); ds.append(sc)
    return gate, gs, up, us, down, ds


def moe_layer_ex(E: int, d: int, mi: int, s: int, dtype: str, act: int = 0, std: float = 0.02):
    """Experts as put_lin stores them in `dtype` ("int4", "q4a", "f16" or
    "f32", src/convert.rs:174-260): per matrix a dict with raw (the stored
    array: packed (out, ceil(in/2)) nibbles for int4 / q4a, (in, out) f16
    bits or f32 otherwise), scale / min (f16 bits, (out, ceil(in/g)); None
    where the dtype has none), g, inp and out.  Returns (gate, up, down),
    lists over experts (up empty for the packed gate_up of act 1)."""
    rng = np.random.default_rng(s + 5)
    gw = mi if act == 0 else 2 * mi

    def lin(out, inp):
        src = (rng.standard_normal((out, inp), dtype=np.float32) * np.float32(std)).astype(np.float32)
        if dtype == "int4":
            packed, s16, g = convert.put_i4(src, transpose=True)
            return {"raw": packed, "scale": s16.view(np.uint16), "min": None, "g": g, "inp": inp, "out": out}
        if dtype == "q4a":
            packed, s16, m16, g = convert.put_q4a(src, transpose=True)
            return {"raw": packed, "scale": s16.view(np.uint16), "min": m16.view(np.uint16), "g": g, "inp": inp,
                    "out": out}
        t = np.ascontiguousarray(src.T)  # (in, out)
        raw = t.astype(np.float16).view(np.uint16) if dtype == "f16" else t
        return {"raw": raw, "scale": None, "min": None, "g": 0, "inp": inp, "out": out}

    gate, up, down = [], [], []
    for _ in range(E):
        gate.append(lin(gw, d))
        if act == 0:
            up.append(lin(mi, d))
        down.append(lin(d, mi))
    return gate, up, down


# ---- synthetic random-init bundles in the reference format (the benchmark
# configs; array names and layouts as src/convert.rs writes them) ----------

def gpt2_prompt(n: int, vocab: int, s: int) -> np.ndarray:
    """A seeded uniform-random prompt of n token ids in [0, vocab)."""
    return np.random.default_rng(s).integers(0, vocab, n).astype(np.int64)


def write_gpt2_bundle(stem: str, s: int, n_layer: int = 12, n_head: int = 12, d: int = 768,
                      n_pos: int = 1024, vocab: int = 50257, std: float = 0.02) -> dict:
    """a GPT-2-small-shaped int8 bundle (convert_gpt2,
    src/convert.rs:505-545 with dtype int8): wte / wpe / ln_f in f16, LN
    gains 1 and biases 0, the four Conv1D linears per layer int8 from
    (in, out) sources with f16 biases.  Weights ~ N(0, std)."""
    from .bundle import BundleWriter, manifest
    rng = np.random.default_rng(s)
    nrm = lambda *shape: (rng.standard_normal(shape, dtype=np.float32) * np.float32(std))
    w = BundleWriter(stem)
    w.put_embed("wte", nrm(vocab, d), "f16", "int8")
    w.put_small("wpe", nrm(n_pos, d), None, "int8")
    w.put_small("ln_f.weight", np.ones(d, np.float32), None, "int8")
    w.put_small("ln_f.bias", np.zeros(d, np.float32), None, "int8")
    for l in range(n_layer):
        for ln in ("ln_1", "ln_2"):
            w.put_small(f"h{l}.{ln}.weight", np.ones(d, np.float32), None, "int8")
            w.put_small(f"h{l}.{ln}.bias", np.zeros(d, np.float32), None, "int8")
        for name, (i, o) in (("attn.c_attn", (d, 3 * d)), ("attn.c_proj", (d, d)),
                             ("mlp.c_fc", (d, 4 * d)), ("mlp.c_proj", (4 * d, d))):
            w.put_i8(f"h{l}.{name}.weight", nrm(i, o), False)
            w.put_small(f"h{l}.{name}.bias", np.zeros(o, np.float32), None, "int8")
    m = manifest("gpt2", [n_layer, n_head, d, n_pos, vocab])
    w.finish(m)
    return m


def write_qwen3moe_layer_bundle(stem: str, s: int, n_exp: int = 128, d: int = 2048, mi: int = 768,
                                topk: int = 8, std: float = 0.02, dtype: str = "int8") -> dict:
    """one Qwen3-MoE routed layer as convert_qwen3moe writes it
    (src/convert.rs:872-936, every linear put_lin at the converter's dtype:
    "int8", "int4", "q4a", "f16" or "f32"): the router l0.gate and the
    experts l0.experts.{e}.gate / .up / .down, each from an (out, in) Linear
    source.  The manifest's config follows that converter's vector for a
    one-layer model (Qwen3-30B-A3B attention dims, all of its arrays but the
    MoE layer absent)."""
    from .bundle import BundleWriter, manifest
    rng = np.random.default_rng(s)
    nrm = lambda *shape: (rng.standard_normal(shape, dtype=np.float32) * np.float32(std))
    w = BundleWriter(stem)
    w.put_lin("l0.gate", nrm(n_exp, d), dtype)
    for e in range(n_exp):
        w.put_lin(f"l0.experts.{e}.gate", nrm(mi, d), dtype)
        w.put_lin(f"l0.experts.{e}.up", nrm(mi, d), dtype)
        w.put_lin(f"l0.experts.{e}.down", nrm(d, mi), dtype)
    nh, nkv, hd, vocab = 32, 4, 128, 151936
    cfg = [1, nh, nkv, hd, d, 6144, vocab, 0, n_exp, topk, mi, 1, 1, 0]
    m = manifest("qwen3moe", cfg, [1e6, 1e-6])
    w.finish(m)
    return m


def _parallel(jobs, workers: int = 8):
    """Run the zero-argument jobs on a thread pool, results in job order
    (numpy's bulk generators release the GIL, so seeded chunks come out
    several times faster; each job owns its generator, so the bytes do not
    depend on the thread count or the scheduling)."""
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(workers) as ex:
        return list(ex.map(lambda f: f(), jobs))


def _f16_table_chunks(ss, rows: int, d: int, std: float):
    """A (rows, d) table of N(0, std) values in f16, 8192-row chunks each
    drawn from its own child of the seed sequence ss."""
    def chunk(r0, child):
        g = np.random.default_rng(child)
        return (g.standard_normal((min(8192, rows - r0), d), dtype=np.float32) * np.float32(std)).astype(np.float16)
    starts = list(range(0, rows, 8192))
    kids = ss.spawn(len(starts))
    return np.concatenate(_parallel([lambda r0=r0, c=c: chunk(r0, c) for r0, c in zip(starts, kids)]))


def write_gemma2_bundle(stem: str, s: int, n_layer: int = 26, n_head: int = 8, n_kv: int = 4, hd: int = 256,
                        d: int = 2304, ffn: int = 9216, vocab: int = 256000, std: float = 0.02,
                        dtype: str = "int4", norm_std: float = 0.0, raw: bool = False, embed: str = "f16") -> dict:
    """a Gemma-2-2b-shaped bundle as convert_gemma writes it
    (src/convert.rs:636-657 via write_layers 1266-1300): the f16 embed (tied
    unembed), the RMSNorm gains with the +1 baked in (1 + w, w = 0 at init,
    or N(0, norm_std)), and the seven projections per layer put_lin from
    (out, in) sources in `dtype` ("int4" groups of 32, "int8", "q4a").
    config [nl, H, nkv, hd, d, ffn, vocab, tied]; config_f [theta, eps,
    attn_cap, final_cap, query_pre_attn_scalar, sqrt(d)] as Gemma-2-2b.
    raw: the int4 linears as seeded random nibbles with f16 scales written
    directly (the configs[2] size in seconds rather than minutes).
    embed: the tied table's type when not raw, "f16", "f32" or "int8"
    (rowi8 with f16 per-row scales, put_embed_i8)."""
    from .bundle import BundleWriter, manifest
    rng = np.random.default_rng(s)
    nrm = lambda *shape: (rng.standard_normal(shape, dtype=np.float32) * np.float32(std))
    gain = lambda: (np.float32(1.0) + rng.standard_normal(d, dtype=np.float32) * np.float32(norm_std)
                    if norm_std else np.ones(d, np.float32))
    w = BundleWriter(stem)
    ss = np.random.SeedSequence([s, 2])  # the raw tensors' streams (one child per chunk / matrix)
    if raw:  # the f16 embed in row chunks (no full-size f32 temporary)
        emb = _f16_table_chunks(ss, vocab, d, std)
        nb = w._write(np.ascontiguousarray(emb.view(np.uint16)))
        w.entry("embed", "f16", emb.shape, nb)
        del emb
    elif embed == "f32":
        w.put_f32("embed", nrm(vocab, d))
    else:
        w.put_embed("embed", nrm(vocab, d), embed, dtype)
    w.put_small("norm", gain(), None, dtype)
    shapes = {"self_attn.q_proj": (n_head * hd, d), "self_attn.k_proj": (n_kv * hd, d),
              "self_attn.v_proj": (n_kv * hd, d), "self_attn.o_proj": (d, n_head * hd),
              "mlp.gate_proj": (ffn, d), "mlp.up_proj": (ffn, d), "mlp.down_proj": (d, ffn)}
    def nibbles(o, i, child, g=32):  # seeded random nibbles and f16 group scales, as stored
        r = np.random.default_rng(child)
        packed = r.integers(0, 256, (o, (i + 1) // 2), dtype=np.uint8)
        return packed, r.uniform(0.5, 1.0, (o, (i + g - 1) // g)).astype(np.float32) * np.float32(std / 2.5)

    for l in range(n_layer):
        for nm in ("input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                   "post_feedforward_layernorm"):
            w.put_small(f"l{l}.{nm}", gain(), None, dtype)
        if raw:
            kids = ss.spawn(len(shapes))
            mats = _parallel([lambda o=o, i=i, c=c: nibbles(o, i, c) for (o, i), c in zip(shapes.values(), kids)])
            for (proj, (o, i)), (packed, s16) in zip(shapes.items(), mats):
                nb = w._write(np.ascontiguousarray(packed))
                w.entry(f"l{l}.{proj}", "i4", (o, i), nb, group=32)
                w.put_f16(f"l{l}.{proj}__scale", s16)
            del mats
            continue
        for proj, (o, i) in shapes.items():
            w.put_lin(f"l{l}.{proj}", nrm(o, i), dtype)
    m = manifest("gemma", [n_layer, n_head, n_kv, hd, d, ffn, vocab, 1],
                 [10000.0, 1e-6, 50.0, 30.0, float(hd), float(np.sqrt(d))])
    w.finish(m)
    return m


def write_rope_bundle(stem: str, s: int, n_layer: int = 28, n_head: int = 28, n_kv: int = 4, hd: int = 128,
                      d: int = 3584, ffn: int = 18944, vocab: int = 152064, std: float = 0.02, dtype: str = "int8",
                      qkv_bias: bool = True, qk_norm: bool = False, tied: bool = False, norm_std: float = 0.0,
                      theta: float = 1e6, eps: float = 1e-6, raw: bool = False) -> dict:
    """a Llama / Qwen2.5-7B-shaped bundle as convert_rope writes
    it (src/convert.rs:619-634 via write_layers 1266-1310): f16 embed (and
    lm_head unless tied), in_ln / post_ln RMSNorm weights (1 at init, or
    1 + N(0, norm_std); no +1 bake), q/k/v biases (Qwen2.5) and per-head
    q/k norms (Qwen3) when asked, the seven projections put_lin from (out,
    in) sources in `dtype`.  raw: int8 linears as seeded random bytes with
    f16 per-column scales written as stored (the 7B size in seconds)."""
    from .bundle import BundleWriter, manifest
    rng = np.random.default_rng(s)
    nrm = lambda *shape: (rng.standard_normal(shape, dtype=np.float32) * np.float32(std))
    gain = lambda n: (np.float32(1.0) + rng.standard_normal(n, dtype=np.float32) * np.float32(norm_std)
                      if norm_std else np.ones(n, np.float32))
    w = BundleWriter(stem)
    ss = np.random.SeedSequence([s, 4])  # the large tensors' streams (one child per chunk / matrix)

    def table(name):
        t = _f16_table_chunks(ss, vocab, d, std)
        nb = w._write(np.ascontiguousarray(t.view(np.uint16)))
        w.entry(name, "f16", t.shape, nb)

    def raw_i8(o, i, child):  # seeded random bytes (in, out) and f16 per-column scales, as stored
        r = np.random.default_rng(child)
        return (r.integers(-127, 128, (i, o), dtype=np.int8),
                r.uniform(0.5, 1.0, o).astype(np.float32) * np.float32(std / 40))

    table("embed")
    w.put_small("norm", gain(d), None, dtype)
    if not tied:
        table("lm_head")
    shapes = {"self_attn.q_proj": (n_head * hd, d), "self_attn.k_proj": (n_kv * hd, d),
              "self_attn.v_proj": (n_kv * hd, d), "self_attn.o_proj": (d, n_head * hd),
              "mlp.gate_proj": (ffn, d), "mlp.up_proj": (ffn, d), "mlp.down_proj": (d, ffn)}
    for l in range(n_layer):
        w.put_small(f"l{l}.in_ln", gain(d), None, dtype)
        w.put_small(f"l{l}.post_ln", gain(d), None, dtype)
        if raw and dtype == "int8":
            kids = ss.spawn(len(shapes))
            mats = _parallel([lambda o=o, i=i, c=c: raw_i8(o, i, c) for (o, i), c in zip(shapes.values(), kids)])
            for (proj, (o, i)), (q, sc) in zip(shapes.items(), mats):
                nb = w._write(np.ascontiguousarray(q))
                w.entry(f"l{l}.{proj}", "i8", (i, o), nb)
                w.put_f16(f"l{l}.{proj}__scale", sc)
            del mats
        else:
            for proj, (o, i) in shapes.items():
                w.put_lin(f"l{l}.{proj}", nrm(o, i), dtype)
        if qkv_bias:
            for proj in ("q_proj", "k_proj", "v_proj"):
                o = shapes[f"self_attn.{proj}"][0]
                w.put_small(f"l{l}.self_attn.{proj}.bias", nrm(o), None, dtype)
        if qk_norm:
            w.put_small(f"l{l}.self_attn.q_norm", gain(hd), None, dtype)
            w.put_small(f"l{l}.self_attn.k_norm", gain(hd), None, dtype)
    m = manifest("rope", [n_layer, n_head, n_kv, hd, d, ffn, vocab, int(tied)], [theta, eps])
    w.finish(m)
    return m
