"""The oracle's Gemma-2 (src/gemma.rs: norm 66-77, rope 79-94,
forward_block 242-291 / _q 293-363, generate 403-431) pinned by an
independent float64 numpy model of the same forward (the int4 linears
through the oracle's pinned mm_i4): tokens equal and logits within f32
tolerance for the f32 cache, and the RMSNorm by closed forms."""
import numpy as np
import pytest

import oracle
from fieldrun_amd import synth


def f64_gemma(m, arrs, prompt, n_new):
    L, H, KV, hd, d, ffn, V = m["config"][:7]
    rope_arch = m["arch"] == "rope"
    if rope_arch:  # rope.rs: no embedding scale, no soft-cap / window / post-norms, SiLU
        (theta, eps), cap, qscalar, escale = m["config_f"][:2], 0.0, float(hd), 1.0
    else:
        theta, eps, cap, _fc, qscalar, escale = m["config_f"][:6]
    rep, half, window = H // KV, hd // 2, 4096
    f = lambda n: arrs[n].astype(np.float64)
    emb = f("embed")
    inv = 1.0 / theta ** (2.0 * np.arange(half) / hd)
    ginfo = {e["name"]: e for e in m["arrays"]}

    def mm(x, name):
        k = ginfo[name]["shape"][1]
        return oracle.mm_i4(x.astype(np.float32), arrs[name], arrs[name + "__scale"].astype(np.float32), k,
                            ginfo[name].get("group") or 32).astype(np.float64)

    def norm(x, name):
        ms = (x * x).mean(-1, keepdims=True)
        return x / np.sqrt(ms + eps) * f(name)

    def proj(a, name):
        y = mm(a, name)
        return y + f(name + ".bias") if name + ".bias" in arrs else y

    def head_norm(x, name, nh):
        if name not in arrs:
            return x
        x = x.reshape(x.shape[0], nh, hd)
        x = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * f(name)
        return x.reshape(x.shape[0], nh * hd)

    def rope(x, nh, pos0):
        x = x.copy()
        for i in range(x.shape[0]):
            ang = (pos0 + i) * inv
            c, s = np.cos(ang), np.sin(ang)
            for h in range(nh):
                a, b = x[i, h * hd:h * hd + half].copy(), x[i, h * hd + half:(h + 1) * hd].copy()
                x[i, h * hd:h * hd + half] = a * c - b * s
                x[i, h * hd + half:(h + 1) * hd] = b * c + a * s
        return x

    K = [np.zeros((0, KV * hd)) for _ in range(L)]
    Vc = [np.zeros((0, KV * hd)) for _ in range(L)]

    def block(x, cur):
        mr = x.shape[0]
        for l in range(L):
            p = f"l{l}."
            a = norm(x, p + ("in_ln" if rope_arch else "input_layernorm"))
            q = rope(head_norm(proj(a, p + "self_attn.q_proj"), p + "self_attn.q_norm", H), H, cur)
            k = rope(head_norm(proj(a, p + "self_attn.k_proj"), p + "self_attn.k_norm", KV), KV, cur)
            v = proj(a, p + "self_attn.v_proj")
            K[l] = np.concatenate([K[l], k])
            Vc[l] = np.concatenate([Vc[l], v])
            att = np.zeros((mr, H * hd))
            for h in range(H):
                kv = h // rep
                s = q[:, h * hd:(h + 1) * hd] @ K[l][:, kv * hd:(kv + 1) * hd].T / np.sqrt(qscalar)
                if cap > 0:
                    s = cap * np.tanh(s / cap)
                for i in range(mr):
                    ab = cur + i
                    s[i, ab + 1:] = -np.inf
                    if not rope_arch and l % 2 == 0 and ab >= window:
                        s[i, :ab - window + 1] = -np.inf
                s = np.exp(s - s.max(1, keepdims=True))
                s /= s.sum(1, keepdims=True)
                att[:, h * hd:(h + 1) * hd] = s @ Vc[l][:, kv * hd:(kv + 1) * hd]
            o = mm(att, p + "self_attn.o_proj")
            x = x + (o if rope_arch else norm(o, p + "post_attention_layernorm"))
            a2 = norm(x, p + ("post_ln" if rope_arch else "pre_feedforward_layernorm"))
            gt, up = mm(a2, p + "mlp.gate_proj"), mm(a2, p + "mlp.up_proj")
            if rope_arch:
                hm = gt / (1 + np.exp(-gt)) * up
            else:
                c = np.sqrt(2 / np.pi)
                hm = 0.5 * gt * (1 + np.tanh(c * (gt + 0.044715 * gt ** 3))) * up
            dn = mm(hm, p + "mlp.down_proj")
            x = x + (dn if rope_arch else norm(dn, p + "post_feedforward_layernorm"))
        return x

    un = f("lm_head") if (rope_arch and not m["config"][7]) else emb

    def head(x):
        lg = un @ norm(x[-1:], "norm")[0]
        return int(np.flatnonzero(lg == lg.max())[-1]), lg

    x = block(emb[prompt] * escale, 0)
    toks, lgs = [], []
    nxt, lg = head(x)
    pos = len(prompt)
    while True:
        toks.append(nxt)
        lgs.append(lg)
        if len(toks) == n_new:
            return np.array(toks), np.array(lgs)
        x = block(emb[[nxt]] * escale, pos)
        nxt, lg = head(x)
        pos += 1


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    stem = str(tmp_path_factory.mktemp("gemma") / "small")
    synth.write_gemma2_bundle(stem, 3, n_layer=2, n_head=4, n_kv=2, hd=32, d=128, ffn=256, vocab=500, std=0.3,
                              norm_std=0.1)
    return oracle.read_bundle(stem)


def test_oracle_gemma_matches_f64_model(small):
    m, arrs = small
    g = oracle.Gemma(m, arrs, nthreads=4)
    prompt = synth.gpt2_prompt(7, 500, 1)
    toks, lg = g.generate(prompt, 10, with_logits=True)
    rt, rlg = f64_gemma(m, arrs, prompt, 10)
    assert np.array_equal(toks, rt)
    assert np.abs(lg - rlg).max() <= 2e-5 * np.abs(rlg).max()


def test_rmsnorm_closed_forms():
    d = 48
    w = np.linspace(0.5, 1.5, d).astype(np.float32)
    x = np.full((1, d), 3.0, np.float32)            # ms = 9 exactly: out = 3 / sqrt(9 + eps) * w
    out = oracle.rmsnorm(x, w, 0.0)
    assert np.array_equal(out[0], (np.float32(3.0) * np.float32(1 / 3) * w).astype(np.float32)) or \
        np.abs(out[0] - w).max() <= 1e-6
    x = np.random.default_rng(2).integers(-20, 20, (4, d)).astype(np.float32)
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * w
    assert np.allclose(oracle.rmsnorm(x, w, 1e-6), ref, rtol=3e-7, atol=1e-7)


@pytest.mark.parametrize("kw", [dict(qkv_bias=True), dict(qkv_bias=False, qk_norm=True, tied=True)])
def test_oracle_rope_matches_f64_model(tmp_path, kw):
    stem = str(tmp_path / "r")
    synth.write_rope_bundle(stem, 4, n_layer=2, n_head=4, n_kv=2, hd=32, d=128, ffn=256, vocab=500, std=0.1,
                            norm_std=0.1, dtype="int4", **kw)
    m, arrs = oracle.read_bundle(stem)
    g = oracle.Rope(m, arrs, nthreads=4)
    prompt = synth.gpt2_prompt(6, 500, 2)
    toks, lg = g.generate(prompt, 10, with_logits=True)
    rt, rlg = f64_gemma(m, arrs, prompt, 10)
    assert np.array_equal(toks, rt)
    assert np.abs(lg - rlg).max() <= 2e-5 * np.abs(rlg).max()
    assert len(set(toks.tolist())) > 3
