// gemma.hip — Gemma-2 greedy decode on the device with a KV cache, gfx950.
//
// Restates Gemma of /root/reference/src/gemma.rs: new (52-60), norm (66-77,
// RMSNorm with the (1 + w) gain baked at export), rope (79-94),
// forward_block (242-291), forward_block_q (293-363, the int8 cache),
// head_argmax (386-390) and generate (403-431).  Per layer, m rows at
// positions cur .. cur+m-1:
//   a    = norm(x, input_layernorm)            (fused into the previous step)
//   qkv  = mm(a, [q_proj | k_proj | v_proj])   (one launch: the three weights'
//                                               output columns side by side)
//   q, k = rope(q, k); k, v -> cache (int8: per kv-head scale)
//   att  = softmax(softcap(q k^T * qscalar^-0.5), causal, sliding on even
//          layers) v, grouped-query (head h reads kv head h / (H / nkv))
//   x    = x + norm(mm(att, o_proj), post_attention_layernorm)
//   a    = norm(x, pre_feedforward_layernorm)
//   gu   = mm(a, [gate_proj | up_proj]);  h = gelu_tanh(gate) * up
//   x    = x + norm(mm(h, down_proj), post_feedforward_layernorm)
// then norm(x, "norm") and the tied f16 unembed with its argmax.
// Every step follows the reference's f32 order, so tokens and logits are
// the reference's bit for bit: the RMSNorm sum of squares is the fold from
// -0.0 in index order; the RoPE cos / sin are the host libm's (the table is
// computed on the host, where the reference computes them); scores and
// values follow a.dot's order (MM_KC-key blocks, each an FMA chain from +0,
// added in order; a head's scores are one block); the soft-cap and GELU use the libm
// tanhf restatement, the softmax the expf one and a key-order sum; the
// linears take their reference-order kernels (int4: i4_dot_avx2's order at
// M = 1, dequantise + a.dot's blocked order above; int8: the bit-exact M <= 16
// path, in chunks).
#include "frq_internal.h"
#include "libm_f32.h"
#include "quant_core.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <vector>

namespace frq {
namespace {

constexpr int GT = 256;

__device__ __forceinline__ float gwave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ float gblock_max(float v, float* red) {
    v = gwave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// rows_f32("embed", ids) * escale (gemma.rs:424, 429): row t is token ids[t]
// (rel: ids[cur - P + t], the token the last argmax wrote).
// (tstride > 0: a batch step, row t is sequence t's last token, ids[t tstride + cur - P])
// The embedding rows (Bundle::rows_f32, src/bundle.rs:936-955: an f32, f16
// or rowi8 table, a rowi8 element q as f32 times its row's scale rs[id])
// times escale (gemma.rs:105; 1 on the Llama / Qwen family).
__global__ __launch_bounds__(GT) void gm_embed_kernel(const uint8_t* __restrict__ tab, size_t pitch, int dt,
                                                      const float* __restrict__ rs, int d, float escale,
                                                      const int64_t* __restrict__ ids, int rel, int P,
                                                      const int* __restrict__ curp, float* __restrict__ x,
                                                      size_t tstride = 0) {
    const int t = blockIdx.x;
    const int64_t id = ids[rel ? (tstride ? t * tstride + *curp - P : *curp - P + t) : t];
    const uint8_t* row = tab + (size_t)id * pitch;
    float* xo = x + (size_t)t * d;
    if (dt == FRQ_DT_F16) {
        for (int c = threadIdx.x; c < d; c += GT) xo[c] = h2f(reinterpret_cast<const uint16_t*>(row)[c]) * escale;
    } else if (dt == FRQ_DT_F32) {
        for (int c = threadIdx.x; c < d; c += GT) xo[c] = reinterpret_cast<const float*>(row)[c] * escale;
    } else {
        const float sc = rs[id];
        for (int c = threadIdx.x; c < d; c += GT) xo[c] = ((float)(int8_t)row[c] * sc) * escale;
    }
}

// Threads of the norm kernel: eight waves, so the fold runs as eight
// speculative segments (seq_sum_spec).
constexpr int NORM_NT = 512;

// One row's norm (gemma.rs:66-77) from LDS v (d values) into dst: ms = the
// fold from -0.0 of v*v in index order / n (seq_sum_spec: bit-identical to
// the one-lane chain), inv = 1 / sqrt(ms + eps), dst = v * inv * w.
template <int NT>
__device__ __forceinline__ void rms_row(const float* v, float* sq, const float* __restrict__ w, int d, float eps, float* dst,
                        float* fsc) {
    for (int c = threadIdx.x; c < d; c += NT) sq[c] = v[c] * v[c];
    __syncthreads();
    const float ms = seq_sum_spec<NT>(sq, d, -0.0f, fsc) / (float)d;
    const float inv = 1.0f / sqrtf(ms + eps);
    for (int c = threadIdx.x; c < d; c += NT) dst[c] = v[c] * inv * w[c];
    __syncthreads();
}

// Row r = row0 + blockIdx.x.  y set: x += norm(y, wpost) (gemma's post-norm
// before the residual) or, wpost NULL, x += y (rope.rs); then out =
// norm(x, wnext).  LDS: three rows of d floats (each 16-byte aligned) and
// the fold's scratch.
template <int NT>
__host__ __device__ inline size_t gm_norm_lds_t(int d) {
    return (3 * (size_t)((d + 3) & ~3) + seq_sum_spec_scratch(NT)) * sizeof(float);
}
__host__ __device__ inline size_t gm_norm_lds(int d) { return gm_norm_lds_t<NORM_NT>(d); }

// The norm kernel's body for NT threads; the normalised row is left in LDS
// (returned) as well as written to out.
template <int NT>
__device__ __forceinline__ float* gm_norm_body(float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ wpost,
                               const float* __restrict__ wnext, float* __restrict__ out, int d, float eps,
                               size_t r, float* lds) {
    const int dp = (d + 3) & ~3;
    float* v = lds;
    float* sq = v + dp;
    float* t = sq + dp;
    float* fsc = t + dp;
    if (y && wpost) {
        for (int c = threadIdx.x; c < d; c += NT) v[c] = y[r + c];
        __syncthreads();
        rms_row<NT>(v, sq, wpost, d, eps, t, fsc);
        for (int c = threadIdx.x; c < d; c += NT) {
            const float nx = x[r + c] + t[c];
            x[r + c] = nx;
            v[c] = nx;
        }
    } else if (y) {  // rope.rs: x = x + y, no post-norm
        for (int c = threadIdx.x; c < d; c += NT) {
            const float nx = x[r + c] + y[r + c];
            x[r + c] = nx;
            v[c] = nx;
        }
    } else {
        for (int c = threadIdx.x; c < d; c += NT) v[c] = x[r + c];
    }
    __syncthreads();
    rms_row<NT>(v, sq, wnext, d, eps, t, fsc);
    for (int c = threadIdx.x; c < d; c += NT) out[r + c] = t[c];
    return t;
}

__global__ __launch_bounds__(NORM_NT) void gm_norm_kernel(float* __restrict__ x, const float* __restrict__ y,
                                                          const float* __restrict__ wpost,
                                                          const float* __restrict__ wnext, float* __restrict__ out,
                                                          int d, float eps, int row0, float* __restrict__ a4) {
    extern __shared__ float4 lds4[];
    const float* t = gm_norm_body<NORM_NT>(x, y, wpost, wnext, out, d, eps, (size_t)(row0 + blockIdx.x) * d,
                                           reinterpret_cast<float*>(lds4));
    if (a4)
        for (int c = threadIdx.x; c < d; c += NORM_NT) a4[(c >> 2) * 64 + 4 * (row0 + blockIdx.x) + (c & 3)] = t[c];
}

// The norm kernel with the row in registers: float4 q = tid + NORM_NT i of
// the row (d % 4 == 0, d <= 4 NORM_NT NV); every global load (y, x and both
// gains) is issued up front, the squares go to LDS for the fold.  The
// arithmetic is gm_norm_body's, operation for operation.  LDS: d floats and
// the fold's scratch.
// NT threads.
template <int NT = NORM_NT>
__host__ __device__ inline size_t gm_norm2_lds(int d) {
    return ((size_t)((d + 3) & ~3) + seq_sum_spec_scratch(NT)) * sizeof(float);
}
template <int NV, int NT>
__global__ __launch_bounds__(NT) void gm_norm2_kernel(float* __restrict__ x, const float* __restrict__ y,
                                                           const float* __restrict__ wpost,
                                                           const float* __restrict__ wnext, float* __restrict__ out,
                                                           int d, float eps, int row0, float* __restrict__ a4) {
    extern __shared__ float4 lds4[];
    float4* sq4 = lds4;
    float* sq = reinterpret_cast<float*>(lds4);
    float* fsc = sq + ((d + 3) & ~3);
    const int tid = threadIdx.x, d4 = d >> 2;
    const size_t r = (size_t)(row0 + blockIdx.x) * d;
    const float4* x4 = reinterpret_cast<const float4*>(x + r);
    const float4* y4 = y ? reinterpret_cast<const float4*>(y + r) : nullptr;
    const float4* wp4 = reinterpret_cast<const float4*>(wpost);
    const float4* wn4 = reinterpret_cast<const float4*>(wnext);
    float4 xv[NV], yv[NV], wpv[NV], wnv[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int q = min(tid + NT * i, d4 - 1);  // clamped: unconditional loads
        xv[i] = x4[q];
        wnv[i] = wn4[q];
        if (y) yv[i] = y4[q];
        if (y && wpost) wpv[i] = wp4[q];
    }
    auto valid = [&](int i) { return tid + NT * i < d4; };
    auto mul = [](float4 a, float4 b) { return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w); };
    auto scl = [](float4 a, float s) { return make_float4(a.x * s, a.y * s, a.z * s, a.w * s); };
    auto add = [](float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); };
    // inv = 1 / sqrt(the fold of v*v / d + eps) of the row held in v
    auto inv_of = [&](const float4 (&v)[NV]) {
#pragma unroll
        for (int i = 0; i < NV; ++i)
            if (valid(i)) sq4[tid + NT * i] = mul(v[i], v[i]);
        __syncthreads();
        const float ms = seq_sum_spec<NT>(sq, d, -0.0f, fsc) / (float)d;
        return 1.0f / sqrtf(ms + eps);
    };
    float4 nv[NV];
    if (y && wpost) {  // gemma: x += norm(y, wpost)
        const float iy = inv_of(yv);
#pragma unroll
        for (int i = 0; i < NV; ++i) nv[i] = add(xv[i], mul(scl(yv[i], iy), wpv[i]));
    } else if (y) {  // rope.rs: x = x + y
#pragma unroll
        for (int i = 0; i < NV; ++i) nv[i] = add(xv[i], yv[i]);
    } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) nv[i] = xv[i];
    }
    if (y) {
#pragma unroll
        for (int i = 0; i < NV; ++i)
            if (valid(i)) reinterpret_cast<float4*>(x + r)[tid + NT * i] = nv[i];
    }
    const float inv = inv_of(nv);
#pragma unroll
    for (int i = 0; i < NV; ++i)
        if (valid(i)) {
            const float4 o = mul(scl(nv[i], inv), wnv[i]);
            reinterpret_cast<float4*>(out + r)[tid + NT * i] = o;
            if (a4) reinterpret_cast<float4*>(a4)[(size_t)(tid + NT * i) * 16 + row0 + blockIdx.x] = o;
        }
}

// ---- the int8 down linear's activation quant, fused into the activation
// kernel (act(gate) * up), so the down linear streams its weights with no
// quant of its own (frq_mm_i8_q_dev).  The quant is quant_core.h's, by 16
// waves: the same bytes as the standalone quant and the fused M == 1
// linear.  (The rows feeding q|k|v and gate|up keep the fused M == 1
// linear, whose per-workgroup quant overlaps its first weight loads:
// measured faster than quantising in the norm kernel.)
constexpr int QNT = 1024;
constexpr int FRQ_QMAXK = 4 * QNT * 5;  // K of the fused quant (NV4 <= 5)

struct Q8 {  // one quantised activation row as frq_mm_i8_q_dev takes it
    int8_t* a8;    // kp bytes, channels past K zero
    float* sa;
    uint32_t* oi;  // the 32 outliers, ascending channel
    float* ov;
    int kp;
};

// The row (K floats of LDS, 16-byte aligned, K % 4 == 0, 32 < K <= 4096 NV4,
// also held in v: v[i] = float4 tid + QNT i, entries past K / 4 ignored)
// quantised into q by the QNT threads; a NaN row sets *err and writes the
// standalone quant's placeholders.
template <int NV4>
__device__ void quant_lds_row(const float* row, int K, const Q8& q, int* err, const float4 (&v)[NV4]) {
    __shared__ qc::RowLdsT<QNT> L;
    __shared__ unsigned long long cand[qc::FCAP];
    __shared__ uint32_t bitmap[FRQ_QMAXK / 32];
    const int tid = threadIdx.x, K4 = K >> 2;
    const qc::RowSel sel = qc::row_select<NV4, QNT>(row, K, v, L, cand, bitmap, (q.kp + 31) / 32);
    uint32_t* a8w = reinterpret_cast<uint32_t*>(q.a8);
    if (sel.nan) {  // the reference panics here; the call reports FRQ_ERR_NAN
        if (tid == 0) atomicOr(err, 1);
        for (int i4 = tid; i4 < K4; i4 += QNT) a8w[i4] = 0u;
    } else {
        qc::row_quantize<NV4, QNT>(v, K4, bitmap, sel.sa, sel.fast, [&](int i4, uint32_t w) { a8w[i4] = w; });
    }
    for (int i4 = K4 + tid; i4 < q.kp / 4; i4 += QNT) a8w[i4] = 0u;
    if (tid < FRQ_T) {
        q.oi[tid] = L.sel_i[tid];
        q.ov[tid] = L.sel_v[tid];
    }
    if (tid == 0) *q.sa = sel.sa;
}

// The down linear's input for one decode row, act(gate) * up as
// gm_geglu_kernel computes it (also written to hm), quantised.
template <int NV4>
__global__ __launch_bounds__(QNT) void gm_act_quant_kernel(const float* __restrict__ gu, int ffn, float c,
                                                           float* __restrict__ hm, int silu, Q8 q,
                                                           int* __restrict__ err) {
    extern __shared__ float4 lds4[];
    const int tid = threadIdx.x, f4 = ffn >> 2;
    const float4* g4 = reinterpret_cast<const float4*>(gu);
    const float4* u4 = reinterpret_cast<const float4*>(gu + ffn);
    // every load issued before the first use (clamped: unconditional)
    float4 gv[NV4], uv[NV4];
#pragma unroll
    for (int j = 0; j < NV4; ++j) {
        const int q4 = min(tid + QNT * j, f4 - 1);
        gv[j] = g4[q4];
        uv[j] = u4[q4];
    }
    auto act = [&](float xv) {
        return silu ? xv / (1.0f + libm::frq_expf(-xv))
                    : 0.5f * xv * (1.0f + libm::frq_tanhf(c * (xv + 0.044715f * xv * xv * xv)));
    };
    float4 v[NV4];
#pragma unroll
    for (int j = 0; j < NV4; ++j) {
        v[j] = make_float4(act(gv[j].x) * uv[j].x, act(gv[j].y) * uv[j].y, act(gv[j].z) * uv[j].z,
                           act(gv[j].w) * uv[j].w);
        const int q4 = tid + QNT * j;
        if (q4 < f4) {
            lds4[q4] = v[j];
            reinterpret_cast<float4*>(hm)[q4] = v[j];
        }
    }
    __syncthreads();
    quant_lds_row<NV4>(reinterpret_cast<const float*>(lds4), ffn, q, err, v);
}

// Checking hook of seq_sum_spec: out[r] = init + x[r][0] + ... + x[r][n-1],
// the sequential f32 fold, one workgroup per row (the norm kernel's shape).
__global__ __launch_bounds__(NORM_NT) void seq_fold_kernel(const float* __restrict__ x, int n, float init,
                                                           float* __restrict__ out) {
    extern __shared__ float4 lds4[];
    float* v = reinterpret_cast<float*>(lds4);
    float* fsc = v + ((n + 3) & ~3);
    for (int c = threadIdx.x; c < n; c += NORM_NT) v[c] = x[(size_t)blockIdx.x * n + c];
    __syncthreads();
    const float r = seq_sum_spec<NORM_NT>(v, n, init, fsc);
    if (threadIdx.x == 0) out[blockIdx.x] = r;
}

// rope (gemma.rs:79-94) on one head of hd values at absolute position pos,
// in place: (a, b) = (x[j], x[j + half]) -> (a c - b s, b c + a s) with the
// host-computed cos / sin of pos * inv[j].
__device__ __forceinline__ void rope_pair(float* xh, int j, int half, const float2* __restrict__ cs) {
    const float2 t = cs[j];
    const float a = xh[j], b = xh[j + half];
    xh[j] = a * t.x - b * t.y;
    xh[j + half] = b * t.x + a * t.y;
}

// The int8 cache quantiser of forward_block_q (314-324): sc = (max|v| /
// 127).max(1e-8), q = clamp(round(v / sc)) (NaN -> 0), by one wave.
__device__ void kv_quant_wave(const float* src, int hd, int8_t* dq, float* sdst) {
    const int lane = threadIdx.x & 63;
    float mx = 0.0f;
    for (int c = lane; c < hd; c += 64) mx = fmaxf(mx, fabsf(src[c]));
    mx = gwave_max(mx);
    const float sc = fmaxf(mx / 127.0f, 1e-8f);
    for (int c = lane; c < hd; c += 64) {
        const float r = roundf(src[c] / sc);
        dq[c] = r != r ? (int8_t)0 : (int8_t)fminf(fmaxf(r, -127.0f), 127.0f);
    }
    if (lane == 0) *sdst = sc;
}

// Rope::head_norm (rope.rs:72-87) on one head of hd values in place, by the
// calling lane: ms = the fold from -0.0 of v*v / hd, v * inv * w.
__device__ void head_norm_lane(float* v, int hd, const float* __restrict__ w, float eps) {
    float ms = -0.0f;
    for (int c = 0; c < hd; ++c) ms = ms + v[c] * v[c];
    ms = ms / (float)hd;
    const float inv = 1.0f / sqrtf(ms + eps);
    for (int c = 0; c < hd; ++c) v[c] = v[c] * inv * w[c];
}

// Prefill: rope the q and k heads of row i in the qkv buffer and append k,
// v to cache row cur + i.  qkv row: [q (H hd) | k (KV hd) | v (KV hd)].
template <bool KV8>
__global__ __launch_bounds__(GT) void gm_qkv_kernel(float* __restrict__ qkv, int H, int KV, int hd,
                                                    const int* __restrict__ curp, const float2* __restrict__ cs,
                                                    float* __restrict__ kc, float* __restrict__ vc,
                                                    int8_t* __restrict__ kq, int8_t* __restrict__ vq,
                                                    float* __restrict__ ks, float* __restrict__ vs,
                                                    const float* __restrict__ bias, const float* __restrict__ qn,
                                                    const float* __restrict__ kn, float eps) {
    const int i = blockIdx.x, half = hd / 2, kvd = KV * hd;
    const size_t pos = (size_t)(*curp + i);
    float* row = qkv + (size_t)i * (H + 2 * KV) * hd;
    const float2* csp = cs + pos * half;
    if (bias) {  // proj: y + bias (rope.rs:110-117)
        for (int c = threadIdx.x; c < (H + 2 * KV) * hd; c += GT) row[c] = row[c] + bias[c];
        __syncthreads();
    }
    if (qn) {  // the QK-norm, a lane per head
        for (int t = threadIdx.x; t < H + KV; t += GT) head_norm_lane(row + t * hd, hd, t < H ? qn : kn, eps);
        __syncthreads();
    }
    for (int t = threadIdx.x; t < (H + KV) * half; t += GT) rope_pair(row + (t / half) * hd, t % half, half, csp);
    __syncthreads();
    if constexpr (!KV8) {
        for (int c = threadIdx.x; c < kvd; c += GT) {
            kc[pos * kvd + c] = row[H * hd + c];
            vc[pos * kvd + c] = row[(H + KV) * hd + c];
        }
    } else {
        const int wave = threadIdx.x >> 6;
        for (int u = wave; u < 2 * KV; u += GT / 64) {
            const int kind = u >= KV, kh = kind ? u - KV : u;
            kv_quant_wave(row + (H + kind * KV + kh) * hd, hd, (kind ? vq : kq) + pos * kvd + (size_t)kh * hd,
                          (kind ? vs : ks) + pos * KV + kh);
        }
    }
}

// Attention of row i (position cur + i), query head h over kv head h / rep
// (forward_block 252-277): s_j = (q . k_j) * qscale as a sequential FMA
// chain, attn_cap * tanh(s / attn_cap), keys past the position or (even
// layers) window or more behind it masked at -1e30 (their exps are 0, the
// mask joins the max), softmax (expf, key-order sum, divide), then the
// value chain.  FUSED (decode): the block ropes its q head and its kv
// head's k from the qkv row and appends k, v to the cache first (blocks of
// one kv group write the same bytes).  LDS: q (hd), k / v staging (2 hd),
// p and the int8 value scales (pstride each).
template <bool KV8, bool FUSED>
__global__ __launch_bounds__(GT) void gm_attn_kernel(const float* __restrict__ qkv, int H, int KV, int hd,
                                                     const int* __restrict__ curp, const float2* __restrict__ cs,
                                                     float* __restrict__ kc, float* __restrict__ vc,
                                                     int8_t* __restrict__ kq, int8_t* __restrict__ vq,
                                                     float* __restrict__ ks, float* __restrict__ vs, float qscale,
                                                     float cap, int sliding, int window, int pstride,
                                                     float* __restrict__ att, int div,
                                                     const float* __restrict__ bias, const float* __restrict__ qn,
                                                     const float* __restrict__ kn, float eps, long long bst = 0,
                                                     float* __restrict__ a4 = nullptr) {
    extern __shared__ float4 lds4[];
    float* q = reinterpret_cast<float*>(lds4);
    float* kvs = q + ((hd + 3) & ~3);
    float* p = kvs + 2 * ((hd + 3) & ~3);
    float* sv = p + pstride;
    __shared__ float red[4];
    const int h = blockIdx.x, i = blockIdx.y, rep = H / KV, kv = h / rep, half = hd / 2, kvd = KV * hd;
    // bst > 0: a batch step, row i is sequence i's decode row (its own cache,
    // bst elements further for each row; every sequence at position cur)
    const int cur = *curp, ab = bst ? cur : cur + i, klen = bst ? cur + 1 : cur + (int)gridDim.y;
    if (bst) {
        const size_t o = (size_t)i * (size_t)bst, os = o / (size_t)hd;
        if (kc) { kc += o; vc += o; }
        if (kq) { kq += o; vq += o; ks += os; vs += os; }
    }
    const float* row = qkv + (size_t)i * (H + 2 * KV) * hd;
    if constexpr (FUSED) {
        const size_t pos = (size_t)ab;
        for (int c = threadIdx.x; c < hd; c += GT) {
            float qv = row[h * hd + c], kv_ = row[(H + kv) * hd + c], vv = row[(H + KV + kv) * hd + c];
            if (bias) {  // proj: y + bias (rope.rs:110-117)
                qv = qv + bias[h * hd + c];
                kv_ = kv_ + bias[(H + kv) * hd + c];
                vv = vv + bias[(H + KV + kv) * hd + c];
            }
            q[c] = qv;
            kvs[c] = kv_;
            kvs[((hd + 3) & ~3) + c] = vv;
        }
        __syncthreads();
        if (qn) {  // the QK-norm of this q head and kv head (two lanes)
            if (threadIdx.x == 0) head_norm_lane(q, hd, qn, eps);
            if (threadIdx.x == 64) head_norm_lane(kvs, hd, kn, eps);
            __syncthreads();
        }
        const float2* csp = cs + pos * half;
        for (int t = threadIdx.x; t < 2 * half; t += GT) rope_pair(t < half ? q : kvs, t % half, half, csp);
        __syncthreads();
        const float* vsrc = kvs + ((hd + 3) & ~3);
        if constexpr (!KV8) {
            for (int c = threadIdx.x; c < hd; c += GT) {
                kc[pos * kvd + (size_t)kv * hd + c] = kvs[c];
                vc[pos * kvd + (size_t)kv * hd + c] = vsrc[c];
            }
        } else {
            const int wave = threadIdx.x >> 6;
            if (wave < 2)
                kv_quant_wave(wave ? vsrc : kvs, hd, (wave ? vq : kq) + pos * kvd + (size_t)kv * hd,
                              (wave ? vs : ks) + pos * KV + kv);
        }
    } else {
        for (int c = threadIdx.x; c < hd; c += GT) q[c] = row[h * hd + c];
    }
    __syncthreads();
    const int j0 = (sliding && ab >= window) ? ab - window + 1 : 0;
    const int nk = ab + 1;
    float mx = -INFINITY;
    for (int j = j0 + threadIdx.x; j < nk; j += GT) {
        float acc = 0.0f;
        if constexpr (!KV8) {
            const float* kr = kc + (size_t)j * kvd + (size_t)kv * hd;
            for (int c = 0; c < hd; c += 4) {
                const float4 k4 = *reinterpret_cast<const float4*>(kr + c);
                acc = __builtin_fmaf(q[c], k4.x, acc);
                acc = __builtin_fmaf(q[c + 1], k4.y, acc);
                acc = __builtin_fmaf(q[c + 2], k4.z, acc);
                acc = __builtin_fmaf(q[c + 3], k4.w, acc);
            }
        } else {
            const int8_t* kr = kq + (size_t)j * kvd + (size_t)kv * hd;
            const float sk = ks[(size_t)j * KV + kv];
            sv[j] = vs[(size_t)j * KV + kv];
            for (int c = 0; c < hd; c += 4) {
                const char4 k4 = *reinterpret_cast<const char4*>(kr + c);
                acc = __builtin_fmaf(q[c], (float)k4.x * sk, acc);
                acc = __builtin_fmaf(q[c + 1], (float)k4.y * sk, acc);
                acc = __builtin_fmaf(q[c + 2], (float)k4.z * sk, acc);
                acc = __builtin_fmaf(q[c + 3], (float)k4.w * sk, acc);
            }
        }
        float sj = div ? acc / qscale : acc * qscale;  // rope.rs: / sqrt(hd); gemma.rs: * qscalar^-0.5
        if (cap > 0.0f) sj = cap * libm::frq_tanhf(sj / cap);
        p[j] = sj;
        mx = fmaxf(mx, sj);
    }
    mx = gblock_max(mx, red);
    if (j0 > 0 || nk < klen) mx = fmaxf(mx, -1e30f);  // a masked entry joins the max
    for (int j = j0 + threadIdx.x; j < nk; j += GT) p[j] = libm::frq_expf(p[j] - mx);
    __syncthreads();
    // the sum in key order (the masked exps are +0: j < j0 add nothing to
    // +0): the keys before the next 16-byte boundary in every thread, the
    // rest by the whole workgroup's speculative segmented fold
    const int ja = min((j0 + 3) & ~3, nk);
    float head = 0.0f;
    for (int j = j0; j < ja; ++j) head = head + p[j];
    const float sum = seq_sum_spec<GT>(p + ja, nk - ja, head, sv + pstride);
    for (int j = j0 + threadIdx.x; j < nk; j += GT) p[j] = p[j] / sum;
    __syncthreads();
    constexpr int B = 16;
    for (int c = threadIdx.x; c < hd; c += GT) {
        const size_t col = (size_t)kv * hd + c;
        // one a.dot block of keys [s, e): the chain from +0, its value loads
        // a 16-key batch ahead
        auto chain = [&](int s, int e) {
            float acc = 0.0f;
            const int nb = (e - s) / B;
            float v0[B], v1[B];
            auto ld = [&](float (&v)[B], int k) {
#pragma unroll
                for (int u = 0; u < B; ++u) {
                    const size_t j = (size_t)(s + k * B + u);
                    if constexpr (!KV8) v[u] = vc[j * kvd + col];
                    else v[u] = (float)vq[j * kvd + col] * sv[j];
                }
            };
            auto fma_b = [&](const float (&v)[B], int k) {
#pragma unroll
                for (int u = 0; u < B; ++u) acc = __builtin_fmaf(p[s + k * B + u], v[u], acc);
            };
            if (nb > 0) {  // both batches of a trip consumed unconditionally, loads pinned a batch ahead
                ld(v0, 0);
                ld(v1, min(1, nb - 1));
                __builtin_amdgcn_sched_barrier(0);
                int k = 0;
                for (; k + 2 <= nb; k += 2) {
                    fma_b(v0, k);
                    ld(v0, min(k + 2, nb - 1));
                    __builtin_amdgcn_sched_barrier(0);
                    fma_b(v1, k + 1);
                    ld(v1, min(k + 3, nb - 1));
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (k < nb) fma_b(v0, k);
            }
            for (int j = s + nb * B; j < e; ++j) {
                const float v = KV8 ? (float)vq[(size_t)j * kvd + col] * sv[j] : vc[(size_t)j * kvd + col];
                acc = __builtin_fmaf(p[j], v, acc);
            }
            return acc;
        };
        const float o = mm_blocks(j0, nk, chain);
        att[(size_t)i * H * hd + (size_t)h * hd + c] = o;
        if (a4) {
            const size_t k = (size_t)h * hd + c;
            a4[(k >> 2) * 64 + 4 * i + (k & 3)] = o;
        }
    }
}

// ---- multi-row attention, one workgroup per (kv head, query row) ----
// The R = H / KV query heads that share a kv head read the same key and
// value rows, so one workgroup takes all R for its query row: each key row
// is loaded once for R score chains, each value element once for up to RC
// (head, dim) chains.  The arithmetic per output is gm_attn_kernel<.., false>'s
// (score = FMA chain over the head dims, softmax max / exp / key-order sum /
// divide, values in a.dot's blocked key order), so the bits are the same.
// Needs GT % hd == 0 and R <= RC * (GT / hd).
template <bool KV8>
__global__ __launch_bounds__(GT) void gm_attn_group_kernel(const float* __restrict__ qkv, int H, int KV, int hd,
                                                           const int* __restrict__ curp,
                                                           const float* __restrict__ kc, const float* __restrict__ vc,
                                                           const int8_t* __restrict__ kq, const int8_t* __restrict__ vq,
                                                           const float* __restrict__ ks, const float* __restrict__ vs,
                                                           float qscale, float cap, int sliding, int window,
                                                           int pstride, float* __restrict__ att, int div) {
    constexpr int RMAX = 16, RC = 4;
    extern __shared__ float4 lds4[];
    const int R = H / KV, hd4 = (hd + 3) & ~3, kvd = KV * hd;
    float* q = reinterpret_cast<float*>(lds4);  // R rows of hd4
    float* p = q + R * hd4;                     // R rows of pstride
    float* sv = p + (size_t)R * pstride;
    __shared__ float red[RMAX][GT / 64];
    const int kv = blockIdx.x, i = blockIdx.y;
    const int cur = *curp, ab = cur + i, klen = cur + (int)gridDim.y;
    const float* row = qkv + (size_t)i * (H + 2 * KV) * hd;
    for (int t = threadIdx.x; t < R * hd; t += GT) q[(t / hd) * hd4 + t % hd] = row[(kv * R + t / hd) * hd + t % hd];
    __syncthreads();
    const int j0 = (sliding && ab >= window) ? ab - window + 1 : 0;
    const int nk = ab + 1;
    float mx[RMAX];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) mx[r] = -INFINITY;
    for (int j = j0 + threadIdx.x; j < nk; j += GT) {
        float acc[RMAX];
#pragma unroll
        for (int r = 0; r < RMAX; ++r) acc[r] = 0.0f;
        if constexpr (!KV8) {
            const float* kr = kc + (size_t)j * kvd + (size_t)kv * hd;
            for (int c = 0; c < hd; c += 4) {
                const float4 k4 = *reinterpret_cast<const float4*>(kr + c);
#pragma unroll
                for (int r = 0; r < RMAX; ++r) {
                    if (r < R) {
                        const float* qr = q + r * hd4;
                        acc[r] = __builtin_fmaf(qr[c], k4.x, acc[r]);
                        acc[r] = __builtin_fmaf(qr[c + 1], k4.y, acc[r]);
                        acc[r] = __builtin_fmaf(qr[c + 2], k4.z, acc[r]);
                        acc[r] = __builtin_fmaf(qr[c + 3], k4.w, acc[r]);
                    }
                }
            }
        } else {
            const int8_t* kr = kq + (size_t)j * kvd + (size_t)kv * hd;
            const float sk = ks[(size_t)j * KV + kv];
            sv[j] = vs[(size_t)j * KV + kv];
            for (int c = 0; c < hd; c += 4) {
                const char4 k4 = *reinterpret_cast<const char4*>(kr + c);
                const float k0 = (float)k4.x * sk, k1 = (float)k4.y * sk, k2 = (float)k4.z * sk,
                            k3 = (float)k4.w * sk;
#pragma unroll
                for (int r = 0; r < RMAX; ++r) {
                    if (r < R) {
                        const float* qr = q + r * hd4;
                        acc[r] = __builtin_fmaf(qr[c], k0, acc[r]);
                        acc[r] = __builtin_fmaf(qr[c + 1], k1, acc[r]);
                        acc[r] = __builtin_fmaf(qr[c + 2], k2, acc[r]);
                        acc[r] = __builtin_fmaf(qr[c + 3], k3, acc[r]);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            if (r < R) {
                float sj = div ? acc[r] / qscale : acc[r] * qscale;
                if (cap > 0.0f) sj = cap * libm::frq_tanhf(sj / cap);
                p[(size_t)r * pstride + j] = sj;
                mx[r] = fmaxf(mx[r], sj);
            }
        }
    }
    // block max per head (max is exact in any order)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
        if (r < R) {
            float v = mx[r];
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
            if (lane == 0) red[r][wave] = v;
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
        if (r < R) {
            float v = red[r][0];
#pragma unroll
            for (int w = 1; w < GT / 64; ++w) v = fmaxf(v, red[r][w]);
            if (j0 > 0 || nk < klen) v = fmaxf(v, -1e30f);  // a masked entry joins the max
            mx[r] = v;
        }
    }
    __syncthreads();  // red is reused for the sums
    for (int j = j0 + threadIdx.x; j < nk; j += GT) {
#pragma unroll
        for (int r = 0; r < RMAX; ++r)
            if (r < R) p[(size_t)r * pstride + j] = libm::frq_expf(p[(size_t)r * pstride + j] - mx[r]);
    }
    __syncthreads();
    if (threadIdx.x < R) {  // one lane per head, in key order; the lanes run in step
        const float* pr = p + (size_t)threadIdx.x * pstride;
        const int ja = min((j0 + 3) & ~3, nk);
        float sum = 0.0f;
        for (int j = j0; j < ja; ++j) sum = sum + pr[j];
        red[threadIdx.x][0] = lds_seq_sum(pr + ja, nk - ja, sum);
    }
    __syncthreads();
    for (int j = j0 + threadIdx.x; j < nk; j += GT) {
#pragma unroll
        for (int r = 0; r < RMAX; ++r)
            if (r < R) p[(size_t)r * pstride + j] = p[(size_t)r * pstride + j] / red[r][0];
    }
    __syncthreads();
    // value chains: thread t takes dim c = t % hd of heads t / hd, t / hd + GT / hd, ...
    const int c = threadIdx.x % hd, r0 = threadIdx.x / hd, rs = GT / hd;
    const size_t col = (size_t)kv * hd + c;
    float tot[RC], acc[RC];
#pragma unroll
    for (int u = 0; u < RC; ++u) tot[u] = 0.0f;
    constexpr int B = 16;
    float v0[B], v1[B];
    // a.dot's order: the keys in blocks of MM_KC at absolute multiples, each
    // block's chains from +0 (value loads a 16-key batch ahead), then added
    for (int s = j0; s < nk && r0 < R;) {
        const int e = min(nk, (s / MM_KC + 1) * MM_KC), nb = (e - s) / B;
#pragma unroll
        for (int u = 0; u < RC; ++u) acc[u] = 0.0f;
        auto ld = [&](float (&v)[B], int k) {
#pragma unroll
            for (int u = 0; u < B; ++u) {
                const size_t j = (size_t)(s + k * B + u);
                if constexpr (!KV8) v[u] = vc[j * kvd + col];
                else v[u] = (float)vq[j * kvd + col] * sv[j];
            }
        };
        auto fma_b = [&](const float (&v)[B], int k) {
#pragma unroll
            for (int w = 0; w < RC; ++w) {
                const int r = r0 + w * rs;
                if (r < R) {
                    const float* pr = p + (size_t)r * pstride + s + k * B;
#pragma unroll
                    for (int u = 0; u < B; ++u) acc[w] = __builtin_fmaf(pr[u], v[u], acc[w]);
                }
            }
        };
        if (nb > 0) {  // both batches of a trip consumed unconditionally, loads pinned a batch ahead
            ld(v0, 0);
            ld(v1, min(1, nb - 1));
            __builtin_amdgcn_sched_barrier(0);
            int k = 0;
            for (; k + 2 <= nb; k += 2) {
                fma_b(v0, k);
                ld(v0, min(k + 2, nb - 1));
                __builtin_amdgcn_sched_barrier(0);
                fma_b(v1, k + 1);
                ld(v1, min(k + 3, nb - 1));
                __builtin_amdgcn_sched_barrier(0);
            }
            if (k < nb) fma_b(v0, k);
        }
        for (int j = s + nb * B; j < e; ++j) {
            const float v = KV8 ? (float)vq[(size_t)j * kvd + col] * sv[j] : vc[(size_t)j * kvd + col];
#pragma unroll
            for (int w = 0; w < RC; ++w) {
                const int r = r0 + w * rs;
                if (r < R) acc[w] = __builtin_fmaf(p[(size_t)r * pstride + j], v, acc[w]);
            }
        }
#pragma unroll
        for (int u = 0; u < RC; ++u) tot[u] = tot[u] + acc[u];
        s = e;
    }
    if (r0 < R) {
#pragma unroll
        for (int w = 0; w < RC; ++w) {
            const int r = r0 + w * rs;
            if (r < R) att[(size_t)i * H * hd + (size_t)(kv * R + r) * hd + c] = tot[w];
        }
    }
}

// ---- multi-row attention over an f32 cache, register-tiled ----
// gm_attn_group_kernel<false>'s arithmetic per output (score = FMA chain
// over the head dims, max, exp, the key-order sum, divide, values in a.dot's
// blocked key order), so the same bits, laid out for throughput:
// - scores: a lane takes two adjacent keys for every head of the group
//   (RP >= R; heads past R are computed on other q values and never
//   leave the kernel), so each q value feeds two chains and each key value
//   RP chains; q is wave-uniform and comes through scalar loads (SGPR
//   operands), the key rows straight from memory a 32-dim block (one
//   128-byte line a key) at a time, the next block in flight;
// - p holds RP rows (rows past R never leave the kernel) so the exps,
//   divides and stores run RP at a time without per-head tests (the exps
//   branch-free, their table loads all in flight); its rows are prow apart
//   with prow % 64 == 4 so the sum lanes' reads spread over the banks;
// - values: a lane takes 2 dims of 4 heads (hd / 2 lanes a head group),
//   so a value load feeds 4 heads' chains; the value loads run three 4-key
//   batches ahead.
// Needs hd % 32 == 0, hd <= 2 GT and R <= RP <= R + 2 KV (the q reads of
// heads past R stay inside the qkv row).
template <int RP>
__global__ __launch_bounds__(GT) void gm_attn_tile_kernel(const float* __restrict__ qkv, int H, int KV, int hd,
                                                          const int* __restrict__ curp,
                                                          const float* __restrict__ kc, const float* __restrict__ vc,
                                                          float qscale, float cap, int sliding, int window, int prow,
                                                          float* __restrict__ att, int div) {
    extern __shared__ float4 lds4[];
    const int R = H / KV, kvd = KV * hd;
    float* p = reinterpret_cast<float*>(lds4);  // [RP][prow]
    __shared__ float red[RP][GT / 64];
    __shared__ float sums[RP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kv = blockIdx.x, i = blockIdx.y;
    const int cur = *curp, ab = cur + i, klen = cur + (int)gridDim.y;
    const float* row = qkv + (size_t)i * (H + 2 * KV) * hd;
    const int j0 = (sliding && ab >= window) ? ab - window + 1 : 0;
    const int nk = ab + 1;
    float mx[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) mx[r] = -INFINITY;
    const int nblk = hd >> 5;
    const float* qrow = row + (size_t)kv * R * hd;  // uniform: scalar loads
    for (int pb = j0; pb < nk; pb += 2 * GT) {
        const int ja = pb + 2 * tid;
        const float* kra = kc + (size_t)min(ja, nk - 1) * kvd + (size_t)kv * hd;
        const float* krb = kc + (size_t)min(ja + 1, nk - 1) * kvd + (size_t)kv * hd;
        float acc[2][RP];
#pragma unroll
        for (int r = 0; r < RP; ++r) acc[0][r] = acc[1][r] = 0.0f;
        float4 ka[2][8], kb[2][8];
        auto ld = [&](int buf, int b) __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                ka[buf][u] = *reinterpret_cast<const float4*>(kra + 32 * b + 4 * u);
                kb[buf][u] = *reinterpret_cast<const float4*>(krb + 32 * b + 4 * u);
            }
        };
        auto fm = [&](int buf, int b) __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
#pragma unroll
                for (int r = 0; r < RP; ++r) {
                    const float4 q4 = *reinterpret_cast<const float4*>(qrow + r * hd + 32 * b + 4 * u);
                    acc[0][r] = __builtin_fmaf(q4.x, ka[buf][u].x, acc[0][r]);
                    acc[0][r] = __builtin_fmaf(q4.y, ka[buf][u].y, acc[0][r]);
                    acc[0][r] = __builtin_fmaf(q4.z, ka[buf][u].z, acc[0][r]);
                    acc[0][r] = __builtin_fmaf(q4.w, ka[buf][u].w, acc[0][r]);
                    acc[1][r] = __builtin_fmaf(q4.x, kb[buf][u].x, acc[1][r]);
                    acc[1][r] = __builtin_fmaf(q4.y, kb[buf][u].y, acc[1][r]);
                    acc[1][r] = __builtin_fmaf(q4.z, kb[buf][u].z, acc[1][r]);
                    acc[1][r] = __builtin_fmaf(q4.w, kb[buf][u].w, acc[1][r]);
                }
            }
        };
        ld(0, 0);
        for (int b = 0; b < nblk; b += 2) {
            ld(1, min(b + 1, nblk - 1));
            __builtin_amdgcn_sched_barrier(0);
            fm(0, b);
            ld(0, min(b + 2, nblk - 1));
            __builtin_amdgcn_sched_barrier(0);
            if (b + 1 < nblk) fm(1, b + 1);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int j = ja + u;
            if (j < nk) {
#pragma unroll
                for (int r = 0; r < RP; ++r) {
                    float sj = div ? acc[u][r] / qscale : acc[u][r] * qscale;
                    if (cap > 0.0f) sj = cap * libm::frq_tanhf(sj / cap);
                    p[(size_t)r * prow + j] = sj;
                    mx[r] = fmaxf(mx[r], sj);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RP; ++r) {
        float v = mx[r];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
        if (lane == 0) red[r][wave] = v;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RP; ++r) {
        float v = red[r][0];
#pragma unroll
        for (int w = 1; w < GT / 64; ++w) v = fmaxf(v, red[r][w]);
        if (j0 > 0 || nk < klen) v = fmaxf(v, -1e30f);  // a masked entry joins the max
        mx[r] = v;
    }
    for (int j = j0 + tid; j < nk; j += GT) {
        float e[RP];
#pragma unroll
        for (int r = 0; r < RP; ++r) e[r] = p[(size_t)r * prow + j];
#pragma unroll
        for (int r = 0; r < RP; ++r) e[r] = libm::frq_expf_sel(e[r] - mx[r]);
#pragma unroll
        for (int r = 0; r < RP; ++r) p[(size_t)r * prow + j] = e[r];
    }
    __syncthreads();
    if (tid < RP) {  // one lane per head, in key order; the lanes run in step
        const float* pr = p + (size_t)tid * prow;
        const int ja = min((j0 + 3) & ~3, nk);
        float sum = 0.0f;
        for (int j = j0; j < ja; ++j) sum = sum + pr[j];
        sums[tid] = lds_seq_sum(pr + ja, nk - ja, sum);
    }
    __syncthreads();
    for (int j = j0 + tid; j < nk; j += GT) {
        float e[RP];
#pragma unroll
        for (int r = 0; r < RP; ++r) e[r] = p[(size_t)r * prow + j];
#pragma unroll
        for (int r = 0; r < RP; ++r) p[(size_t)r * prow + j] = e[r] / sums[r];
    }
    __syncthreads();
    // values: lane (dims 2dg, 2dg + 1 of heads r4 .. r4 + 3); a.dot's order:
    // blocks of MM_KC keys at absolute multiples, each chained from +0, added
    const int DG = hd >> 1, HG = GT / DG;  // lanes a head group, head groups a pass
    for (int g0 = 0; 4 * g0 < R; g0 += HG) {
        const int r4 = 4 * (g0 + tid / DG), dg = tid % DG;
        if (r4 < R) {
            const float* pr = p + (size_t)r4 * prow;
            const float* vb = vc + (size_t)kv * hd + 2 * dg;
            float2 a[4], tot[4];
#pragma unroll
            for (int h = 0; h < 4; ++h) tot[h] = make_float2(0.0f, 0.0f);
          for (int s = j0; s < nk;) {
            const int e = min(nk, (s / MM_KC + 1) * MM_KC);
            const int ja = min((s + 3) & ~3, e);  // keys before ja one at a time, then 4-key batches
            const int nb = (e - ja) >> 2;
#pragma unroll
            for (int h = 0; h < 4; ++h) a[h] = make_float2(0.0f, 0.0f);
            auto step = [&](int h, float pj, float2 v) __attribute__((always_inline)) {
                a[h].x = __builtin_fmaf(pj, v.x, a[h].x);
                a[h].y = __builtin_fmaf(pj, v.y, a[h].y);
            };
            for (int j = s; j < ja; ++j) {
                const float2 v = *reinterpret_cast<const float2*>(vb + (size_t)j * kvd);
#pragma unroll
                for (int h = 0; h < 4; ++h) step(h, pr[(size_t)h * prow + j], v);
            }
            float2 vv[3][4];
            auto vld = [&](int buf, int k) __attribute__((always_inline)) {
                const int jb = ja + 4 * min(k, nb - 1);
#pragma unroll
                for (int u = 0; u < 4; ++u) vv[buf][u] = *reinterpret_cast<const float2*>(vb + (size_t)(jb + u) * kvd);
            };
            auto vfm = [&](int buf, int k) __attribute__((always_inline)) {
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const float4 p4 = *reinterpret_cast<const float4*>(pr + (size_t)h * prow + ja + 4 * k);
                    step(h, p4.x, vv[buf][0]);
                    step(h, p4.y, vv[buf][1]);
                    step(h, p4.z, vv[buf][2]);
                    step(h, p4.w, vv[buf][3]);
                }
            };
            if (nb > 0) {  // three batches in flight, each consumed unconditionally
                vld(0, 0);
                vld(1, 1);
                vld(2, 2);
                __builtin_amdgcn_sched_barrier(0);
                int k = 0;
                for (; k + 3 <= nb; k += 3) {
                    vfm(0, k);
                    vld(0, k + 3);
                    __builtin_amdgcn_sched_barrier(0);
                    vfm(1, k + 1);
                    vld(1, k + 4);
                    __builtin_amdgcn_sched_barrier(0);
                    vfm(2, k + 2);
                    vld(2, k + 5);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (k < nb) vfm(0, k);
                if (k + 1 < nb) vfm(1, k + 1);
            }
            for (int j = ja + 4 * nb; j < e; ++j) {
                const float2 v = *reinterpret_cast<const float2*>(vb + (size_t)j * kvd);
#pragma unroll
                for (int h = 0; h < 4; ++h) step(h, pr[(size_t)h * prow + j], v);
            }
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                tot[h].x = tot[h].x + a[h].x;
                tot[h].y = tot[h].y + a[h].y;
            }
            s = e;
          }
#pragma unroll
            for (int h = 0; h < 4; ++h)
                if (r4 + h < R)
                    *reinterpret_cast<float2*>(att + (size_t)i * H * hd + (size_t)(kv * R + r4 + h) * hd + 2 * dg) = tot[h];
        }
    }
}

// ---- prefill attention over an f32 cache in two tiled launches ----
// The per-output arithmetic of gm_attn_group_kernel<false> (score =
// FMA chain over the head dims, scale / cap, max over the row's keys, exp,
// the key-order sum from +0, p = e / sum, values in a.dot's blocked key
// order), so the same bits, with each key and value row read once
// per block of rows rather than once per row.  A block is AP (row, head)
// pairs: AP / RP consecutive rows times RP >= R heads of one kv head (pair
// p = row * RP + head; heads past R and rows past m are computed on zeros
// and never leave).  The scores go through a key-major buffer
// st[kv][block][key][pair] (kpad keys a block) that the second launch turns
// into exps in place.
constexpr int PF_AP = 64, PF_KT = 128, PF_VK = 64, PF_NT = 256;
static_assert(MM_KC % PF_VK == 0, "a value chunk lies in one a.dot block");
constexpr size_t PF_MIN_ROWS = 1024;  // shorter prompts take the one-launch kernels (more workgroups)
constexpr size_t PF_MAX_BYTES = (size_t)2 << 30;  // score buffer cap (570 MB at configs[4]'s 2048 + 128)
__host__ __device__ inline int pf_rows(int rp) { return PF_AP / rp; }

struct PfRow {
    int nk, j0, ok;  // keys [j0, nk) of the row; ok: a row of the launch
};
__device__ __forceinline__ PfRow pf_row(int i, int cur, int m, int sliding, int window) {
    const int ab = cur + i;
    return {ab + 1, (sliding && ab >= window) ? ab - window + 1 : 0, i < m};
}

// 1. scores: workgroup (kv, block b), heaviest blocks first; the block's q
// pairs in LDS, then its key tiles in order, each tile's 128 key rows in
// LDS (rows HD + 4 floats apart) while the next tile's rows load into
// registers; a lane 8 pairs x 4 keys (keys kg + 32u); writes the scaled
// (capped) scores and each pair's max over every tile key its row sees.
template <int RP, int RV, int HD>
__global__ __launch_bounds__(PF_NT) void gm_pf_scores_kernel(const float* __restrict__ qkv, int H, int KV,
                                                             const int* __restrict__ curp, int m,
                                                             const float* __restrict__ kc, float qscale, float cap,
                                                             int sliding, int window, int nrb, int nkt, int kpad,
                                                             float* __restrict__ st, float* __restrict__ pmax,
                                                             int div) {
    constexpr int RB = PF_AP / RP, HP = HD + 4, H4 = HD / 4;
    constexpr int QN = PF_AP * H4 / PF_NT, KN = PF_KT * H4 / PF_NT;  // float4 loads a thread
    static_assert(QN * PF_NT == PF_AP * H4 && KN * PF_NT == PF_KT * H4, "whole loads");
    extern __shared__ float4 lds4[];
    float* Qs = reinterpret_cast<float*>(lds4);  // [PF_AP][HP]
    float* Ks = Qs + PF_AP * HP;                  // [PF_KT][HP]
    const int R = H / KV, kvd = KV * HD, tid = threadIdx.x;
    const int bx = (int)(gridDim.x - 1 - blockIdx.x);  // the longest blocks start first
    const int b = bx % nrb, kv = bx / nrb;
    const int cur = *curp, r0 = b * RB, klen = cur + m;
    const int ntile = (cur + min(r0 + RB, m) + PF_KT - 1) / PF_KT;
    float4 qv[QN];
#pragma unroll
    for (int u = 0; u < QN; ++u) {
        const int x = tid + u * PF_NT, pq = x / H4, c4 = x % H4, h = pq % RP, i = r0 + pq / RP;
        qv[u] = (h < R && i < m)
                    ? *reinterpret_cast<const float4*>(qkv + (size_t)i * (H + 2 * KV) * HD + (size_t)(kv * R + h) * HD + 4 * c4)
                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    float4 kv4[KN];
    auto kload = [&](int c) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < KN; ++u) {
            const int x = tid + u * PF_NT, t = x / H4, c4 = x % H4, j = c * PF_KT + t;
            kv4[u] = j < klen ? *reinterpret_cast<const float4*>(kc + (size_t)j * kvd + (size_t)kv * HD + 4 * c4)
                              : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    kload(0);
#pragma unroll
    for (int u = 0; u < QN; ++u) {
        const int x = tid + u * PF_NT;
        *reinterpret_cast<float4*>(Qs + (x / H4) * HP + 4 * (x % H4)) = qv[u];
    }
    const int kg = tid & 31, pg = tid >> 5;
    float* sb = st + ((size_t)kv * nrb + b) * (size_t)kpad * PF_AP;
    // rows of this lane's pairs: keys [j0, nk) (nk 0 past m)
    int rj0[8], rnk[8];
#pragma unroll
    for (int a = 0; a < 8; ++a) {
        const PfRow rw = pf_row(r0 + (8 * pg + a) / RP, cur, m, sliding, window);
        rj0[a] = rw.j0;
        rnk[a] = rw.ok ? rw.nk : 0;
    }
    float mxl[8];
#pragma unroll
    for (int a = 0; a < 8; ++a) mxl[a] = -INFINITY;
    for (int c = 0; c < ntile; ++c) {
        __syncthreads();  // the previous tile is consumed
#pragma unroll
        for (int u = 0; u < KN; ++u) {
            const int x = tid + u * PF_NT;
            *reinterpret_cast<float4*>(Ks + (x / H4) * HP + 4 * (x % H4)) = kv4[u];
        }
        __syncthreads();
        if (c + 1 < ntile) kload(c + 1);  // in flight during this tile
        float acc[8][4];
#pragma unroll
        for (int a = 0; a < 8; ++a)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[a][u] = 0.0f;
        const float* qb = Qs + (8 * pg) * HP;
        const float* kb = Ks + kg * HP;
#pragma unroll 2
        for (int sd = 0; sd < H4; ++sd) {
            float4 q4[8], k4[4];
#pragma unroll
            for (int a = 0; a < 8; ++a)
                if (a % RP < RV) q4[a] = *reinterpret_cast<const float4*>(qb + a * HP + 4 * sd);
#pragma unroll
            for (int u = 0; u < 4; ++u) k4[u] = *reinterpret_cast<const float4*>(kb + 32 * u * HP + 4 * sd);
#pragma unroll
            for (int a = 0; a < 8; ++a)
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (a % RP >= RV) continue;  // a spare head: never leaves the kernel
                    acc[a][u] = __builtin_fmaf(q4[a].x, k4[u].x, acc[a][u]);
                    acc[a][u] = __builtin_fmaf(q4[a].y, k4[u].y, acc[a][u]);
                    acc[a][u] = __builtin_fmaf(q4[a].z, k4[u].z, acc[a][u]);
                    acc[a][u] = __builtin_fmaf(q4[a].w, k4[u].w, acc[a][u]);
                }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int j = c * PF_KT + kg + 32 * u;
            float sv[8];
#pragma unroll
            for (int a = 0; a < 8; ++a) {
                float sj = div ? acc[a][u] / qscale : acc[a][u] * qscale;
                if (cap > 0.0f) sj = cap * libm::frq_tanhf(sj / cap);
                sv[a] = sj;
                if (j >= rj0[a] && j < rnk[a]) mxl[a] = fmaxf(mxl[a], sj);
            }
            float4* dst = reinterpret_cast<float4*>(sb + (size_t)j * PF_AP + 8 * pg);
            dst[0] = make_float4(sv[0], sv[1], sv[2], sv[3]);
            dst[1] = make_float4(sv[4], sv[5], sv[6], sv[7]);
        }
    }
#pragma unroll
    for (int a = 0; a < 8; ++a) {
        float v = mxl[a];
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
        if (kg == 0) pmax[((size_t)kv * nrb + b) * PF_AP + 8 * pg + a] = v;
    }
}

// 2. workgroup (kv, block b), heaviest first: the pairs' maxes (one per
// pair from the first launch); per key tile the exps (branch-free) into LDS
// and, in place of the scores, into st, then wave 0 adds them in key order
// (a lane a pair); then the value chains, a lane 8 pairs x 4 dims, over
// 64-key chunks of p = e / sum and the value rows staged in LDS, the next
// chunk loading into registers meanwhile (chunks every row of the block
// sees entirely run without per-key tests).
template <int RP, int RV, int HD>
__global__ __launch_bounds__(PF_NT) void gm_pf_values_kernel(int H, int KV, const int* __restrict__ curp, int m,
                                                             const float* __restrict__ vc, int sliding, int window,
                                                             int nrb, int kpad, float* __restrict__ st,
                                                             const float* __restrict__ pmax,
                                                             float* __restrict__ att) {
    constexpr int RB = PF_AP / RP, HP = HD + 4, H4 = HD / 4;
    constexpr int PN = PF_VK * PF_AP / PF_NT, VN = (PF_VK * H4 + PF_NT - 1) / PF_NT;
    extern __shared__ float4 lds4[];
    __shared__ float mx[PF_AP], sums[PF_AP];
    const int R = H / KV, kvd = KV * HD, tid = threadIdx.x;
    const int bx = (int)(gridDim.x - 1 - blockIdx.x);
    const int b = bx % nrb, kv = bx / nrb;
    const int cur = *curp, r0 = b * RB, klen = cur + m;
    const int kend = cur + min(r0 + RB, m);  // keys [0, kend) cover every row of the block
    const int ntile = (kend + PF_KT - 1) / PF_KT;
    float* sb = st + ((size_t)kv * nrb + b) * (size_t)kpad * PF_AP;
    if (tid < PF_AP) {
        const PfRow rw = pf_row(r0 + tid / RP, cur, m, sliding, window);
        float v = pmax[((size_t)kv * nrb + b) * PF_AP + tid];
        if (rw.j0 > 0 || rw.nk < klen) v = fmaxf(v, -1e30f);  // a masked entry joins the max
        mx[tid] = v;
    }
    __syncthreads();
    float* Es = reinterpret_cast<float*>(lds4);  // [PF_KT][PF_AP]
    float sm = 0.0f;                              // wave 0: pair tid's sum
    const PfRow rs = pf_row(r0 + (tid & (PF_AP - 1)) / RP, cur, m, sliding, window);
    const int pq = tid & (PF_AP - 1);             // the pair of every element this thread touches
    const PfRow rq = rs;
    const float mxq = mx[pq];
    for (int c = 0; c < ntile; ++c) {
        const int jt = c * PF_KT;
        constexpr int EN = PF_KT * PF_AP / PF_NT;  // 32 exps a thread, loads first
        float e[EN];
#pragma unroll
        for (int u = 0; u < EN; ++u) e[u] = sb[(size_t)jt * PF_AP + tid + u * PF_NT];
#pragma unroll
        for (int u = 0; u < EN; ++u) {
            const int x = tid + u * PF_NT, j = jt + x / PF_AP;
            const float ev = libm::frq_expf_sel(e[u] - mxq);
            e[u] = (rq.ok && j >= rq.j0 && j < rq.nk) ? ev : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < EN; ++u) {
            Es[tid + u * PF_NT] = e[u];
            sb[(size_t)jt * PF_AP + tid + u * PF_NT] = e[u];
        }
        __syncthreads();
        if (tid < PF_AP && rs.ok) {
            // the tile's keys of this pair's row in order, reads 16 ahead
            const int ja = max(rs.j0, jt), jb = min(rs.nk, jt + PF_KT);
            const float* ep = Es + tid;
            int j = ja;
            for (; j + 16 <= jb; j += 16) {
                float ev[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) ev[u] = ep[(j - jt + u) * PF_AP];
#pragma unroll
                for (int u = 0; u < 16; ++u) sm = sm + ev[u];
            }
            for (; j < jb; ++j) sm = sm + ep[(j - jt) * PF_AP];
        }
        __syncthreads();
    }
    if (tid < PF_AP) sums[tid] = sm;
    __syncthreads();
    // values
    float* Ps = reinterpret_cast<float*>(lds4);  // [PF_VK][PF_AP]
    float* Vs = Ps + PF_VK * PF_AP;              // [PF_VK][HP]
    const int pg = tid >> 5, dg = tid & 31;
    const bool lane_on = dg < H4;
    int rj0[8], rnk[8];
#pragma unroll
    for (int a = 0; a < 8; ++a) {
        const PfRow rw = pf_row(r0 + (8 * pg + a) / RP, cur, m, sliding, window);
        rj0[a] = rw.j0;
        rnk[a] = rw.ok ? rw.nk : 0;
    }
    // keys every row of the block sees: [j0 of the last row, nk of the first)
    const PfRow rfirst = pf_row(r0, cur, m, sliding, window);
    const PfRow rlast = pf_row(min(r0 + RB, m) - 1, cur, m, sliding, window);
    const float rsum = sums[pq];
    // a.dot's order: each MM_KC-key block (chunks from 0, MM_KC a multiple
    // of PF_VK) chained from +0 in acc, the blocks added in order into tot
    float acc[8][4], tot[8][4];
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int d = 0; d < 4; ++d) acc[a][d] = tot[a][d] = 0.0f;
    const int nvc = (kend + PF_VK - 1) / PF_VK;
    float pn[PN];
    float4 vn[VN];
    auto cload = [&](int c) __attribute__((always_inline)) {
        const int jc = c * PF_VK;
#pragma unroll
        for (int u = 0; u < PN; ++u) {
            const int x = tid + u * PF_NT;
            pn[u] = jc + x / PF_AP < kend ? sb[(size_t)jc * PF_AP + x] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < VN; ++u) {
            const int x = tid + u * PF_NT, t = x / H4, c4 = x % H4, j = jc + t;
            vn[u] = (x < PF_VK * H4 && j < kend)
                        ? *reinterpret_cast<const float4*>(vc + (size_t)j * kvd + (size_t)kv * HD + 4 * c4)
                        : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    cload(0);
    for (int c = 0; c < nvc; ++c) {
        const int jc = c * PF_VK;
        __syncthreads();  // the previous chunk is consumed
#pragma unroll
        for (int u = 0; u < PN; ++u) Ps[tid + u * PF_NT] = pn[u] / rsum;  // pair tid % 64 throughout
#pragma unroll
        for (int u = 0; u < VN; ++u) {
            const int x = tid + u * PF_NT;
            if (x < PF_VK * H4) *reinterpret_cast<float4*>(Vs + (x / H4) * HP + 4 * (x % H4)) = vn[u];
        }
        __syncthreads();
        if (c + 1 < nvc) cload(c + 1);
        if (jc > 0 && jc % MM_KC == 0) {
#pragma unroll
            for (int a = 0; a < 8; ++a)
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    tot[a][d] = tot[a][d] + acc[a][d];
                    acc[a][d] = 0.0f;
                }
        }
        const bool full = jc >= rlast.j0 && jc + PF_VK <= rfirst.nk;
        if (lane_on && full) {
            for (int t = 0; t < PF_VK; ++t) {
                const float4 pa = *reinterpret_cast<const float4*>(Ps + t * PF_AP + 8 * pg);
                const float4 pb = *reinterpret_cast<const float4*>(Ps + t * PF_AP + 8 * pg + 4);
                const float4 v = *reinterpret_cast<const float4*>(Vs + t * HP + 4 * dg);
                const float pv[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
                const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int a = 0; a < 8; ++a) {
                    if (a % RP >= RV) continue;
#pragma unroll
                    for (int d = 0; d < 4; ++d) acc[a][d] = __builtin_fmaf(pv[a], vv[d], acc[a][d]);
                }
            }
        } else if (lane_on) {
            for (int t = 0; t < PF_VK; ++t) {
                const int j = jc + t;
                const float4 pa = *reinterpret_cast<const float4*>(Ps + t * PF_AP + 8 * pg);
                const float4 pb = *reinterpret_cast<const float4*>(Ps + t * PF_AP + 8 * pg + 4);
                const float4 v = *reinterpret_cast<const float4*>(Vs + t * HP + 4 * dg);
                const float pv[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
                const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int a = 0; a < 8; ++a) {
                    if (a % RP >= RV) continue;
                    const bool on = j >= rj0[a] && j < rnk[a];
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const float n = __builtin_fmaf(pv[a], vv[d], acc[a][d]);
                        acc[a][d] = on ? n : acc[a][d];
                    }
                }
            }
        }
    }
    if (lane_on) {
#pragma unroll
        for (int a = 0; a < 8; ++a) {
            const int pp = 8 * pg + a, h = pp % RP, i = r0 + pp / RP;
            if (h < R && i < m)
                *reinterpret_cast<float4*>(att + (size_t)i * H * HD + (size_t)(kv * R + h) * HD + 4 * dg) =
                    make_float4(tot[a][0] + acc[a][0], tot[a][1] + acc[a][1], tot[a][2] + acc[a][2],
                                tot[a][3] + acc[a][3]);
        }
    }
}

// LDS and scratch of the two-launch prefill attention
inline size_t pf_scores_lds(int hd) { return (size_t)(PF_AP + PF_KT) * (hd + 4) * sizeof(float); }
inline size_t pf_values_lds(int hd) {
    return std::max((size_t)PF_KT * PF_AP, (size_t)PF_VK * PF_AP + (size_t)PF_VK * (hd + 4)) * sizeof(float);
}
inline size_t pf_kpad(size_t npos) { return (npos + PF_KT - 1) / PF_KT * PF_KT; }

template <int RP, int RV, int HD>
hipError_t launch_pf_t(const float* qkv, int H, int KV, const int* cur, int m, const float* kc, const float* vc,
                       float qscale, float cap, int sl, int win, int nrb, int nkt, int kpad, float* st, float* pmx,
                       float* att, int div, hipStream_t s) {
    const size_t l1 = pf_scores_lds(HD), l2 = pf_values_lds(HD);
    static bool attr = false;  // per process; the attribute is per function
    if (!attr) {
        if (hipError_t e = hipFuncSetAttribute((const void*)gm_pf_scores_kernel<RP, RV, HD>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)l1))
            return e;
        if (hipError_t e = hipFuncSetAttribute((const void*)gm_pf_values_kernel<RP, RV, HD>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)l2))
            return e;
        attr = true;
    }
    gm_pf_scores_kernel<RP, RV, HD><<<dim3((unsigned)(KV * nrb)), dim3(PF_NT), l1, s>>>(
        qkv, H, KV, cur, m, kc, qscale, cap, sl, win, nrb, nkt, kpad, st, pmx, div);
    if (hipError_t e = hipGetLastError()) return e;
    gm_pf_values_kernel<RP, RV, HD><<<dim3((unsigned)(KV * nrb)), dim3(PF_NT), l2, s>>>(H, KV, cur, m, vc, sl, win, nrb,
                                                                                 kpad, st, pmx, att);
    return hipGetLastError();
}

template <int HD>
hipError_t launch_pf_h(int rp, const float* qkv, int H, int KV, const int* cur, int m, const float* kc,
                       const float* vc, float qscale, float cap, int sl, int win, int nrb, int nkt, int kpad, float* st,
                       float* pmx, float* att, int div, hipStream_t s) {
    // RV: the heads the FMAs run on (the spare ones of RP > R only where
    // R == 7, the Qwen2.5-7B group; elsewhere they run on zero q)
    const int R = H / KV;
    if (rp == 2) return launch_pf_t<2, 2, HD>(qkv, H, KV, cur, m, kc, vc, qscale, cap, sl, win, nrb, nkt, kpad, st, pmx, att, div, s);
    if (rp == 4) return launch_pf_t<4, 4, HD>(qkv, H, KV, cur, m, kc, vc, qscale, cap, sl, win, nrb, nkt, kpad, st, pmx, att, div, s);
    if (R == 7) return launch_pf_t<8, 7, HD>(qkv, H, KV, cur, m, kc, vc, qscale, cap, sl, win, nrb, nkt, kpad, st, pmx, att, div, s);
    return launch_pf_t<8, 8, HD>(qkv, H, KV, cur, m, kc, vc, qscale, cap, sl, win, nrb, nkt, kpad, st, pmx, att, div, s);
}

hipError_t launch_pf_attention(int rp, int hd, const float* qkv, int H, int KV, const int* cur, int m,
                               const float* kc, const float* vc, float qscale, float cap, int sl, int win, int nrb,
                               int nkt, int kpad, float* st, float* pmx, float* att, int div, hipStream_t s) {
    if (hd == 32) return launch_pf_h<32>(rp, qkv, H, KV, cur, m, kc, vc, qscale, cap, sl, win, nrb, nkt, kpad, st, pmx, att, div, s);
    if (hd == 64) return launch_pf_h<64>(rp, qkv, H, KV, cur, m, kc, vc, qscale, cap, sl, win, nrb, nkt, kpad, st, pmx, att, div, s);
    if (hd == 128) return launch_pf_h<128>(rp, qkv, H, KV, cur, m, kc, vc, qscale, cap, sl, win, nrb, nkt, kpad, st, pmx, att, div, s);
    return hipErrorInvalidValue;
}

// ---- decode attention for long caches, split into three launches ----
// The scores of the keys are independent (each a sequential FMA chain over
// the head dims), so they spread over many blocks; the softmax sum and the
// value chains stay one lane each, in key order.  Same arithmetic as
// gm_attn_kernel<.., true>, so the same bits.

// 1. Block b < H: bias, QK-norm and RoPE of q head b into qr; block H + kh:
// the same for k head kh (no norm on v), then k, v appended at cache row cur.
template <bool KV8>
__global__ __launch_bounds__(GT) void gm_dec_prep_kernel(const float* __restrict__ qkv, int H, int KV, int hd,
                                                         const int* __restrict__ curp, const float2* __restrict__ cs,
                                                         float* __restrict__ kc, float* __restrict__ vc,
                                                         int8_t* __restrict__ kq, int8_t* __restrict__ vq,
                                                         float* __restrict__ ks, float* __restrict__ vs,
                                                         const float* __restrict__ bias, const float* __restrict__ qn,
                                                         const float* __restrict__ kn, float eps,
                                                         float* __restrict__ qr) {
    extern __shared__ float4 lds4[];
    float* hv = reinterpret_cast<float*>(lds4);  // this head's vector (and v after it)
    const int b = blockIdx.x, half = hd / 2, kvd = KV * hd, hd4 = (hd + 3) & ~3;
    const bool isq = b < H;
    const int head = isq ? b : b - H;
    const size_t pos = (size_t)*curp;
    const int col0 = isq ? head * hd : (H + head) * hd;
    for (int c = threadIdx.x; c < hd; c += GT) {
        float v = qkv[col0 + c];
        if (bias) v = v + bias[col0 + c];
        hv[c] = v;
        if (!isq) {
            float w = qkv[(H + KV + head) * hd + c];
            if (bias) w = w + bias[(H + KV + head) * hd + c];
            hv[hd4 + c] = w;
        }
    }
    __syncthreads();
    if (qn) {
        if (threadIdx.x == 0) head_norm_lane(hv, hd, isq ? qn : kn, eps);
        __syncthreads();
    }
    const float2* csp = cs + pos * half;
    for (int j = threadIdx.x; j < half; j += GT) rope_pair(hv, j, half, csp);
    __syncthreads();
    if (isq) {
        for (int c = threadIdx.x; c < hd; c += GT) qr[head * hd + c] = hv[c];
    } else if constexpr (!KV8) {
        for (int c = threadIdx.x; c < hd; c += GT) {
            kc[pos * kvd + (size_t)head * hd + c] = hv[c];
            vc[pos * kvd + (size_t)head * hd + c] = hv[hd4 + c];
        }
    } else {
        const int wave = threadIdx.x >> 6;
        if (wave < 2)
            kv_quant_wave(hv + wave * hd4, hd, (wave ? vq : kq) + pos * kvd + (size_t)head * hd,
                          (wave ? vs : ks) + pos * KV + head);
    }
}

// 2. Scores: grid (H, key chunks of GT): thread j of chunk z scores key
// z GT + j of the window [j0, cur] into sc[h * pstride + j].
template <bool KV8, int HD = 0>
__global__ __launch_bounds__(GT) void gm_dec_score_kernel(const float* __restrict__ qr, int H, int KV, int hd,
                                                          const int* __restrict__ curp, const float* __restrict__ kc,
                                                          const int8_t* __restrict__ kq, const float* __restrict__ ks,
                                                          float qscale, float cap, int sliding, int window, int div,
                                                          int pstride, float* __restrict__ sc) {
    extern __shared__ float4 lds4[];
    float* q = reinterpret_cast<float*>(lds4);
    const int h = blockIdx.x, kv = h / (H / KV), kvd = KV * hd;
    const int ab = *curp, nk = ab + 1, j0 = (sliding && ab >= window) ? ab - window + 1 : 0;
    const int j = blockIdx.y * GT + threadIdx.x;
    if ((int)(blockIdx.y * GT) >= nk) return;  // block-uniform: past the cache
    for (int c = threadIdx.x; c < hd; c += GT) q[c] = qr[h * hd + c];
    __syncthreads();
    if (j < j0 || j >= nk) return;
    float acc = 0.0f;
    if constexpr (!KV8 && HD > 0) {
        // the whole key row requested at once (the old rows come from HBM)
        const float* kr = kc + (size_t)j * kvd + (size_t)kv * HD;
        float4 k4[HD / 4];
#pragma unroll
        for (int u = 0; u < HD / 4; ++u) k4[u] = *reinterpret_cast<const float4*>(kr + 4 * u);
        __builtin_amdgcn_sched_barrier(0);  // every load issued before the chain starts
#pragma unroll
        for (int u = 0; u < HD / 4; ++u) {
            acc = __builtin_fmaf(q[4 * u], k4[u].x, acc);
            acc = __builtin_fmaf(q[4 * u + 1], k4[u].y, acc);
            acc = __builtin_fmaf(q[4 * u + 2], k4[u].z, acc);
            acc = __builtin_fmaf(q[4 * u + 3], k4[u].w, acc);
        }
    } else if constexpr (!KV8) {
        const float* kr = kc + (size_t)j * kvd + (size_t)kv * hd;
        for (int c = 0; c < hd; c += 4) {
            const float4 k4 = *reinterpret_cast<const float4*>(kr + c);
            acc = __builtin_fmaf(q[c], k4.x, acc);
            acc = __builtin_fmaf(q[c + 1], k4.y, acc);
            acc = __builtin_fmaf(q[c + 2], k4.z, acc);
            acc = __builtin_fmaf(q[c + 3], k4.w, acc);
        }
    } else {
        const int8_t* kr = kq + (size_t)j * kvd + (size_t)kv * hd;
        const float sk = ks[(size_t)j * KV + kv];
        for (int c = 0; c < hd; c += 4) {
            const char4 k4 = *reinterpret_cast<const char4*>(kr + c);
            acc = __builtin_fmaf(q[c], (float)k4.x * sk, acc);
            acc = __builtin_fmaf(q[c + 1], (float)k4.y * sk, acc);
            acc = __builtin_fmaf(q[c + 2], (float)k4.z * sk, acc);
            acc = __builtin_fmaf(q[c + 3], (float)k4.w * sk, acc);
        }
    }
    float sj = div ? acc / qscale : acc * qscale;
    if (cap > 0.0f) sj = cap * libm::frq_tanhf(sj / cap);
    sc[(size_t)h * pstride + j] = sj;
}

// 1 + 2 fused for the f32 cache: grid (H, key chunks of GT).  Every
// workgroup prepares its own q head as gm_dec_prep_kernel does (bias,
// QK-norm, RoPE at position cur) and scores its chunk's keys; the chunk
// holding key cur prepares that key's k as well and scores it from LDS,
// and for the first head of each kv group also appends k and v at cache
// row cur (read by the value step, a launch later; no workgroup of this
// launch reads that row from the cache).  Same arithmetic, so the same
// bits; key rows requested whole before each chain.
template <int HD>
__global__ __launch_bounds__(GT) void gm_dec_qks_kernel(const float* __restrict__ qkv, int H, int KV,
                                                        const int* __restrict__ curp, const float2* __restrict__ cs,
                                                        float* __restrict__ kc, float* __restrict__ vc,
                                                        const float* __restrict__ bias, const float* __restrict__ qn,
                                                        const float* __restrict__ kn, float eps, float qscale,
                                                        float cap, int sliding, int window, int div, int pstride,
                                                        float* __restrict__ sc) {
    __shared__ float qs[HD], kl[HD];
    constexpr int half = HD / 2;
    const int h = blockIdx.x, R = H / KV, kv = h / R, kvd = KV * HD, tid = threadIdx.x;
    const int ab = *curp, nk = ab + 1, j0 = (sliding && ab >= window) ? ab - window + 1 : 0;
    const int zb = (int)blockIdx.y * GT;
    if (zb >= nk) return;  // block-uniform: past the cache
    const bool last = zb + GT >= nk;  // this chunk holds key ab
    const size_t pos = (size_t)ab;
    for (int c = tid; c < HD; c += GT) {
        float v = qkv[h * HD + c];
        if (bias) v = v + bias[h * HD + c];
        qs[c] = v;
        if (last) {
            float w = qkv[(H + kv) * HD + c];
            if (bias) w = w + bias[(H + kv) * HD + c];
            kl[c] = w;
        }
    }
    __syncthreads();
    if (qn) {
        if (tid == 0) head_norm_lane(qs, HD, qn, eps);
        if (last && tid == 64) head_norm_lane(kl, HD, kn, eps);
        __syncthreads();
    }
    const float2* csp = cs + pos * half;
    for (int t = tid; t < (last ? 2 : 1) * half; t += GT) rope_pair(t < half ? qs : kl, t % half, half, csp);
    __syncthreads();
    if (last && h % R == 0) {
        for (int c = tid; c < HD; c += GT) {
            float w = qkv[(H + KV + kv) * HD + c];
            if (bias) w = w + bias[(H + KV + kv) * HD + c];
            kc[pos * kvd + (size_t)kv * HD + c] = kl[c];
            vc[pos * kvd + (size_t)kv * HD + c] = w;
        }
    }
    const int j = zb + tid;
    if (j < j0 || j >= nk) return;
    float acc = 0.0f;
    if (j == ab) {
#pragma unroll 8
        for (int c = 0; c < HD; ++c) acc = __builtin_fmaf(qs[c], kl[c], acc);
    } else {
        const float* kr = kc + (size_t)j * kvd + (size_t)kv * HD;
        float4 k4[HD / 4];
#pragma unroll
        for (int u = 0; u < HD / 4; ++u) k4[u] = *reinterpret_cast<const float4*>(kr + 4 * u);
        __builtin_amdgcn_sched_barrier(0);  // every load issued before the chain starts
#pragma unroll
        for (int u = 0; u < HD / 4; ++u) {
            acc = __builtin_fmaf(qs[4 * u], k4[u].x, acc);
            acc = __builtin_fmaf(qs[4 * u + 1], k4[u].y, acc);
            acc = __builtin_fmaf(qs[4 * u + 2], k4[u].z, acc);
            acc = __builtin_fmaf(qs[4 * u + 3], k4[u].w, acc);
        }
    }
    float sj = div ? acc / qscale : acc * qscale;
    if (cap > 0.0f) sj = cap * libm::frq_tanhf(sj / cap);
    sc[(size_t)h * pstride + j] = sj;
}

// 3. Per head: max, exp, the key-order sum, divide, then the value chains.
template <bool KV8>
__global__ __launch_bounds__(GT) void gm_dec_value_kernel(const float* __restrict__ sc, int H, int KV, int hd,
                                                          const int* __restrict__ curp, const float* __restrict__ vc,
                                                          const int8_t* __restrict__ vq, const float* __restrict__ vs,
                                                          int sliding, int window, int pstride,
                                                          float* __restrict__ att) {
    extern __shared__ float4 lds4[];
    float* p = reinterpret_cast<float*>(lds4);
    float* sv = p + pstride;
    __shared__ float red[4];
    const int h = blockIdx.x, kv = h / (H / KV), kvd = KV * hd;
    const int ab = *curp, nk = ab + 1, j0 = (sliding && ab >= window) ? ab - window + 1 : 0;
    float mx = -INFINITY;
    for (int j = j0 + threadIdx.x; j < nk; j += GT) {
        const float v = sc[(size_t)h * pstride + j];
        p[j] = v;
        mx = fmaxf(mx, v);
        if constexpr (KV8) sv[j] = vs[(size_t)j * KV + kv];
    }
    mx = gblock_max(mx, red);
    if (j0 > 0) mx = fmaxf(mx, -1e30f);  // a masked entry joins the max
    for (int j = j0 + threadIdx.x; j < nk; j += GT) p[j] = libm::frq_expf(p[j] - mx);
    __syncthreads();
    // key order from j0: the few keys before the next 16-byte boundary in
    // every thread, the rest by the workgroup's speculative segmented fold
    const int ja = min((j0 + 3) & ~3, nk);
    float head = 0.0f;
    for (int j = j0; j < ja; ++j) head = head + p[j];
    const float sum = seq_sum_spec<GT>(p + ja, nk - ja, head, sv + pstride);
    for (int j = j0 + threadIdx.x; j < nk; j += GT) p[j] = p[j] / sum;
    __syncthreads();
    // three batches of B keys in flight (48 loads a wave, within the 63 the
    // wave's vector-memory counter tracks): the cache is read from L2 / HBM
    constexpr int B = 16;
    for (int c = threadIdx.x; c < hd; c += GT) {
        const size_t col = (size_t)kv * hd + c;
        // one a.dot block of keys [s, e), chained from +0
        auto chain = [&](int s, int e) {
            float acc = 0.0f;
            const int nb = (e - s) / B;
            float v0[B], v1[B], v2[B];
            auto ld = [&](float (&v)[B], int k) {
#pragma unroll
                for (int u = 0; u < B; ++u) {
                    const size_t j = (size_t)(s + k * B + u);
                    if constexpr (!KV8) v[u] = vc[j * kvd + col];
                    else v[u] = (float)vq[j * kvd + col] * sv[j];
                }
            };
            auto fma_b = [&](const float (&v)[B], int k) {
#pragma unroll
                for (int u = 0; u < B; ++u) acc = __builtin_fmaf(p[s + k * B + u], v[u], acc);
            };
            if (nb > 0) {
                ld(v0, 0);
                ld(v1, min(1, nb - 1));
                ld(v2, min(2, nb - 1));
                __builtin_amdgcn_sched_barrier(0);
                int k = 0;
                for (; k + 3 <= nb; k += 3) {
                    fma_b(v0, k);
                    ld(v0, min(k + 3, nb - 1));
                    __builtin_amdgcn_sched_barrier(0);
                    fma_b(v1, k + 1);
                    ld(v1, min(k + 4, nb - 1));
                    __builtin_amdgcn_sched_barrier(0);
                    fma_b(v2, k + 2);
                    ld(v2, min(k + 5, nb - 1));
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (k < nb) fma_b(v0, k);
                if (k + 1 < nb) fma_b(v1, k + 1);
            }
            for (int j = s + nb * B; j < e; ++j) {
                const float v = KV8 ? (float)vq[(size_t)j * kvd + col] * sv[j] : vc[(size_t)j * kvd + col];
                acc = __builtin_fmaf(p[j], v, acc);
            }
            return acc;
        };
        att[(size_t)h * hd + c] = mm_blocks(j0, nk, chain);
    }
}

// ---- long-cache decode value step, a.dot's blocks in parallel -------------
// gm_dec_value_kernel's work for VB_CW channels of one head per workgroup:
// the softmax as there, by VT threads (the in-order sum a speculative fold
// over 16 segments by 512 of them), then the value product in a.dot's order, whose
// blocks of MM_KC keys (at absolute multiples) are independent chains from
// +0: thread t takes channel t % VB_CW of block t / VB_CW (and every
// VT / VB_CW-th block after it), its chain fed by 16-key batches of value
// loads two batches ahead (a key's VB_CW channels one coalesced row piece);
// the block results go to LDS and the first VB_CW threads add them in block
// order.  Per output the arithmetic is gm_dec_value_kernel's, bit for bit.
constexpr int VT = 1024, VB_CW = 32;

template <bool KV8>
__global__ __launch_bounds__(VT) void gm_dec_value_blk_kernel(const float* __restrict__ sc, int H, int KV, int hd,
                                                              const int* __restrict__ curp,
                                                              const float* __restrict__ vc,
                                                              const int8_t* __restrict__ vq,
                                                              const float* __restrict__ vs, int sliding, int window,
                                                              int pstride, float* __restrict__ att) {
    constexpr int NW = VT / 64, BPP = VT / VB_CW;
    extern __shared__ float4 lds4[];
    // p and sv hold key j at index j - j0
    float* p = reinterpret_cast<float*>(lds4);
    float* sv = p + pstride;
    float* fsc = sv + pstride;
    float* part = fsc + seq_sum_spec_scratch(VT);  // [block][VB_CW]
    __shared__ float red[NW];
    const int h = blockIdx.x, kv = h / (H / KV), kvd = KV * hd, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ab = *curp, nk = ab + 1, j0 = (sliding && ab >= window) ? ab - window + 1 : 0;
    const int n = nk - j0;
    // the softmax, as gm_dec_value_kernel (the key-order sum from +0 over
    // the keys j0 .. nk - 1); the scores SB to a thread at a time, every
    // load of a batch issued before the first is used
    constexpr int SB = 4;
    float mx = -INFINITY;
    for (int b0 = 0; b0 < n; b0 += SB * VT) {
        float vv[SB], ss[SB];
#pragma unroll
        for (int u = 0; u < SB; ++u) {
            const int j = min(b0 + (int)threadIdx.x + u * VT, n - 1);
            vv[u] = sc[(size_t)h * pstride + j0 + j];
            if constexpr (KV8) ss[u] = vs[(size_t)(j0 + j) * KV + kv];
        }
#pragma unroll
        for (int u = 0; u < SB; ++u) {
            const int j = b0 + (int)threadIdx.x + u * VT;
            if (j < n) {
                p[j] = vv[u];
                mx = fmaxf(mx, vv[u]);
                if constexpr (KV8) sv[j] = ss[u];
            }
        }
    }
    mx = gwave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = fmaxf(mx, red[w]);
    if (j0 > 0) mx = fmaxf(mx, -1e30f);  // a masked entry joins the max
    for (int j = threadIdx.x; j < n; j += VT) p[j] = libm::frq_expf(p[j] - mx);
    __syncthreads();
    // (folded by 512 of the threads: the chains cost the same, the barriers
    // and the resolve over half the segments less; 2.7 against 3.8 us at
    // 2176 keys)
    const float sum = seq_sum_spec<VT, 512>(p, n, 0.0f, fsc);
    for (int j = threadIdx.x; j < n; j += VT) p[j] = p[j] / sum;
    __syncthreads();
    // the blocks of keys [j0, nk)
    const int bf = j0 / MM_KC, nblk = (nk - 1) / MM_KC - bf + 1;
    const int c = threadIdx.x % VB_CW;
    const size_t col = (size_t)kv * hd + blockIdx.y * VB_CW + c;
    constexpr int B = 16;
    for (int bi = threadIdx.x / VB_CW; bi < nblk; bi += BPP) {
        const int s = max(j0, (bf + bi) * MM_KC), e = min(nk, (bf + bi + 1) * MM_KC), nb = (e - s) / B;
        float acc = 0.0f;
        float v0[B], v1[B];
        auto ld = [&](float (&v)[B], int k) __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < B; ++u) {
                const size_t j = (size_t)(s + k * B + u);
                if constexpr (!KV8) v[u] = vc[j * kvd + col];
                else v[u] = (float)vq[j * kvd + col] * sv[j - j0];
            }
        };
        auto fma_b = [&](const float (&v)[B], int k) __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < B; ++u) acc = __builtin_fmaf(p[s - j0 + k * B + u], v[u], acc);
        };
        if (nb > 0) {  // both batches of a trip consumed unconditionally, loads pinned a batch ahead
            ld(v0, 0);
            ld(v1, min(1, nb - 1));
            __builtin_amdgcn_sched_barrier(0);
            int k = 0;
            for (; k + 2 <= nb; k += 2) {
                fma_b(v0, k);
                ld(v0, min(k + 2, nb - 1));
                __builtin_amdgcn_sched_barrier(0);
                fma_b(v1, k + 1);
                ld(v1, min(k + 3, nb - 1));
                __builtin_amdgcn_sched_barrier(0);
            }
            if (k < nb) fma_b(v0, k);
        }
        for (int j = s + nb * B; j < e; ++j) {
            const float v = KV8 ? (float)vq[(size_t)j * kvd + col] * sv[j - j0] : vc[(size_t)j * kvd + col];
            acc = __builtin_fmaf(p[j - j0], v, acc);
        }
        part[bi * VB_CW + c] = acc;
    }
    __syncthreads();
    if (threadIdx.x < VB_CW) {
        float t = 0.0f;
        for (int bi = 0; bi < nblk; ++bi) t = t + part[bi * VB_CW + threadIdx.x];
        att[(size_t)h * hd + blockIdx.y * VB_CW + threadIdx.x] = t;
    }
}

// h = act(gate) * up over m rows of the [gate | up] buffer: gelu_tanh
// (gemma.rs:31-34) or, silu, x / (1 + exp(-x)) (rope.rs:39-41).
// a4 (a batch's rows, <= 16, feeding an int4 linear): the rows also in the
// k-quad interleaved layout of launch_i4_rows_a4.
// hr > 0: the pair's columns interleaved in runs of hr (gated_col: gate
// column col at gated_col(col, hr), up hr further), else [gate | up].
__global__ __launch_bounds__(GT) void gm_geglu_kernel(const float* __restrict__ gu, int ffn, size_t total,
                                                      float c, float* __restrict__ hm, int silu, int hr,
                                                      float* __restrict__ a4 = nullptr) {
    auto act = [&](float x) __attribute__((always_inline)) {
        return silu ? x / (1.0f + libm::frq_expf_sel(-x))
                    : 0.5f * x * (1.0f + libm::frq_tanhf(c * (x + 0.044715f * x * x * x)));
    };
    const size_t up = hr ? (size_t)hr : (size_t)ffn;  // up column's offset from its gate column
    if (silu && (ffn & 3) == 0 && hr == 2 && total >= (size_t)16 * ffn) {
        // prefill SiLU on pairs in runs of 2: columns 4 c4 .. 4 c4 + 3 are
        // the gates and ups of two float4s, [g g u u][g g u u]
        const size_t f4 = (size_t)ffn >> 2, t4 = total >> 2;
        for (size_t i = (size_t)blockIdx.x * GT + threadIdx.x; i < t4; i += (size_t)gridDim.x * GT) {
            const size_t r = i / f4, c4 = i - r * f4;
            const float4 p = *reinterpret_cast<const float4*>(gu + r * 2 * ffn + 8 * c4);
            const float4 q = *reinterpret_cast<const float4*>(gu + r * 2 * ffn + 8 * c4 + 4);
            const float4 h = make_float4(act(p.x) * p.z, act(p.y) * p.w, act(q.x) * q.z, act(q.y) * q.w);
            reinterpret_cast<float4*>(hm)[i] = h;
            if (a4) reinterpret_cast<float4*>(a4)[c4 * 16 + r] = h;
        }
        return;
    }
    if (silu && (ffn & 3) == 0 && (hr & 3) == 0 && total >= (size_t)16 * ffn) {
        // prefill SiLU: four adjacent columns a thread, float4 loads, four
        // independent exps (decode rows keep a column a thread: more threads)
        const size_t f4 = (size_t)ffn >> 2, t4 = total >> 2;
        for (size_t i = (size_t)blockIdx.x * GT + threadIdx.x; i < t4; i += (size_t)gridDim.x * GT) {
            const size_t r = i / f4, c4 = i - r * f4, gcol = gated_col(4 * c4, (size_t)hr);  // 4 | hr
            const float4 g = *reinterpret_cast<const float4*>(gu + r * 2 * ffn + gcol);
            const float4 u = *reinterpret_cast<const float4*>(gu + r * 2 * ffn + gcol + up);
            const float4 h = make_float4(act(g.x) * u.x, act(g.y) * u.y, act(g.z) * u.z, act(g.w) * u.w);
            reinterpret_cast<float4*>(hm)[i] = h;
            if (a4) reinterpret_cast<float4*>(a4)[c4 * 16 + r] = h;
        }
        return;
    }
    for (size_t i = (size_t)blockIdx.x * GT + threadIdx.x; i < total; i += (size_t)gridDim.x * GT) {
        const size_t r = i / ffn, col = i - r * ffn, gcol = gated_col(col, (size_t)hr);
        const float h = act(gu[r * 2 * ffn + gcol]) * gu[r * 2 * ffn + gcol + up];
        hm[i] = h;
        if (a4) a4[(col >> 2) * 64 + 4 * r + (col & 3)] = h;
    }
}

// The token the unembed's folded argmax chose goes to out[cur + m - P];
// cur += m; the key is cleared.
// A batch step's tokens: sequence b's argmax to out[b tstride + cur + 1 - P]
// (after its previous token), then every sequence one position on.
__global__ void gm_argmax_batch_kernel(unsigned long long* __restrict__ best, int* __restrict__ curp, int nb, int P,
                                       int64_t* __restrict__ out, int tstride) {
    const int cur = *curp;
    for (int b = threadIdx.x; b < nb; b += blockDim.x) {
        out[(size_t)b * tstride + cur + 1 - P] = (int64_t)(uint32_t)(best[b] & 0xffffffffull);
        best[b] = 0ull;
    }
    __syncthreads();
    if (threadIdx.x == 0) *curp = cur + 1;
}

__global__ void gm_argmax_done_kernel(unsigned long long* __restrict__ best, int* __restrict__ curp, int m, int P,
                                      int64_t* __restrict__ out) {
    if (threadIdx.x == 0) {
        const int cur = *curp;
        out[cur + m - P] = (int64_t)(uint32_t)(*best & 0xffffffffull);
        *curp = cur + m;
        *best = 0ull;
    }
}

}  // namespace
}  // namespace frq

using namespace frq;

struct frq_gemma {
    int device = 0;
    size_t L = 0, H = 0, KV = 0, hd = 0, d = 0, ffn = 0, vocab = 0;
    size_t window = 4096;
    float theta = 0, eps = 0, cap = 0, qscale = 0, escale = 0;
    int kv8 = 0, graphs = 1;
    int arch = 0;                    // 0 gemma (gemma.rs), 1 the Llama / Qwen family (rope.rs)
    std::vector<float> inv;          // RoPE inverse frequencies
    std::vector<frq_w*> qkv, o, gu, down;
    // per layer: the int8 gate|up pair's rows interleaved in runs of gu_hr
    // (gated_col; the decode row's activation then runs in the fused
    // linear's epilogue), or 0: [gate | up]
    std::vector<int> gu_hr;
    frq_w* embed = nullptr;
    frq_w* unembed = nullptr;        // rope, untied: lm_head (else the embed table)
    float* norms = nullptr;          // 4 per layer + the final norm, f32 (d each)
    float* qkvbias = nullptr;        // rope: (H + 2 nkv) hd per layer, or NULL
    float* qknorm = nullptr;         // rope (Qwen3): q_norm, k_norm (hd each) per layer, or NULL
    // sized to the largest call so far: positions (cache, RoPE table) and rows
    size_t cap_pos = 0, cap_rows = 0;
    char* buf = nullptr;
    float2* cs = nullptr;
    float *kc = nullptr, *vc = nullptr, *ks = nullptr, *vs = nullptr;
    int8_t *kq = nullptr, *vq = nullptr;
    float *x = nullptr, *a = nullptr, *qkvb = nullptr, *att = nullptr, *ob = nullptr, *gub = nullptr, *hm = nullptr,
          *logits = nullptr;
    int* cur = nullptr;
    unsigned long long* best = nullptr;
    int64_t *tok = nullptr, *ids = nullptr;
    float *qr = nullptr, *sc = nullptr;  // long-cache decode attention: roped q, scores
    float* xt = nullptr;                 // batches: 16 staging rows (the head's input transposed,
                                         // the int4 linears' a4 layout), 16 (max(d, ffn, H hd) + 4)
    float* pst = nullptr;                // prefill attention: scores / exps, [KV][block][kpad][64]
    float* pmx = nullptr;                // prefill attention: the pairs' maxima, [KV][block][64]
    // the quantised decode rows of the int8 linears (d- and ffn-wide: the
    // padding of each stays zero), their scales and outliers
    int8_t* q8f = nullptr;
    float* qsa = nullptr;     // [1]
    uint32_t* qoi = nullptr;  // [32]
    float* qov = nullptr;     // [32]
    // batches of sequences: the caches and token arrays hold cap_b
    // sequences; seq is the sequence a one-sequence call (a prefill) works on
    size_t cap_b = 0, seq = 0;
    ~frq_gemma() {
        for (auto* v : {&qkv, &o, &gu, &down})
            for (frq_w* w : *v) frq_w_free(w);
        frq_w_free(embed);
        frq_w_free(unembed);
        if (norms) (void)hipFree(norms);
        if (qkvbias) (void)hipFree(qkvbias);
        if (qknorm) (void)hipFree(qknorm);
        if (buf) (void)hipFree(buf);
    }
    const float* norm_of(size_t l, int j) const { return norms + (4 * l + j) * d; }
    // the post-norms before the residuals (gemma); rope has none
    const float* post_of(size_t l, int j) const { return arch == 0 ? norm_of(l, j) : nullptr; }
    const float* bias_of(size_t l) const { return qkvbias ? qkvbias + l * (H + 2 * KV) * hd : nullptr; }
    const float* qn_of(size_t l) const { return qknorm ? qknorm + l * 2 * hd : nullptr; }
    const float* kn_of(size_t l) const { return qknorm ? qknorm + l * 2 * hd + hd : nullptr; }
    const float* final_norm() const { return norms + 4 * L * d; }
};

namespace {

int gfail(hipError_t e, const char* what) { return set_error(FRQ_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e)); }
#define GMCHK(expr, what)                              \
    do {                                               \
        hipError_t e_ = (expr);                        \
        if (e_ != hipSuccess) return gfail(e_, what);  \
    } while (0)

struct GDev {
    int prev = -1;
    explicit GDev(int d) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != d) (void)hipSetDevice(d);
    }
    ~GDev() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

// Two or three linears with the same input concatenated along the output:
// the stored arrays' output rows (int4 / q4a: rows of the (out, in) store;
// int8: columns of the (in, out) store) side by side, scales likewise.
// hr > 0, int8, two linears of equal width divisible by hr (a gated pair):
// their columns interleaved in runs of hr instead (gated_col), *hr_out = hr;
// else *hr_out = 0.
int concat_linear(frq_ctx* c, const frq_bundle* b, const std::vector<std::string>& names, size_t k, frq_w** out,
                  size_t hr = 0, int* hr_out = nullptr) {
    if (hr_out) *hr_out = 0;
    struct Arr {
        std::string dt;
        size_t shape[4], nd = 4, grp = 0, bytes = 0;
        const void* data = nullptr;
    };
    auto get = [&](const std::string& nm, Arr& a) {
        char dt[16];
        const int rc = frq_bundle_array(b, nm.c_str(), dt, sizeof dt, a.shape, &a.nd, &a.grp, &a.data, &a.bytes);
        a.dt = dt;
        return rc;
    };
    std::vector<Arr> w(names.size()), s(names.size()), mn(names.size());
    size_t ntot = 0;
    for (size_t i = 0; i < names.size(); ++i) {
        if (int rc = get(names[i], w[i])) return rc;
        if (int rc = get(names[i] + "__scale", s[i])) return rc;
        if (w[i].dt != w[0].dt || w[i].nd != 2) return set_error(FRQ_ERR_FORMAT, names[i] + ": mixed or bad dtype");
        if (w[i].dt == "q4a")
            if (int rc = get(names[i] + "__min", mn[i])) return rc;
        const bool i8 = w[i].dt == "i8";
        const size_t kin = i8 ? w[i].shape[0] : w[i].shape[1];
        if (kin != k) return set_error(FRQ_ERR_FORMAT, names[i] + ": input width " + std::to_string(kin));
        if (s[i].dt != "f16") return set_error(FRQ_ERR_FORMAT, names[i] + "__scale: f16 expected");
        ntot += i8 ? w[i].shape[1] : w[i].shape[0];
    }
    const std::string dt = w[0].dt;
    if (dt == "i8") {
        std::vector<int8_t> cat(k * ntot);
        std::vector<uint16_t> sc(ntot);
        const size_t h = w[0].shape[1];
        if (hr && names.size() == 2 && w[1].shape[1] == h && h % hr == 0) {
            // a gated pair in runs of hr: gate column c at gated_col(c, hr),
            // up column c hr further
            const int8_t* gs = static_cast<const int8_t*>(w[0].data);
            const int8_t* us = static_cast<const int8_t*>(w[1].data);
            const uint16_t* gsc = static_cast<const uint16_t*>(s[0].data);
            const uint16_t* usc = static_cast<const uint16_t*>(s[1].data);
            for (size_t p0 = 0; p0 < h; p0 += hr) {
                const size_t dst = gated_col(p0, hr);
                for (size_t r = 0; r < k; ++r) {
                    std::memcpy(&cat[r * ntot + dst], gs + r * h + p0, hr);
                    std::memcpy(&cat[r * ntot + dst + hr], us + r * h + p0, hr);
                }
                std::memcpy(&sc[dst], gsc + p0, hr * 2);
                std::memcpy(&sc[dst + hr], usc + p0, hr * 2);
            }
            if (hr_out) *hr_out = (int)hr;
        } else {
            size_t off = 0;
            for (size_t i = 0; i < names.size(); ++i) {
                const size_t n = w[i].shape[1];
                const int8_t* src = static_cast<const int8_t*>(w[i].data);
                for (size_t r = 0; r < k; ++r) std::memcpy(&cat[r * ntot + off], src + r * n, n);
                std::memcpy(&sc[off], s[i].data, n * 2);
                off += n;
            }
        }
        *out = frq_upload_i8_bundle(c, cat.data(), sc.data(), k, ntot);
    } else if (dt == "i4" || dt == "q4a") {
        const size_t g = w[0].grp ? w[0].grp : (dt == "i4" ? 32 : 64), rb = (k + 1) / 2, ng = (k + g - 1) / g;
        std::vector<uint8_t> cat(ntot * rb);
        std::vector<uint16_t> sc(ntot * ng), mv(dt == "q4a" ? ntot * ng : 0);
        size_t off = 0;
        for (size_t i = 0; i < names.size(); ++i) {
            const size_t n = w[i].shape[0];
            if ((w[i].grp ? w[i].grp : g) != g) return set_error(FRQ_ERR_FORMAT, names[i] + ": group differs");
            std::memcpy(&cat[off * rb], w[i].data, n * rb);
            std::memcpy(&sc[off * ng], s[i].data, n * ng * 2);
            if (dt == "q4a") std::memcpy(&mv[off * ng], mn[i].data, n * ng * 2);
            off += n;
        }
        *out = dt == "i4" ? frq_upload_i4(c, cat.data(), sc.data(), ntot, k, g)
                          : frq_upload_q4a(c, cat.data(), sc.data(), mv.data(), ntot, k, g);
    } else {
        return set_error(FRQ_ERR_DTYPE, names[0] + ": gemma linears must be i8, i4 or q4a");
    }
    return *out ? FRQ_OK : last_code();
}

int one_linear(frq_ctx* c, const frq_bundle* b, const std::string& name, size_t k, size_t n, frq_w** out) {
    if (int rc = frq_bundle_weight(c, b, name.c_str(), out)) return rc;
    int dt = 0;
    size_t wn = 0, wk = 0, g = 0;
    (void)frq_w_info(*out, &dt, &wn, &wk, &g);
    if (dt != FRQ_DT_I8 && dt != FRQ_DT_I4 && dt != FRQ_DT_Q4A)
        return set_error(FRQ_ERR_DTYPE, name + ": gemma linears must be i8, i4 or q4a");
    if (wk != k || wn != n) return set_error(FRQ_ERR_FORMAT, name + ": unexpected shape");
    return FRQ_OK;
}

// Bundle::mm in the reference's order for m rows.
int gm_mm(frq_ctx* c, const frq_w* wh, const float* in, size_t m, float* outp) {
    const Weight& w = *weight_of(wh);
    hipStream_t s = (hipStream_t)frq_get_stream(c);
    if (w.dtype == FRQ_DT_I4) {
        GMCHK(launch_i4_exact(w, m, in, outp, s), "launch i4");
        return FRQ_OK;
    }
    if (w.dtype == FRQ_DT_Q4A) {
        GMCHK(launch_q4a(w, m, in, outp, s), "launch q4a");
        return FRQ_OK;
    }
    if (m <= 16) return frq_mm_dev(c, wh, in, m, outp);
    if (i8_rows_exact_ok(wh, m)) return mm_i8_rows_exact(c, wh, in, m, outp);
    const size_t nch = (m + 15) / 16;  // int8: the bit-exact multi-row path in chunks of 8..16 rows
    size_t r0 = 0;
    for (size_t i = 0; i < nch; ++i) {
        const size_t rows = m / nch + (i < m % nch ? 1 : 0);
        if (int rc = frq_mm_dev(c, wh, in + r0 * w.k, rows, outp + r0 * w.n)) return rc;
        r0 += rows;
    }
    return FRQ_OK;
}

// The linears of a batch step: m rows, each its own sequence's decode row,
// so each row in the M == 1 order of its dtype (int8: the multi-row path is
// bit-identical to M == 1 up to 16 rows; int4: i4_dot_avx2's order for every
// row, a4 the broadcast kernel's staging of i4_a4_floats(K) floats; q4a: one
// M == 1 call a row).
int gm_mm_rows(frq_ctx* c, const frq_w* wh, const float* in, size_t m, float* outp, float* a4) {
    const Weight& w = *weight_of(wh);
    hipStream_t s = (hipStream_t)frq_get_stream(c);
    if (w.dtype == FRQ_DT_I4) {
        GMCHK(launch_i4_m1_rows(w, m, in, outp, a4, s), "launch i4 rows");
        return FRQ_OK;
    }
    if (w.dtype == FRQ_DT_Q4A) {
        for (size_t i = 0; i < m; ++i)
            GMCHK(launch_q4a(w, 1, in + i * w.k, outp + i * w.n, s), "launch q4a");
        return FRQ_OK;
    }
    for (size_t r0 = 0; r0 < m; r0 += 16)
        if (int rc = frq_mm_dev(c, wh, in + r0 * w.k, std::min<size_t>(16, m - r0), outp + r0 * w.n)) return rc;
    return FRQ_OK;
}

size_t gm_pstride_n(size_t npos) { return (npos + 3) & ~(size_t)3; }
size_t gm_pstride(const frq_gemma* g) { return gm_pstride_n(g->cap_pos); }
// LDS of the one-launch attention (gm_attn_kernel: q, two hd-vectors and
// two score rows of the padded position count); the long-cache value
// kernel needs the two score rows only, so this bounds both.
size_t gm_attn_lds_n(size_t hd, size_t npos) {
    return (3 * ((hd + 3) & ~(size_t)3) + 2 * gm_pstride_n(npos) + seq_sum_spec_scratch(GT)) * sizeof(float);
}
size_t gm_attn_lds(const frq_gemma* g) { return gm_attn_lds_n(g->hd, g->cap_pos); }
constexpr size_t GM_LDS_MAX = 160 * 1024;  // gfx950's LDS per workgroup

// Dynamic LDS above the default 64 KB for the kernels whose need grows with
// the cache length.
hipError_t gm_allow_lds(size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    const void* ks[] = {(const void*)gm_attn_kernel<false, false>, (const void*)gm_attn_kernel<false, true>,
                        (const void*)gm_attn_kernel<true, false>, (const void*)gm_attn_kernel<true, true>,
                        (const void*)gm_dec_value_kernel<false>, (const void*)gm_dec_value_kernel<true>};
    for (const void* k : ks)
        if (hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds)) return e;
    return hipSuccess;
}

// LDS of the block-parallel value kernel for a padded position count ps:
// p and sv, the fold's scratch, and a VB_CW-float row per block of keys.
size_t value_blk_lds(size_t ps) {
    return (2 * ps + seq_sum_spec_scratch(VT) + (ps / MM_KC + 2) * VB_CW) * sizeof(float);
}

// The long-cache value step, blocks in parallel, when the head size and the
// LDS allow it; hipErrorNotSupported sends the caller to gm_dec_value_kernel.
hipError_t launch_value_blk(const frq_gemma* g, int sl, int win, int ps, const float* vc, const int8_t* vq,
                            const float* vs, float* att, hipStream_t s) {
    const size_t lds = value_blk_lds(ps);
    if (g->hd % VB_CW || lds > GM_LDS_MAX) return hipErrorNotSupported;
    const dim3 grid((unsigned)g->H, (unsigned)(g->hd / VB_CW));
    if (g->kv8)
        gm_dec_value_blk_kernel<true><<<grid, dim3(VT), lds, s>>>(g->sc, (int)g->H, (int)g->KV, (int)g->hd, g->cur,
                                                                   vc, vq, vs, sl, win, ps, att);
    else
        gm_dec_value_blk_kernel<false><<<grid, dim3(VT), lds, s>>>(g->sc, (int)g->H, (int)g->KV, (int)g->hd, g->cur,
                                                                    vc, vq, vs, sl, win, ps, att);
    return hipGetLastError();
}

hipError_t allow_value_blk_lds(size_t ps) {
    const size_t lds = value_blk_lds(ps);
    if (lds > GM_LDS_MAX || lds <= 64 * 1024) return hipSuccess;  // the caller takes the other kernel / the default
    const void* ks[] = {(const void*)gm_dec_value_blk_kernel<false>, (const void*)gm_dec_value_blk_kernel<true>};
    for (const void* k : ks)
        if (hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds)) return e;
    return hipSuccess;
}

// NV4 of the fused quant for a row of K: 0 when it does not apply.
int quant_nv4(size_t k) {
    if (k <= FRQ_T || k % 4 || k > (size_t)FRQ_QMAXK) return 0;
    return (int)((k / 4 + QNT - 1) / QNT);
}

template <int NV4>
hipError_t allow_quant_kernel(size_t alds) {
    // (its static LDS, the quant's selection state, counts against the same
    // limit, so the attribute is set whatever the dynamic size)
    return hipFuncSetAttribute((const void*)gm_act_quant_kernel<NV4>, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)alds);
}

// The activation + quant kernel's dynamic LDS: the activation row.
size_t act_quant_lds(int ffn) { return (size_t)((ffn + 3) & ~3) * sizeof(float); }

hipError_t gm_allow_quant_lds(const frq_gemma* g) {
    const size_t al = act_quant_lds((int)g->ffn);
    for (hipError_t e : {allow_quant_kernel<1>(al), allow_quant_kernel<2>(al), allow_quant_kernel<3>(al),
                         allow_quant_kernel<4>(al), allow_quant_kernel<5>(al)})
        if (e != hipSuccess) return e;
    return hipSuccess;
}

Q8 gm_q8(frq_gemma* g, int which, size_t k) {
    (void)which;
    return Q8{g->q8f, g->qsa, g->qoi, g->qov, (int)round_up(k, FRQ_KALIGN)};
}

hipError_t launch_act_quant(frq_gemma* g, float c, Q8 q, int* err, hipStream_t s) {
    const int f = (int)g->ffn, silu = g->arch == 1 ? 1 : 0;
    const size_t lds = act_quant_lds(f);
    switch (quant_nv4(g->ffn)) {
        case 1: gm_act_quant_kernel<1><<<1, QNT, lds, s>>>(g->gub, f, c, g->hm, silu, q, err); break;
        case 2: gm_act_quant_kernel<2><<<1, QNT, lds, s>>>(g->gub, f, c, g->hm, silu, q, err); break;
        case 3: gm_act_quant_kernel<3><<<1, QNT, lds, s>>>(g->gub, f, c, g->hm, silu, q, err); break;
        case 4: gm_act_quant_kernel<4><<<1, QNT, lds, s>>>(g->gub, f, c, g->hm, silu, q, err); break;
        case 5: gm_act_quant_kernel<5><<<1, QNT, lds, s>>>(g->gub, f, c, g->hm, silu, q, err); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Points every buffer of the model at nothing and the capacities at zero:
// the state after a failed reserve, so the next call reserves again.
void gm_drop_buffers(frq_gemma* g) {
    if (g->buf) (void)hipFree(g->buf);
    g->buf = nullptr;
    g->cap_pos = g->cap_rows = g->cap_b = 0;
    g->cs = nullptr;
    g->kc = g->vc = g->ks = g->vs = nullptr;
    g->kq = g->vq = nullptr;
    g->x = g->a = g->qkvb = g->att = g->ob = g->gub = g->hm = g->logits = nullptr;
    g->cur = nullptr;
    g->best = nullptr;
    g->tok = g->ids = nullptr;
    g->qr = g->sc = g->xt = nullptr;
    g->pst = g->pmx = nullptr;
    g->q8f = nullptr;
    g->qsa = nullptr;
    g->qoi = nullptr;
    g->qov = nullptr;
}

// Device buffers for up to npos positions and rows prompt rows; the RoPE
// table cos / sin(pos * inv[j]) from the host libm (the reference's f32
// cos / sin).  A request the attention cannot serve is refused before
// anything changes; any later failure leaves the model with no buffers
// (capacities 0), never with pointers into freed memory.
// RP of the two-launch prefill attention for this model (0: not served):
// the f32 cache, 2 <= R <= 8 query heads a kv head, hd a multiple of 32 up
// to 128, and RP - R spare heads' q reads inside the qkv row.
int gm_pf_rp(const frq_gemma* g) {
    const size_t R = g->H / g->KV;
    if (g->kv8 || R < 2 || R > 8 || (g->hd != 32 && g->hd != 64 && g->hd != 128)) return 0;
    const int rp = R <= 2 ? 2 : R <= 4 ? 4 : 8;
    return (size_t)rp <= R + 2 * g->KV ? rp : 0;
}

int gm_reserve(frq_ctx* c, frq_gemma* g, size_t npos, size_t rows, size_t nb = 1) {
    if (npos <= g->cap_pos && rows <= g->cap_rows && nb <= g->cap_b && g->buf) return FRQ_OK;
    const size_t N = std::max(npos, g->cap_pos), R = std::max(rows, g->cap_rows), B = std::max(nb, g->cap_b);
    const size_t need = gm_attn_lds_n(g->hd, N);
    if (need > GM_LDS_MAX)
        return set_error(FRQ_ERR_ARG, "gemma: " + std::to_string(N) +
                                          " positions exceed the attention scores' LDS (" + std::to_string(need) +
                                          " > " + std::to_string(GM_LDS_MAX) + " bytes)");
    hipStream_t s = (hipStream_t)frq_get_stream(c);
    GMCHK(hipStreamSynchronize(s), "hipStreamSynchronize");
    gm_drop_buffers(g);
    GMCHK(gm_allow_lds(need), "hipFuncSetAttribute");
    if (gm_norm_lds((int)g->d) > 64 * 1024)
        GMCHK(hipFuncSetAttribute((const void*)gm_norm_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)gm_norm_lds((int)g->d)),
              "hipFuncSetAttribute(norm)");
    GMCHK(gm_allow_quant_lds(g), "hipFuncSetAttribute(quant)");
    GMCHK(allow_value_blk_lds(gm_pstride_n(N)), "hipFuncSetAttribute(value blocks)");
    const size_t L = g->L, kvd = g->KV * g->hd, half = g->hd / 2;
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off += round_up(bytes, 256); return o; };
    const size_t o_cs = take(N * half * sizeof(float2));
    size_t o_kc, o_vc, o_ks = 0, o_vs = 0;
    if (g->kv8) {
        o_kc = take(L * B * N * kvd); o_vc = take(L * B * N * kvd);
        o_ks = take(L * B * N * g->KV * 4); o_vs = take(L * B * N * g->KV * 4);
    } else {
        o_kc = take(L * B * N * kvd * 4); o_vc = take(L * B * N * kvd * 4);
    }
    const size_t o_x = take(R * g->d * 4), o_a = take(R * g->d * 4),
                 o_qkv = take(R * (g->H + 2 * g->KV) * g->hd * 4), o_att = take(R * g->H * g->hd * 4),
                 o_o = take(R * g->d * 4), o_gu = take(R * 2 * g->ffn * 4), o_hm = take(R * g->ffn * 4),
                 o_lg = take(B * g->vocab * 4), o_cur = take(4), o_best = take(B * 8), o_tok = take(B * N * 8),
                 o_ids = take(R * 8),
                 o_qr = take(g->H * g->hd * 4), o_sc = take(g->H * gm_pstride_n(N) * 4),
                 o_xt = take(B > 1 ? 16 * (std::max({g->d, g->ffn, g->H * g->hd}) + 4) * 4 : 0),
                 o_q8f = take(round_up(g->ffn, FRQ_KALIGN)), o_qsa = take(4), o_qoi = take(FRQ_T * 4),
                 o_qov = take(FRQ_T * 4);
    // the two-launch prefill attention's scores and tile maxima: only for
    // prompts that take it (PF_MIN_ROWS rows or more), and only while the
    // buffer stays within PF_MAX_BYTES (longer prompts take the one-launch
    // kernels, which need no buffer)
    const int rp = gm_pf_rp(g);
    const size_t kpad = pf_kpad(N);
    size_t pf_nrb = (rp && R >= PF_MIN_ROWS) ? (R + pf_rows(rp) - 1) / pf_rows(rp) : 0;
    if (pf_nrb * g->KV * kpad * PF_AP * 4 > PF_MAX_BYTES) pf_nrb = 0;
    const size_t o_pst = take(pf_nrb * g->KV * kpad * PF_AP * 4), o_pmx = take(pf_nrb * g->KV * PF_AP * 4);
    char* m = nullptr;
    GMCHK(hipMalloc(&m, off), "hipMalloc(gemma)");
    if (hipError_t e = hipMemsetAsync(m, 0, off, s)) {
        (void)hipFree(m);
        return gfail(e, "hipMemsetAsync(gemma)");
    }
    std::vector<float2> cs(N * half);
    for (size_t pos = 0; pos < N; ++pos)
        for (size_t j = 0; j < half; ++j) {
            const float ang = (float)pos * g->inv[j];
            cs[pos * half + j] = make_float2(cosf(ang), sinf(ang));
        }
    hipError_t e = hipMemcpyAsync(m + o_cs, cs.data(), cs.size() * sizeof(float2), hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);  // cs is released on return
    if (e != hipSuccess) {
        (void)hipFree(m);
        return gfail(e, "hipMemcpyAsync(gemma RoPE table)");
    }
    g->buf = m;
    g->cap_pos = N;
    g->cap_rows = R;
    g->cap_b = B;
    g->cs = reinterpret_cast<float2*>(m + o_cs);
    g->kc = g->kv8 ? nullptr : reinterpret_cast<float*>(m + o_kc);
    g->vc = g->kv8 ? nullptr : reinterpret_cast<float*>(m + o_vc);
    g->kq = g->kv8 ? reinterpret_cast<int8_t*>(m + o_kc) : nullptr;
    g->vq = g->kv8 ? reinterpret_cast<int8_t*>(m + o_vc) : nullptr;
    g->ks = g->kv8 ? reinterpret_cast<float*>(m + o_ks) : nullptr;
    g->vs = g->kv8 ? reinterpret_cast<float*>(m + o_vs) : nullptr;
    g->x = reinterpret_cast<float*>(m + o_x); g->a = reinterpret_cast<float*>(m + o_a);
    g->qkvb = reinterpret_cast<float*>(m + o_qkv); g->att = reinterpret_cast<float*>(m + o_att);
    g->ob = reinterpret_cast<float*>(m + o_o); g->gub = reinterpret_cast<float*>(m + o_gu);
    g->hm = reinterpret_cast<float*>(m + o_hm); g->logits = reinterpret_cast<float*>(m + o_lg);
    g->cur = reinterpret_cast<int*>(m + o_cur); g->best = reinterpret_cast<unsigned long long*>(m + o_best);
    g->tok = reinterpret_cast<int64_t*>(m + o_tok); g->ids = reinterpret_cast<int64_t*>(m + o_ids);
    g->qr = reinterpret_cast<float*>(m + o_qr); g->sc = reinterpret_cast<float*>(m + o_sc);
    g->xt = B > 1 ? reinterpret_cast<float*>(m + o_xt) : nullptr;
    g->pst = pf_nrb ? reinterpret_cast<float*>(m + o_pst) : nullptr;
    g->pmx = pf_nrb ? reinterpret_cast<float*>(m + o_pmx) : nullptr;
    g->q8f = reinterpret_cast<int8_t*>(m + o_q8f);
    g->qsa = reinterpret_cast<float*>(m + o_qsa); g->qoi = reinterpret_cast<uint32_t*>(m + o_qoi);
    g->qov = reinterpret_cast<float*>(m + o_qov);
    return FRQ_OK;
}

// One step of the model: m prompt rows (rel 0: ids; the prefill) or, rel 1,
// the decode row of the last token; batch > 0: m = batch rows, row i the
// decode row of sequence i, every sequence at the same position (logits
// row i at logits_out + i los).
int gm_block(frq_ctx* c, frq_gemma* g, size_t m, int rel, int P, float* logits_out, int batch = 0,
             size_t los = 0) {
    hipStream_t s = (hipStream_t)frq_get_stream(c);
    const int d = (int)g->d, H = (int)g->H, KV = (int)g->KV, hd = (int)g->hd, ffn = (int)g->ffn;
    const Weight& et = *weight_of(g->embed);
    const size_t nlds = gm_norm_lds(d);
    int* err = ctx_err(c);
    auto is_i8 = [&](const frq_w* w) { return weight_of(w)->dtype == FRQ_DT_I8; };
    // one decode row of an int8 down linear takes its quant from the
    // activation kernel
    const bool q8f = m == 1 && !batch && quant_nv4(g->ffn) > 0;
    // A batch step's int4 linears read their rows in the k-quad interleaved
    // layout, which the kernel producing those rows also writes (into the
    // staging rows xt): a4_for(w) is where, or NULL when w does not take it.
    auto a4_for = [&](const frq_w* w) -> float* {
        return batch && m <= 16 && g->xt && weight_of(w)->dtype == FRQ_DT_I4 && i4_rows_a4_ok(*weight_of(w))
                   ? g->xt
                   : nullptr;
    };
    auto norm = [&](const float* y, const float* wpost, const float* wnext, int rows, int row0, float* a4) {
        const size_t n2 = gm_norm2_lds(d);
        switch ((d / 4 + NORM_NT - 1) / NORM_NT) {
            case 1: gm_norm2_kernel<1, NORM_NT><<<dim3(rows), dim3(NORM_NT), n2, s>>>(g->x, y, wpost, wnext, g->a, d, g->eps, row0, a4); break;
            case 2: gm_norm2_kernel<2, NORM_NT><<<dim3(rows), dim3(NORM_NT), n2, s>>>(g->x, y, wpost, wnext, g->a, d, g->eps, row0, a4); break;
            case 3: gm_norm2_kernel<3, NORM_NT><<<dim3(rows), dim3(NORM_NT), n2, s>>>(g->x, y, wpost, wnext, g->a, d, g->eps, row0, a4); break;
            case 4: gm_norm2_kernel<4, NORM_NT><<<dim3(rows), dim3(NORM_NT), n2, s>>>(g->x, y, wpost, wnext, g->a, d, g->eps, row0, a4); break;
            default: gm_norm_kernel<<<dim3(rows), dim3(NORM_NT), nlds, s>>>(g->x, y, wpost, wnext, g->a, d, g->eps, row0, a4);
        }
        return hipGetLastError();
    };
    // the linears: in a batch step each row is its own sequence's decode row;
    // a4 set: the rows are already staged there (a4_for)
    auto mm = [&](const frq_w* w, const float* in, float* outp, const float* a4) -> int {
        if (!batch) return gm_mm(c, w, in, m, outp);
        if (a4) {
            GMCHK(launch_i4_rows_a4(*weight_of(w), m, a4, outp, s), "launch i4 rows");
            return FRQ_OK;
        }
        return gm_mm_rows(c, w, in, m, outp, g->xt);
    };
    int64_t* tokp = g->tok + g->seq * g->cap_pos;  // this sequence's tokens (batch: sequence 0's)
    gm_embed_kernel<<<dim3((unsigned)m), dim3(GT), 0, s>>>(et.rowp, et.rpitch, et.dtype, et.scale, d, g->escale,
                                                           rel ? tokp : g->ids, rel, P, g->cur, g->x,
                                                           batch ? g->cap_pos : 0);
    GMCHK(hipGetLastError(), "launch embed");
    GMCHK(norm(nullptr, nullptr, g->norm_of(0, 0), (int)m, 0, a4_for(g->qkv[0])), "launch norm");
    const size_t kvd = g->KV * g->hd;
    // the caches: [layer][sequence][position][kv width]; a batch step's row i
    // is sequence i (bst elements further per row)
    const size_t bst = g->cap_pos * kvd;
    for (size_t l = 0; l < g->L; ++l) {
        if (int rc = mm(g->qkv[l], g->a, g->qkvb, a4_for(g->qkv[l]))) return rc;
        const size_t cb = (l * g->cap_b + g->seq) * g->cap_pos;  // this layer's (and sequence's) first position
        float* kc0 = g->kv8 ? nullptr : g->kc + cb * kvd;
        float* vc0 = g->kv8 ? nullptr : g->vc + cb * kvd;
        int8_t* kq0 = g->kv8 ? g->kq + cb * kvd : nullptr;
        int8_t* vq0 = g->kv8 ? g->vq + cb * kvd : nullptr;
        float* ks0 = g->kv8 ? g->ks + cb * g->KV : nullptr;
        float* vs0 = g->kv8 ? g->vs + cb * g->KV : nullptr;
        float *kc = kc0, *vc = vc0, *ks = ks0, *vs = vs0;
        int8_t *kq = kq0, *vq = vq0;
        const dim3 ag((unsigned)H, (unsigned)m);
        const size_t lds = gm_attn_lds(g);
        const int ps = (int)gm_pstride(g), sl = (g->arch == 0 && l % 2 == 0) ? 1 : 0, win = (int)g->window;
        const float* qb = g->bias_of(l);
        const float* qn = g->qn_of(l);
        const float* kn = g->kn_of(l);
        const int div = g->arch == 1;
        // the one-launch decode attention also stages o's rows
        float* a4o = (m == 1 || batch) && g->cap_pos <= 512 ? a4_for(g->o[l]) : nullptr;
        if ((m == 1 || batch) && g->cap_pos > 512) {  // long caches: the three-launch decode attention
          for (size_t bi = 0; bi < m; ++bi) {  // (a batch: each sequence in turn, on its own cache)
            const int hd4 = (hd + 3) & ~3;
            const size_t plds = (size_t)2 * hd4 * sizeof(float);
            const dim3 sg((unsigned)H, (unsigned)((g->cap_pos + GT - 1) / GT));
            const size_t vlds = ((size_t)2 * ps + seq_sum_spec_scratch(GT)) * sizeof(float);
            float* qkvr = g->qkvb + bi * (H + 2 * KV) * hd;
            float* attr = g->att + bi * H * hd;
            float* kc = kc0 ? kc0 + bi * bst : nullptr;
            float* vc = vc0 ? vc0 + bi * bst : nullptr;
            int8_t* kq = kq0 ? kq0 + bi * bst : nullptr;
            int8_t* vq = vq0 ? vq0 + bi * bst : nullptr;
            float* ks = ks0 ? ks0 + bi * (bst / hd) : nullptr;
            float* vs = vs0 ? vs0 + bi * (bst / hd) : nullptr;
            if (g->kv8) {
                gm_dec_prep_kernel<true><<<dim3((unsigned)(H + KV)), dim3(GT), plds, s>>>(
                    qkvr, H, KV, hd, g->cur, g->cs, kc, vc, kq, vq, ks, vs, qb, qn, kn, g->eps, g->qr);
                gm_dec_score_kernel<true><<<sg, dim3(GT), hd4 * sizeof(float), s>>>(
                    g->qr, H, KV, hd, g->cur, kc, kq, ks, g->qscale, g->cap, sl, win, div, ps, g->sc);
                const hipError_t er = launch_value_blk(g, sl, win, ps, vc, vq, vs, attr, s);
                if (er == hipErrorNotSupported)
                    gm_dec_value_kernel<true><<<dim3((unsigned)H), dim3(GT), vlds, s>>>(g->sc, H, KV, hd, g->cur, vc,
                                                                                        vq, vs, sl, win, ps, attr);
                else
                    GMCHK(er, "launch value blocks");
            } else {
                if (hd == 128 || hd == 64 || hd == 32) {  // prep fused into the scores
                    auto qk = hd == 128 ? gm_dec_qks_kernel<128> : hd == 64 ? gm_dec_qks_kernel<64> : gm_dec_qks_kernel<32>;
                    qk<<<sg, dim3(GT), 0, s>>>(qkvr, H, KV, g->cur, g->cs, kc, vc, qb, qn, kn, g->eps, g->qscale,
                                               g->cap, sl, win, div, ps, g->sc);
                } else {
                    gm_dec_prep_kernel<false><<<dim3((unsigned)(H + KV)), dim3(GT), plds, s>>>(
                        qkvr, H, KV, hd, g->cur, g->cs, kc, vc, kq, vq, ks, vs, qb, qn, kn, g->eps, g->qr);
                    gm_dec_score_kernel<false><<<sg, dim3(GT), hd4 * sizeof(float), s>>>(
                        g->qr, H, KV, hd, g->cur, kc, kq, ks, g->qscale, g->cap, sl, win, div, ps, g->sc);
                }
                const hipError_t er = launch_value_blk(g, sl, win, ps, vc, vq, vs, attr, s);
                if (er == hipErrorNotSupported)
                    gm_dec_value_kernel<false><<<dim3((unsigned)H), dim3(GT), vlds, s>>>(g->sc, H, KV, hd, g->cur,
                                                                                         vc, vq, vs, sl, win, ps,
                                                                                         attr);
                else
                    GMCHK(er, "launch value blocks");
            }
          }
        } else if (m == 1 || batch) {
            const long long bs = batch ? (long long)bst : 0;
            if (g->kv8)
                gm_attn_kernel<true, true><<<ag, dim3(GT), lds, s>>>(g->qkvb, H, KV, hd, g->cur, g->cs, kc, vc, kq,
                                                                     vq, ks, vs, g->qscale, g->cap, sl, win, ps,
                                                                     g->att, div, qb, qn, kn, g->eps, bs, a4o);
            else
                gm_attn_kernel<false, true><<<ag, dim3(GT), lds, s>>>(g->qkvb, H, KV, hd, g->cur, g->cs, kc, vc, kq,
                                                                      vq, ks, vs, g->qscale, g->cap, sl, win, ps,
                                                                      g->att, div, qb, qn, kn, g->eps, bs, a4o);
        } else {
            if (g->kv8)
                gm_qkv_kernel<true><<<dim3((unsigned)m), dim3(GT), 0, s>>>(g->qkvb, H, KV, hd, g->cur, g->cs, kc, vc,
                                                                           kq, vq, ks, vs, qb, qn, kn, g->eps);
            else
                gm_qkv_kernel<false><<<dim3((unsigned)m), dim3(GT), 0, s>>>(g->qkvb, H, KV, hd, g->cur, g->cs, kc,
                                                                            vc, kq, vq, ks, vs, qb, qn, kn, g->eps);
            GMCHK(hipGetLastError(), "launch qkv");
            // the heads of a kv group in one workgroup where the shape and LDS allow
            const int R = H / KV;
            const size_t glds = ((size_t)R * (((size_t)hd + 3) & ~(size_t)3) + (size_t)R * ps + (g->kv8 ? (size_t)ps : 0)) * sizeof(float);
            const bool grouped = R > 1 && R <= 16 && GT % hd == 0 && R <= 4 * (GT / hd) && glds + 1024 <= 160 * 1024 &&
                                 m <= 65535;
            // the register-tiled kernel for the f32 cache: p rows prow apart
            // (prow % 64 == 4), RP >= R query heads a lane
            const size_t prow = (ps + 59) / 64 * 64 + 4;
            const int RP = R <= 2 ? 2 : R <= 4 ? 4 : 8;
            const size_t tlds = (size_t)RP * prow * sizeof(float);
            const bool tiled = !g->kv8 && R > 1 && R <= 8 && hd % 32 == 0 && hd <= 2 * GT && RP <= R + 2 * KV &&
                               tlds + 1024 <= GM_LDS_MAX && m <= 65535;
            const int prp = gm_pf_rp(g);
            if (prp && g->pst && m >= PF_MIN_ROWS && m <= 65535) {
                // the two-launch form: each key / value row read once a block of rows
                const int nrb = (int)((m + pf_rows(prp) - 1) / pf_rows(prp));
                const int kpad = (int)pf_kpad(g->cap_pos), nkt = kpad / PF_KT;
                GMCHK(launch_pf_attention(prp, hd, g->qkvb, H, KV, g->cur, (int)m, kc, vc, g->qscale, g->cap, sl, win,
                                          nrb, nkt, kpad, g->pst, g->pmx, g->att, div, s),
                      "launch prefill attention");
            } else if (tiled) {
                auto kern = RP == 2 ? gm_attn_tile_kernel<2> : RP == 4 ? gm_attn_tile_kernel<4> : gm_attn_tile_kernel<8>;
                if (tlds > 64 * 1024)
                    GMCHK(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                              (int)tlds),
                          "hipFuncSetAttribute");
                kern<<<dim3((unsigned)KV, (unsigned)m), dim3(GT), tlds, s>>>(g->qkvb, H, KV, hd, g->cur, kc, vc,
                                                                             g->qscale, g->cap, sl, win, (int)prow,
                                                                             g->att, div);
            } else if (grouped) {
                auto kern = g->kv8 ? gm_attn_group_kernel<true> : gm_attn_group_kernel<false>;
                if (glds > 64 * 1024)
                    GMCHK(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                              (int)glds),
                          "hipFuncSetAttribute");
                kern<<<dim3((unsigned)KV, (unsigned)m), dim3(GT), glds, s>>>(g->qkvb, H, KV, hd, g->cur, kc, vc, kq,
                                                                             vq, ks, vs, g->qscale, g->cap, sl, win,
                                                                             ps, g->att, div);
            } else if (g->kv8)
                gm_attn_kernel<true, false><<<ag, dim3(GT), lds, s>>>(g->qkvb, H, KV, hd, g->cur, g->cs, kc, vc, kq,
                                                                      vq, ks, vs, g->qscale, g->cap, sl, win, ps,
                                                                      g->att, div, nullptr, nullptr, nullptr, g->eps);
            else
                gm_attn_kernel<false, false><<<ag, dim3(GT), lds, s>>>(g->qkvb, H, KV, hd, g->cur, g->cs, kc, vc,
                                                                       kq, vq, ks, vs, g->qscale, g->cap, sl, win,
                                                                       ps, g->att, div, nullptr, nullptr, nullptr,
                                                                       g->eps);
        }
        GMCHK(hipGetLastError(), "launch attention");
        if (int rc = mm(g->o[l], g->att, g->ob, a4o)) return rc;
        GMCHK(norm(g->ob, g->post_of(l, 1), g->norm_of(l, 2), (int)m, 0, a4_for(g->gu[l])), "launch norm");
        const float gc = sqrtf(2.0f / 3.14159274101257324f);
        // rows the fused quant + GEMV covers take the elementwise act, then
        // that linear (an act inside it would be recomputed by every one of
        // its workgroups); longer int8 rows the act + quant kernel, then the
        // GEMV on the quantised row
        const bool down_q = q8f && is_i8(g->down[l]) && !linear_m1_ok(*weight_of(g->down[l]), g->hm);
        // one decode row of an int8 gate|up pair otherwise: the activation in
        // the fused linear's epilogue (no separate act launch)
        const int hr = g->gu_hr[l];
        const bool act_fused = m == 1 && !batch && !down_q && hr && linear_m1_act_ok(*weight_of(g->gu[l]), g->a, hr);
        if (act_fused)
            GMCHK(launch_linear_m1_act(*weight_of(g->gu[l]), g->a, g->hm, hr, g->arch == 1 ? 1 : 0, gc, err, s),
                  "launch gate|up + act");
        else if (int rc = mm(g->gu[l], g->a, g->gub, a4_for(g->gu[l])))
            return rc;
        if (down_q) {
            const Q8 q = gm_q8(g, 1, g->ffn);
            GMCHK(launch_act_quant(g, gc, q, err, s), "launch act + quant");
            if (int rc = frq_mm_i8_q_dev(c, g->down[l], q.a8, q.sa, q.oi, q.ov, 1, g->ob)) return rc;
        } else {
            if (!act_fused) {
                const size_t tot = m * g->ffn, items = g->arch == 1 && g->ffn % 4 == 0 && m >= 16 ? tot / 4 : tot;
                gm_geglu_kernel<<<dim3((unsigned)std::min<size_t>((items + GT - 1) / GT, 4096)), dim3(GT), 0, s>>>(
                    g->gub, ffn, tot, gc, g->hm, g->arch == 1 ? 1 : 0, hr, a4_for(g->down[l]));
                GMCHK(hipGetLastError(), "launch geglu");
            }
            if (int rc = mm(g->down[l], g->hm, g->ob, a4_for(g->down[l]))) return rc;
        }
        if (l + 1 < g->L)
            GMCHK(norm(g->ob, g->post_of(l, 3), g->norm_of(l + 1, 0), (int)m, 0, a4_for(g->qkv[l + 1])),
                  "launch norm");
        else if (batch)  // every sequence's row feeds the head
            GMCHK(norm(g->ob, g->post_of(l, 3), g->final_norm(), (int)m, 0, nullptr), "launch norm");
        else  // only the last row feeds the head
            GMCHK(norm(g->ob, g->post_of(l, 3), g->final_norm(), 1, (int)m - 1, nullptr), "launch norm");
    }
    float* lg = logits_out ? logits_out : g->logits;
    const Weight& ut = g->unembed ? *weight_of(g->unembed) : et;
    if (batch) {
        GMCHK(launch_rowdot_argmax_batch(ut, m, g->a, g->d, g->xt, lg, logits_out ? los : g->vocab, g->best, err, s),
              "launch unembed");
        gm_argmax_batch_kernel<<<dim3(1), dim3(64), 0, s>>>(g->best, g->cur, (int)m, P, g->tok, (int)g->cap_pos);
    } else {
        GMCHK(launch_rowdot_argmax(ut, g->a + (m - 1) * g->d, lg, g->best, err, s), "launch unembed");
        gm_argmax_done_kernel<<<dim3(1), dim3(64), 0, s>>>(g->best, g->cur, (int)m, P, tokp);
    }
    GMCHK(hipGetLastError(), "launch argmax");
    return FRQ_OK;
}

int gm_run(frq_ctx* c, frq_gemma* g, const int64_t* prompt, size_t P, size_t n_new, int64_t* out, float* logits) {
    if (!c || !g) return set_error(FRQ_ERR_ARG, "null context / model");
    if (ctx_device(c) != g->device) return set_error(FRQ_ERR_ARG, "model lives on another device");
    if (!P || !n_new) return set_error(FRQ_ERR_ARG, "empty prompt or no tokens asked for");
    if (!prompt || !out) return set_error(FRQ_ERR_ARG, "null prompt / output");
    for (size_t i = 0; i < P; ++i)
        if (prompt[i] < 0 || (size_t)prompt[i] >= g->vocab)
            return set_error(FRQ_ERR_ARG, "token id " + std::to_string(prompt[i]) + " beyond the vocabulary");
    GDev dv(g->device);
    if (int rc = gm_reserve(c, g, P + n_new, P)) return rc;
    hipStream_t s = (hipStream_t)frq_get_stream(c);
    float* lgd = nullptr;
    if (logits) GMCHK(hipMalloc(&lgd, n_new * g->vocab * sizeof(float)), "hipMalloc(logits)");
    struct Free {
        float* p;
        ~Free() { if (p) (void)hipFree(p); }
    } fr{lgd};
    GMCHK(hipMemcpyAsync(g->ids, prompt, P * sizeof(int64_t), hipMemcpyHostToDevice, s), "hipMemcpyAsync(prompt)");
    GMCHK(hipMemsetAsync(g->cur, 0, sizeof(int), s), "hipMemsetAsync(cur)");
    if (int rc = gm_block(c, g, P, 0, (int)P, lgd)) return rc;
    if (g->graphs && !logits && n_new > 2 && s != nullptr) {
        hipGraph_t gr = nullptr;
        hipGraphExec_t ex = nullptr;
        GMCHK(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
        const int rc = gm_block(c, g, 1, 1, (int)P, nullptr);
        const hipError_t e = hipStreamEndCapture(s, &gr);
        if (rc) { if (gr) (void)hipGraphDestroy(gr); return rc; }
        GMCHK(e, "hipStreamEndCapture");
        const hipError_t ei = hipGraphInstantiate(&ex, gr, nullptr, nullptr, 0);
        (void)hipGraphDestroy(gr);
        GMCHK(ei, "hipGraphInstantiate");
        hipError_t el = hipSuccess;
        for (size_t t = 1; t < n_new && el == hipSuccess; ++t) el = hipGraphLaunch(ex, s);
        (void)hipGraphExecDestroy(ex);
        GMCHK(el, "hipGraphLaunch");
    } else {
        for (size_t t = 1; t < n_new; ++t)
            if (int rc = gm_block(c, g, 1, 1, (int)P, lgd ? lgd + t * g->vocab : nullptr)) return rc;
    }
    GMCHK(hipMemcpyAsync(out, g->tok, n_new * sizeof(int64_t), hipMemcpyDeviceToHost, s), "hipMemcpyAsync(tokens)");
    if (logits)
        GMCHK(hipMemcpyAsync(logits, lgd, n_new * g->vocab * sizeof(float), hipMemcpyDeviceToHost, s),
              "hipMemcpyAsync(logits)");
    return frq_sync(c);
}

// nb sequences (prompts nb x P), each its own Model::generate: every
// sequence prefilled alone on its own cache, then the decode steps of all nb
// at once, row i of a step being sequence i's.  Tokens out (nb x n_new),
// logits (nb x n_new x vocab) as nb calls of gm_run give them.
int gm_run_batch(frq_ctx* c, frq_gemma* g, const int64_t* prompts, size_t nb, size_t P, size_t n_new, int64_t* out,
                 float* logits) {
    if (!c || !g) return set_error(FRQ_ERR_ARG, "null context / model");
    if (ctx_device(c) != g->device) return set_error(FRQ_ERR_ARG, "model lives on another device");
    if (!nb || !P || !n_new) return set_error(FRQ_ERR_ARG, "no sequence, empty prompt or no tokens asked for");
    if (!prompts || !out) return set_error(FRQ_ERR_ARG, "null prompts / output");
    if (nb > 65535) return set_error(FRQ_ERR_ARG, "too many sequences");
    for (size_t i = 0; i < nb * P; ++i)
        if (prompts[i] < 0 || (size_t)prompts[i] >= g->vocab)
            return set_error(FRQ_ERR_ARG, "token id " + std::to_string(prompts[i]) + " beyond the vocabulary");
    GDev dv(g->device);
    if (int rc = gm_reserve(c, g, P + n_new, std::max(P, nb), nb)) return rc;
    hipStream_t s = (hipStream_t)frq_get_stream(c);
    const size_t V = g->vocab;
    float* lgd = nullptr;
    if (logits) GMCHK(hipMalloc(&lgd, nb * n_new * V * sizeof(float)), "hipMalloc(logits)");
    struct Free {
        float* p;
        ~Free() { if (p) (void)hipFree(p); }
    } fr{lgd};
    struct Seq0 {  // one-sequence calls of gm_block use sequence seq
        frq_gemma* g;
        ~Seq0() { g->seq = 0; }
    } sq{g};
    for (size_t b = 0; b < nb; ++b) {
        g->seq = b;
        GMCHK(hipMemcpyAsync(g->ids, prompts + b * P, P * sizeof(int64_t), hipMemcpyHostToDevice, s),
              "hipMemcpyAsync(prompt)");
        GMCHK(hipMemsetAsync(g->cur, 0, sizeof(int), s), "hipMemsetAsync(cur)");
        if (int rc = gm_block(c, g, P, 0, (int)P, lgd ? lgd + b * n_new * V : nullptr)) return rc;
    }
    g->seq = 0;
    const int B = (int)nb;
    if (g->graphs && !logits && n_new > 2 && s != nullptr) {
        hipGraph_t gr = nullptr;
        hipGraphExec_t ex = nullptr;
        GMCHK(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
        const int rc = gm_block(c, g, nb, 1, (int)P, nullptr, B, 0);
        const hipError_t e = hipStreamEndCapture(s, &gr);
        if (rc) { if (gr) (void)hipGraphDestroy(gr); return rc; }
        GMCHK(e, "hipStreamEndCapture");
        const hipError_t ei = hipGraphInstantiate(&ex, gr, nullptr, nullptr, 0);
        (void)hipGraphDestroy(gr);
        GMCHK(ei, "hipGraphInstantiate");
        hipError_t el = hipSuccess;
        for (size_t t = 1; t < n_new && el == hipSuccess; ++t) el = hipGraphLaunch(ex, s);
        (void)hipGraphExecDestroy(ex);
        GMCHK(el, "hipGraphLaunch");
    } else {
        for (size_t t = 1; t < n_new; ++t)
            if (int rc = gm_block(c, g, nb, 1, (int)P, lgd ? lgd + t * V : nullptr, B, n_new * V)) return rc;
    }
    GMCHK(hipMemcpy2DAsync(out, n_new * sizeof(int64_t), g->tok, g->cap_pos * sizeof(int64_t),
                           n_new * sizeof(int64_t), nb, hipMemcpyDeviceToHost, s),
          "hipMemcpy2DAsync(tokens)");
    if (logits)
        GMCHK(hipMemcpyAsync(logits, lgd, nb * n_new * V * sizeof(float), hipMemcpyDeviceToHost, s),
              "hipMemcpyAsync(logits)");
    return frq_sync(c);
}

float f16_host(uint16_t h) {
    const uint32_t sg = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, mt = h & 1023;
    uint32_t bits;
    if (e == 0) {
        if (!mt) bits = sg;
        else {
            int sh = 0;
            uint32_t mm = mt;
            while (!(mm & 1024)) { mm <<= 1; ++sh; }
            bits = sg | ((uint32_t)(113 - sh) << 23) | ((mm & 1023) << 13);
        }
    } else if (e == 31) {
        bits = sg | 0x7F800000u | (mt << 13);
    } else {
        bits = sg | ((e + 112) << 23) | (mt << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

int norm_vec(const frq_bundle* b, const std::string& name, size_t d, float* dst) {
    char dt[16];
    size_t shape[4], nd = 4, grp = 0, bytes = 0;
    const void* data = nullptr;
    if (int rc = frq_bundle_array(b, name.c_str(), dt, sizeof dt, shape, &nd, &grp, &data, &bytes)) return rc;
    const std::string t = dt;
    if (nd != 1 || shape[0] != d || (t != "f16" && t != "f32"))
        return set_error(FRQ_ERR_FORMAT, name + ": expected " + std::to_string(d) + " f16 / f32 values");
    if (t == "f32") std::memcpy(dst, data, d * 4);
    else for (size_t i = 0; i < d; ++i) dst[i] = f16_host(static_cast<const uint16_t*>(data)[i]);
    return FRQ_OK;
}

}  // namespace

extern "C" {

static int decoder_load(frq_ctx* c, const frq_bundle* b, int kv_int8, int want_arch, frq_gemma** out) {
    if (!out) return set_error(FRQ_ERR_ARG, "null output handle");
    *out = nullptr;
    if (!c || !b) return set_error(FRQ_ERR_ARG, "null context / bundle");
    char arch[32];
    int64_t cfg[8];
    double cff[8];
    size_t nc = 8, nf = 8;
    if (int rc = frq_bundle_header(b, arch, sizeof arch, cfg, &nc, cff, &nf)) return rc;
    const char* name = want_arch == 0 ? "gemma" : "rope";
    if (std::string(arch) != name)
        return set_error(FRQ_ERR_FORMAT, std::string("not a ") + name + " bundle: " + arch);
    if (nc < 8 || nf < (want_arch == 0 ? 6u : 2u))
        return set_error(FRQ_ERR_FORMAT, want_arch == 0
                                             ? "gemma config needs [n_layer, H, nkv, hd, d, ffn, vocab, tied] and "
                                               "config_f [theta, eps, attn_cap, final_cap, qscalar, escale]"
                                             : "rope config needs [n_layer, H, nkv, hd, d, ffn, vocab, tied] and "
                                               "config_f [theta, eps]");
    for (int i = 0; i < 7; ++i)
        if (cfg[i] <= 0) return set_error(FRQ_ERR_FORMAT, "gemma config entries must be positive");
    auto g = std::make_unique<frq_gemma>();
    g->device = ctx_device(c);
    g->L = cfg[0]; g->H = cfg[1]; g->KV = cfg[2]; g->hd = cfg[3]; g->d = cfg[4]; g->ffn = cfg[5]; g->vocab = cfg[6];
    g->kv8 = kv_int8 ? 1 : 0;
    g->arch = want_arch;
    // a head's scores are one a.dot block (hd <= MM_KC): a single FMA chain
    if (g->H % g->KV || g->hd % 4 || g->d % 4 || g->d > 8192 || g->hd > (size_t)MM_KC)
        return set_error(FRQ_ERR_ARG, "gemma shape outside this build's kernels (H % nkv, head dim and d % 4, "
                                      "head dim <= 256, d <= 8192)");
    // Gemma::new (52-60): f32 of the f64 config values; RoPE frequencies and
    // the query scale through the host libm's powf, as the reference
    const float theta = (float)cff[0];
    g->theta = theta; g->eps = (float)cff[1];
    if (want_arch == 0) {
        g->cap = (float)cff[2]; g->escale = (float)cff[5];
        g->qscale = powf((float)cff[4], -0.5f);
    } else {  // Rope::new (rope.rs:56-64): scores / sqrt(hd), no scale, no soft-cap
        g->cap = 0.0f; g->escale = 1.0f;
        g->qscale = sqrtf((float)g->hd);
    }
    for (size_t j = 0; j < g->hd / 2; ++j) g->inv.push_back(1.0f / powf(theta, 2.0f * (float)j / (float)g->hd));
    const size_t L = g->L, d = g->d, qd = g->H * g->hd, kvd = g->KV * g->hd;
    (void)kvd;
    for (size_t l = 0; l < L; ++l) {
        const std::string p = "l" + std::to_string(l) + ".";
        frq_w* w = nullptr;
        if (int rc = concat_linear(c, b, {p + "self_attn.q_proj", p + "self_attn.k_proj", p + "self_attn.v_proj"}, d, &w))
            return rc;
        g->qkv.push_back(w);
        if (int rc = one_linear(c, b, p + "self_attn.o_proj", qd, d, &w)) return rc;
        g->o.push_back(w);
        // the decode row of an int8 pair takes the fused linear with the
        // activation in its epilogue where both linears fit the fused form
        // (d and ffn multiples of 4 in (32, 20480]): rows in runs of its RPP / 2
        const bool fuse = g->d % 4 == 0 && g->d > 32 && round_up(g->d, 128) <= 20480 && g->ffn % 4 == 0 &&
                          g->ffn > 32 && round_up(g->ffn, 128) <= 20480;
        const size_t hr = fuse ? (size_t)linear_m1_rpp(round_up(g->d, 128), 2 * g->ffn) / 2 : 0;
        int ghr = 0;
        if (int rc = concat_linear(c, b, {p + "mlp.gate_proj", p + "mlp.up_proj"}, d, &w, hr, &ghr)) return rc;
        g->gu.push_back(w);
        g->gu_hr.push_back(ghr);
        if (int rc = one_linear(c, b, p + "mlp.down_proj", g->ffn, d, &w)) return rc;
        g->down.push_back(w);
    }
    auto table = [&](const char* nm, frq_w** w) -> int {
        if (int rc = frq_bundle_weight(c, b, nm, w)) return rc;
        int dt = 0;
        size_t n = 0, k = 0, gg = 0;
        (void)frq_w_info(*w, &dt, &n, &k, &gg);
        if ((dt != FRQ_DT_F16 && dt != FRQ_DT_F32 && dt != FRQ_DT_ROWI8) || n != g->vocab || k != d)
            return set_error(FRQ_ERR_FORMAT, std::string(nm) + ": expected an f32, f16 or rowi8 (vocab, d) table");
        return FRQ_OK;
    };
    if (int rc = table("embed", &g->embed)) return rc;
    // the unembed: gemma ties it; rope reads lm_head unless tied (rope.rs:306-308)
    if (want_arch == 1 && cfg[7] == 0)
        if (int rc = table("lm_head", &g->unembed)) return rc;
    std::vector<float> hv((4 * L + 1) * d, 0.0f);
    static const char* nn[4] = {"input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                                "post_feedforward_layernorm"};
    static const char* rn[4] = {"in_ln", nullptr, "post_ln", nullptr};
    for (size_t l = 0; l < L; ++l)
        for (int j = 0; j < 4; ++j) {
            const char* nm = want_arch == 0 ? nn[j] : rn[j];
            if (nm)
                if (int rc = norm_vec(b, "l" + std::to_string(l) + "." + nm, d, &hv[(4 * l + j) * d])) return rc;
        }
    if (int rc = norm_vec(b, "norm", d, &hv[4 * L * d])) return rc;
    // rope: q / k / v biases (Qwen2.5) and the per-head q / k norms (Qwen3),
    // all present or all absent per kind
    std::vector<float> bias, qkn;
    auto has = [&](const std::string& nm) {
        size_t nd = 0;
        return frq_bundle_array(b, nm.c_str(), nullptr, 0, nullptr, &nd, nullptr, nullptr, nullptr) == FRQ_OK;
    };
    if (want_arch == 1 && has("l0.self_attn.q_proj.bias")) {
        const size_t w = (g->H + 2 * g->KV) * g->hd;
        bias.assign(L * w, 0.0f);
        for (size_t l = 0; l < L; ++l) {
            const std::string p = "l" + std::to_string(l) + ".self_attn.";
            if (int rc = norm_vec(b, p + "q_proj.bias", g->H * g->hd, &bias[l * w])) return rc;
            if (int rc = norm_vec(b, p + "k_proj.bias", g->KV * g->hd, &bias[l * w + g->H * g->hd])) return rc;
            if (int rc = norm_vec(b, p + "v_proj.bias", g->KV * g->hd, &bias[l * w + (g->H + g->KV) * g->hd]))
                return rc;
        }
    }
    if (want_arch == 1 && has("l0.self_attn.q_norm")) {
        qkn.assign(L * 2 * g->hd, 0.0f);
        for (size_t l = 0; l < L; ++l) {
            const std::string p = "l" + std::to_string(l) + ".self_attn.";
            if (int rc = norm_vec(b, p + "q_norm", g->hd, &qkn[l * 2 * g->hd])) return rc;
            if (int rc = norm_vec(b, p + "k_norm", g->hd, &qkn[l * 2 * g->hd + g->hd])) return rc;
        }
    }
    GDev dv(g->device);
    hipStream_t s = (hipStream_t)frq_get_stream(c);
    auto up = [&](const std::vector<float>& v, float** dst) -> int {
        if (v.empty()) return FRQ_OK;
        GMCHK(hipMalloc(dst, v.size() * 4), "hipMalloc(vectors)");
        GMCHK(hipMemcpyAsync(*dst, v.data(), v.size() * 4, hipMemcpyHostToDevice, s), "hipMemcpyAsync(vectors)");
        return FRQ_OK;
    };
    if (int rc = up(hv, &g->norms)) return rc;
    if (int rc = up(bias, &g->qkvbias)) return rc;
    if (int rc = up(qkn, &g->qknorm)) return rc;
    GMCHK(hipStreamSynchronize(s), "hipStreamSynchronize");
    *out = g.release();
    return FRQ_OK;
}

int frq_gemma_load(frq_ctx* c, const frq_bundle* b, int kv_int8, frq_gemma** out) {
    return decoder_load(c, b, kv_int8, 0, out);
}

int frq_rope_load(frq_ctx* c, const frq_bundle* b, int kv_int8, frq_gemma** out) {
    return decoder_load(c, b, kv_int8, 1, out);
}

void frq_gemma_free(frq_gemma* g) { delete g; }

int frq_gemma_set_graphs(frq_gemma* g, int on) {
    if (!g) return set_error(FRQ_ERR_ARG, "null model");
    g->graphs = on ? 1 : 0;
    return FRQ_OK;
}

int frq_gemma_info(const frq_gemma* g, size_t* n_layer, size_t* d, size_t* vocab) {
    if (!g) return set_error(FRQ_ERR_ARG, "null model");
    if (n_layer) *n_layer = g->L;
    if (d) *d = g->d;
    if (vocab) *vocab = g->vocab;
    return FRQ_OK;
}

int frq_gemma_generate(frq_ctx* c, frq_gemma* g, const int64_t* prompt, size_t n_prompt, size_t n_new,
                       int64_t* out, float* logits) {
    return gm_run(c, g, prompt, n_prompt, n_new, out, logits);
}

int frq_gemma_predict(frq_ctx* c, frq_gemma* g, const int64_t* ids, size_t n, int64_t* token, float* logits) {
    return gm_run(c, g, ids, n, 1, token, logits);
}

int frq_mm_exact_dev(frq_ctx* c, const frq_w* w, const float* d_a, size_t m, float* d_out) {
    if (!c) return set_error(FRQ_ERR_ARG, "null context");
    if (!w) return set_error(FRQ_ERR_ARG, "null weight");
    const Weight& ww = *weight_of(w);
    if (ww.dtype != FRQ_DT_I8 && ww.dtype != FRQ_DT_I4 && ww.dtype != FRQ_DT_Q4A)
        return set_error(FRQ_ERR_DTYPE, "frq_mm_exact_dev: not a linear weight");
    if (ww.device != ctx_device(c)) return set_error(FRQ_ERR_ARG, "weight lives on another device");
    if (m == 0 || ww.n == 0) return FRQ_OK;
    if (!d_a || !d_out) return set_error(FRQ_ERR_ARG, "null activation/output pointer");
    GDev dv(ctx_device(c));
    return gm_mm(c, w, d_a, m, d_out);
}

int frq_mm_rows_dev(frq_ctx* c, const frq_w* w, const float* d_a, size_t m, float* d_out) {
    if (!c) return set_error(FRQ_ERR_ARG, "null context");
    if (!w) return set_error(FRQ_ERR_ARG, "null weight");
    const Weight& ww = *weight_of(w);
    if (ww.dtype != FRQ_DT_I8 && ww.dtype != FRQ_DT_I4 && ww.dtype != FRQ_DT_Q4A)
        return set_error(FRQ_ERR_DTYPE, "frq_mm_rows_dev: not a linear weight");
    if (ww.device != ctx_device(c)) return set_error(FRQ_ERR_ARG, "weight lives on another device");
    if (m == 0 || ww.n == 0) return FRQ_OK;
    if (!d_a || !d_out) return set_error(FRQ_ERR_ARG, "null activation/output pointer");
    GDev dv(ctx_device(c));
    void* a4 = nullptr;
    if (ww.dtype == FRQ_DT_I4)
        if (int rc = ctx_ws(c, i4_a4_floats(ww.k) * sizeof(float), &a4)) return rc;
    return gm_mm_rows(c, w, d_a, m, d_out, (float*)a4);
}

int frq_seq_fold_f32(frq_ctx* c, const float* x, size_t rows, size_t n, float init, float* out) {
    if (!c) return set_error(FRQ_ERR_ARG, "null context");
    if (!rows) return FRQ_OK;
    if ((!x && n) || !out) return set_error(FRQ_ERR_ARG, "null input / output");
    const size_t lds = (((n + 3) & ~(size_t)3) + seq_sum_spec_scratch(NORM_NT)) * sizeof(float);
    if (lds > GM_LDS_MAX || rows > 65535) return set_error(FRQ_ERR_ARG, "row too long for the fold's LDS");
    GDev dv(ctx_device(c));
    hipStream_t s = (hipStream_t)frq_get_stream(c);
    float* dx = nullptr;
    GMCHK(hipMalloc(&dx, (rows * n + rows) * sizeof(float)), "hipMalloc(fold)");
    struct Free {
        float* p;
        ~Free() { (void)hipFree(p); }
    } fr{dx};
    if (lds > 64 * 1024)
        GMCHK(hipFuncSetAttribute((const void*)seq_fold_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
              "hipFuncSetAttribute");
    if (n) GMCHK(hipMemcpyAsync(dx, x, rows * n * sizeof(float), hipMemcpyHostToDevice, s), "hipMemcpyAsync");
    seq_fold_kernel<<<dim3((unsigned)rows), dim3(NORM_NT), lds, s>>>(dx, (int)n, init, dx + rows * n);
    GMCHK(hipGetLastError(), "launch fold");
    GMCHK(hipMemcpyAsync(out, dx + rows * n, rows * sizeof(float), hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
    GMCHK(hipStreamSynchronize(s), "hipStreamSynchronize");
    return FRQ_OK;
}

int frq_gemma_generate_batch(frq_ctx* c, frq_gemma* g, const int64_t* prompts, size_t nb, size_t n_prompt,
                             size_t n_new, int64_t* out, float* logits) {
    return gm_run_batch(c, g, prompts, nb, n_prompt, n_new, out, logits);
}

}  // extern "C"
