// gpt2.hip — GPT-2 greedy decode on the device with a KV cache, gfx950.
//
// Restates Gpt2 of /root/reference/src/composition.rs: generate (317-341;
// the int8 cache 251-270), forward_block (175-209), forward_block_q
// (214-249), head_argmax (296-300), predict (304-308), and its layernorm,
// gelu and softmax_rows (20-50).  The linears are this library's Bundle::mm
// (frq_mm_dev) and the tied unembed its rowdot_f32 (frq_rowdot_f32_dev);
// the kernels here are the ops between them.
//
// Everything stays in HBM for a whole generate call: the embedding lookup
// reads the token the previous step's argmax wrote, and the absolute
// position `cur` lives in a device word that the argmax advances, so a
// decode step has the same launches every time and is captured once into a
// HIP graph and replayed per token.
//
// Op order per layer (m rows at positions cur .. cur+m-1):
//   a   = LN1(x)                          (fused into the previous residual)
//   qkv = mm(a, c_attn) ; qkv += bias ; K/V rows -> cache (int8: quantised)
//   att = softmax(q k^T / sqrt(hd), causal) v          per (head, row)
//   x   = x + (mm(att, attn.c_proj) + bias) ; a = LN2(x)
//   h   = gelu(mm(a, c_fc) + bias)
//   x   = x + (mm(h, mlp.c_proj) + bias) ; a = LN1 of the next layer (ln_f)
// Every step follows the reference's f32 operation order, so the tokens and
// logits are the reference's bit for bit.  This matters beyond tidiness:
// each linear quantises its input per token (round(a / sa) to int8 and the
// top-32 |a| as outliers), so a one-ulp difference in an activation can
// flip an int8 value and move the logits by ~1e-3.  Hence: layernorm's mean
// is ndarray's eight-lane sum and its variance a sequential fold; the
// softmax sum runs in key order; the score and value products follow
// matrixmultiply's order (MM_KC-long k blocks, each an FMA chain from +0,
// added in order; a head's scores are one block); exp and tanh
// are the libm algorithms Rust's f32::exp / f32::tanh reach (libm_f32.h);
// and prefill rows go through the bit-exact M <= 16 linear in chunks.
#include "frq_internal.h"
#include "libm_f32.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <vector>

namespace frq {
namespace {

constexpr int NT = 256;  // threads of the row kernels

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
// Block-wide max of NT threads (every thread gets the same value).
__device__ float block_max(float v, float* red) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// rows_f32("wte", ids) + rows_f32("wpe", positions) (src/bundle.rs:936-955):
// row t is token ids[t] (rel: ids[cur - P + t], the token the last argmax
// wrote) at position cur + t.  Ids and positions were checked on the host
// (prompt) or come from the argmax (in range).
__global__ __launch_bounds__(NT) void embed_kernel(const uint8_t* __restrict__ wte, size_t pitch,
                                                   const float* __restrict__ wpe, int d,
                                                   const int64_t* __restrict__ ids, int rel, int P,
                                                   const int* __restrict__ curp, float* __restrict__ x) {
    const int t = blockIdx.x;
    const int cur = *curp;
    const int64_t id = ids[rel ? cur - P + t : t];
    const uint16_t* row = reinterpret_cast<const uint16_t*>(wte + (size_t)id * pitch);
    const float* pe = wpe + (size_t)(cur + t) * d;
    for (int c = threadIdx.x; c < d; c += NT) x[(size_t)t * d + c] = h2f(row[c]) + pe[c];
}

// The same over p[0], p[8], p[16], ... (n values): one of ndarray's eight
// partial sums.
__device__ float seq_sum8(const float* p, int n, float acc) {
    constexpr int B = 16;
    const int nb = n / B;
    float b0[B], b1[B];
    auto ld = [&](float (&b)[B], int k) {
#pragma unroll
        for (int u = 0; u < B; ++u) b[u] = p[(k * B + u) * 8];
    };
    auto add = [&](const float (&b)[B]) {
#pragma unroll
        for (int u = 0; u < B; ++u) acc = acc + b[u];
    };
    if (nb > 0) {  // as lds_seq_sum: loads pinned a batch ahead of their adds
        ld(b0, 0);
        ld(b1, min(1, nb - 1));
        __builtin_amdgcn_sched_barrier(0);
        int k = 0;
        for (; k + 2 <= nb; k += 2) {
            add(b0);
            ld(b0, min(k + 2, nb - 1));
            __builtin_amdgcn_sched_barrier(0);
            add(b1);
            ld(b1, min(k + 3, nb - 1));
            __builtin_amdgcn_sched_barrier(0);
        }
        if (k < nb) add(b0);
    }
    for (int i = nb * B; i < n; ++i) acc = acc + p[i * 8];
    return acc;
}

// x[r] = x[r] + (y[r] + bias) (when y is set), then out[r] = layernorm(x[r])
// for rows row0 .. row0 + gridDim.x, in layernorm's order (composition.rs:
// 20-33): mu = row.sum() / n with ndarray 0.16's sum (eight partial sums
// p0..p7 over the leading multiple of 8, combined acc += p0+p4, p1+p5,
// p2+p6, p3+p7 from 0, then the tail in order), var = the fold from -0.0 of
// (v - mu)^2 in index order / n, inv = 1 / sqrt(var + 1e-5), out =
// (v - mu) * inv * g + b.  The chains run in one lane each (eight for the
// partial sums); the row and the squares sit in LDS (2d floats).
__global__ __launch_bounds__(NT) void resid_ln_kernel(float* __restrict__ x, const float* __restrict__ y,
                                                      const float* __restrict__ bias, const float* __restrict__ g,
                                                      const float* __restrict__ b, float* __restrict__ out, int d,
                                                      int row0) {
    extern __shared__ float4 lds4[];
    float* xs = reinterpret_cast<float*>(lds4);  // row (d), squares (d)
    __shared__ float part[8], stat[2];
    float* sq = xs + d;
    const size_t r = (size_t)(row0 + blockIdx.x) * d;
    for (int c = threadIdx.x; c < d; c += NT) {
        float t = x[r + c];
        if (y) {
            t = t + (y[r + c] + bias[c]);
            x[r + c] = t;
        }
        xs[c] = t;
    }
    __syncthreads();
    const int n8 = d & ~7;
    if (threadIdx.x < 8) part[threadIdx.x] = seq_sum8(xs + threadIdx.x, n8 / 8, 0.0f);
    __syncthreads();
    if (threadIdx.x == 0) {
        float acc = 0.0f;
        acc = acc + (part[0] + part[4]);
        acc = acc + (part[1] + part[5]);
        acc = acc + (part[2] + part[6]);
        acc = acc + (part[3] + part[7]);
        for (int i = n8; i < d; ++i) acc = acc + xs[i];
        stat[0] = acc / (float)d;
    }
    __syncthreads();
    const float mu = stat[0];
    for (int c = threadIdx.x; c < d; c += NT) sq[c] = (xs[c] - mu) * (xs[c] - mu);
    __syncthreads();
    if (threadIdx.x == 0) stat[1] = lds_seq_sum(sq, d, -0.0f) / (float)d;
    __syncthreads();
    const float inv = 1.0f / sqrtf(stat[1] + 1e-5f);
    for (int c = threadIdx.x; c < d; c += NT) out[r + c] = (xs[c] - mu) * inv * g[c] + b[c];
}

// qkv[i] += bias, and the K / V parts of row i go to cache row cur + i:
// f32 as is, or int8 per (position, head) as forward_block_q quantises
// them (composition.rs:224-235): sc = max|v| / 127 (1 when 0),
// q = clamp(round(v / sc), -127, 127).
template <bool KV8>
__global__ __launch_bounds__(NT) void qkv_kernel(float* __restrict__ qkv, const float* __restrict__ bias, int d,
                                                 int H, int hd, const int* __restrict__ curp,
                                                 float* __restrict__ kc, float* __restrict__ vc,
                                                 int8_t* __restrict__ kq, int8_t* __restrict__ vq,
                                                 float* __restrict__ ks, float* __restrict__ vs) {
    const int i = blockIdx.x;
    const size_t pos = (size_t)(*curp + i);
    float* row = qkv + (size_t)i * 3 * d;
    for (int c = threadIdx.x; c < 3 * d; c += NT) {
        const float v = row[c] + bias[c];
        row[c] = v;
        if constexpr (!KV8) {
            if (c >= 2 * d) vc[pos * d + (c - 2 * d)] = v;
            else if (c >= d) kc[pos * d + (c - d)] = v;
        }
    }
    if constexpr (KV8) {
        __syncthreads();  // the biased row is visible to the whole block
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        for (int u = wave; u < 2 * H; u += NT / 64) {  // u < H: K head u, else V head u - H
            const int kind = u >= H, h = kind ? u - H : u;
            const float* src = row + (size_t)(1 + kind) * d + (size_t)h * hd;
            float mx = 0.0f;
            for (int c = lane; c < hd; c += 64) mx = fmaxf(mx, fabsf(src[c]));
            mx = wave_max(mx);
            float sc = mx / 127.0f;
            if (!(sc > 0.0f)) sc = 1.0f;
            int8_t* dq = (kind ? vq : kq) + pos * d + (size_t)h * hd;
            for (int c = lane; c < hd; c += 64) {
                const float r = roundf(src[c] / sc);  // NaN -> 0 (Rust's saturating `as i8`)
                dq[c] = r != r ? (int8_t)0 : (int8_t)fminf(fmaxf(r, -127.0f), 127.0f);
            }
            if (lane == 0) (kind ? vs : ks)[pos * H + h] = sc;
        }
    }
}

// Causal attention of row i (position cur + i) and head h over cache rows
// 0 .. cur + i (forward_block 189-201): s_j = (q . k_j) / sqrt(hd) as a
// sequential FMA chain over the head dims (one thread per key), softmax
// (max, expf, the sum in key order, divide), then out_c = sum_j p_j v_jc in
// a.dot's order (each MM_KC-key block an FMA chain over j from +0, the
// blocks added in order; one lane per output dim, its loads a 16-key batch
// ahead).  Keys past cur + i carry the reference's -1e10
// mask: it joins the max, and its exp is exactly 0 (for any max above
// -1e10 + 104), so those keys add nothing and are skipped.
// FUSED (decode, one row): the block also adds the bias to its head's q, k,
// v and appends k, v to cache row cur (as qkv_kernel), before attending.
// LDS: q (hd), p and the int8 value scales (pstride each).
template <bool KV8, bool FUSED>
__global__ __launch_bounds__(NT) void attn_kernel(const float* __restrict__ qkv, const float* __restrict__ bias,
                                                  int d, int H, int hd, const int* __restrict__ curp,
                                                  float* __restrict__ kc, float* __restrict__ vc,
                                                  int8_t* __restrict__ kq, int8_t* __restrict__ vq,
                                                  float* __restrict__ ks, float* __restrict__ vs, float rs,
                                                  int pstride, float* __restrict__ att) {
    extern __shared__ float4 lds4[];
    float* q = reinterpret_cast<float*>(lds4);
    float* p = q + ((hd + 3) & ~3);
    float* sv = p + pstride;  // pstride >= max(klen_max, 2 hd), a multiple of 4
    __shared__ float red[4];
    const int h = blockIdx.x, i = blockIdx.y;
    const int cur = *curp;
    const int nk = cur + i + 1;
    const float* row = qkv + (size_t)i * 3 * d + (size_t)h * hd;
    if constexpr (FUSED) {
        const size_t pos = (size_t)cur;
        float* kv = p;  // the new k (hd) and v (hd), staged for the int8 scales
        for (int t = threadIdx.x; t < 3 * hd; t += NT) {
            const int part = t / hd, c = t - part * hd;
            const size_t col = (size_t)part * d + (size_t)h * hd + c;
            const float v = row[(size_t)part * d + c] + bias[col];
            if (part == 0) q[c] = v;
            else if constexpr (!KV8) (part == 1 ? kc : vc)[pos * d + (size_t)h * hd + c] = v;
            else kv[(part - 1) * hd + c] = v;
        }
        if constexpr (KV8) {
            __syncthreads();
            const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
            if (wave < 2) {  // wave 0: k, wave 1: v (forward_block_q 224-235)
                const float* src = kv + wave * hd;
                float mx = 0.0f;
                for (int c = lane; c < hd; c += 64) mx = fmaxf(mx, fabsf(src[c]));
                mx = wave_max(mx);
                float sc = mx / 127.0f;
                if (!(sc > 0.0f)) sc = 1.0f;
                int8_t* dq = (wave ? vq : kq) + pos * d + (size_t)h * hd;
                for (int c = lane; c < hd; c += 64) {
                    const float r = roundf(src[c] / sc);
                    dq[c] = r != r ? (int8_t)0 : (int8_t)fminf(fmaxf(r, -127.0f), 127.0f);
                }
                if (lane == 0) (wave ? vs : ks)[pos * H + h] = sc;
            }
        }
    } else {
        for (int c = threadIdx.x; c < hd; c += NT) q[c] = row[c];
    }
    __syncthreads();  // q, and (FUSED) the new cache row, visible to the block
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < nk; j += NT) {
        float acc = 0.0f;
        if constexpr (!KV8) {
            const float* kr = kc + (size_t)j * d + (size_t)h * hd;
            for (int c = 0; c < hd; c += 4) {
                const float4 k4 = *reinterpret_cast<const float4*>(kr + c);
                acc = __builtin_fmaf(q[c], k4.x, acc);
                acc = __builtin_fmaf(q[c + 1], k4.y, acc);
                acc = __builtin_fmaf(q[c + 2], k4.z, acc);
                acc = __builtin_fmaf(q[c + 3], k4.w, acc);
            }
        } else {
            const int8_t* kr = kq + (size_t)j * d + (size_t)h * hd;
            const float sk = ks[(size_t)j * H + h];
            sv[j] = vs[(size_t)j * H + h];
            for (int c = 0; c < hd; c += 4) {
                const char4 k4 = *reinterpret_cast<const char4*>(kr + c);
                acc = __builtin_fmaf(q[c], (float)k4.x * sk, acc);
                acc = __builtin_fmaf(q[c + 1], (float)k4.y * sk, acc);
                acc = __builtin_fmaf(q[c + 2], (float)k4.z * sk, acc);
                acc = __builtin_fmaf(q[c + 3], (float)k4.w * sk, acc);
            }
        }
        const float sj = acc / rs;
        p[j] = sj;
        mx = fmaxf(mx, sj);
    }
    mx = block_max(mx, red);
    if (nk < cur + (int)gridDim.y) mx = fmaxf(mx, -1e10f);  // a masked entry joins the max
    for (int j = threadIdx.x; j < nk; j += NT) p[j] = libm::frq_expf(p[j] - mx);
    __syncthreads();
    if (threadIdx.x == 0) red[0] = lds_seq_sum(p, nk, 0.0f);  // masked exps are +0
    __syncthreads();
    const float sum = red[0];
    for (int j = threadIdx.x; j < nk; j += NT) p[j] = p[j] / sum;
    __syncthreads();
    // out_c: one lane per dim; the value loads (coalesced over the lanes)
    // run one 16-key batch ahead of the chain
    constexpr int B = 16;
    for (int c = threadIdx.x; c < hd; c += NT) {
        const size_t col = (size_t)h * hd + c;
        // one a.dot block of keys [s, e), chained from +0
        auto chain = [&](int s, int e) {
            float acc = 0.0f;
            const int nb = (e - s) / B;
            float v0[B], v1[B];
            auto ld = [&](float (&v)[B], int k) {
#pragma unroll
                for (int u = 0; u < B; ++u) {
                    const size_t j = (size_t)(s + k * B + u);
                    if constexpr (!KV8) v[u] = vc[j * d + col];
                    else v[u] = (float)vq[j * d + col] * sv[j];
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
                const float v = KV8 ? (float)vq[(size_t)j * d + col] * sv[j] : vc[(size_t)j * d + col];
                acc = __builtin_fmaf(p[j], v, acc);
            }
            return acc;
        };
        att[(size_t)i * d + col] = mm_blocks(0, nk, chain);
    }
}

// h = gelu(h + bias) (composition.rs:35-38; bias over the row of n).
__global__ __launch_bounds__(NT) void bias_gelu_kernel(float* __restrict__ hm, const float* __restrict__ bias,
                                                       int n, size_t total, float c) {
    for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < total; i += (size_t)gridDim.x * NT) {
        const float v = hm[i] + bias[i % n];
        hm[i] = 0.5f * v * (1.0f + libm::frq_tanhf(c * (v + 0.044715f * v * v * v)));
    }
}

// head_argmax's max_by(partial_cmp) (composition.rs:299): the unembed
// folded the argmax (the LAST index of the maximum) into *best; a NaN logit
// (a panic there) set the error word.  The token goes to out[cur + m - P],
// then cur += m and *best is cleared for the next step.
__global__ void argmax_done_kernel(unsigned long long* __restrict__ best, int* __restrict__ curp, int m, int P,
                                   int64_t* __restrict__ out) {
    if (threadIdx.x == 0) {
        const int cur = *curp;
        out[cur + m - P] = (int64_t)(uint32_t)(*best & 0xffffffffull);
        *curp = cur + m;
        *best = 0ull;
    }
}

float gelu_c() { return sqrtf(2.0f / 3.14159274101257324f); }  // (2/PI as f32).sqrt()

__host__ __device__ inline float libm_fn(int fn, float x) {
    return fn == 0 ? libm::frq_expf(x)
                   : fn == 1 ? libm::frq_expm1f(x) : fn == 2 ? libm::frq_tanhf(x) : libm::frq_expf_sel(x);
}
__global__ __launch_bounds__(NT) void libm_kernel(int fn, const float* __restrict__ x, size_t n,
                                                  float* __restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT)
        out[i] = libm_fn(fn, x[i]);
}

}  // namespace
}  // namespace frq

using namespace frq;

struct frq_gpt2 {
    int device = 0;
    size_t L = 0, H = 0, d = 0, npos = 0, vocab = 0, hd = 0;
    int kv8 = 0;
    int graphs = 1;
    std::vector<frq_w*> lin;  // 4 per layer: c_attn, attn.c_proj, c_fc, mlp.c_proj
    frq_w* wte = nullptr;     // f16 row table: the embedding rows and the tied unembed
    // device memory (one allocation): f32 vectors and the activations
    char* mem = nullptr;
    float *wpe = nullptr, *lnf_g = nullptr, *lnf_b = nullptr, *ln = nullptr, *bias = nullptr;
    float *kc = nullptr, *vc = nullptr, *ks = nullptr, *vs = nullptr;
    int8_t *kq = nullptr, *vq = nullptr;
    float *x = nullptr, *a = nullptr, *qkv = nullptr, *att = nullptr, *y = nullptr, *hm = nullptr, *logits = nullptr;
    int* cur = nullptr;
    unsigned long long* best = nullptr;  // the unembed's folded argmax
    int64_t *tok = nullptr, *ids = nullptr;
    ~frq_gpt2() {
        for (frq_w* w : lin) frq_w_free(w);
        frq_w_free(wte);
        if (mem) (void)hipFree(mem);
    }
    // per-layer vectors: ln (4 per layer: ln_1 g, b, ln_2 g, b) and bias
    // (c_attn 3d, attn.c_proj d, c_fc 4d, mlp.c_proj d)
    const float* ln_of(size_t l, int j) const { return ln + (4 * l + j) * d; }
    const float* bias_of(size_t l, int j) const {
        static const size_t off[4] = {0, 3, 4, 8};
        return bias + (9 * l + off[j]) * d;
    }
};

namespace {

int fail_hip(hipError_t e, const char* what) {
    return set_error(FRQ_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}
#define GCHK(expr, what)                                  \
    do {                                                  \
        hipError_t e_ = (expr);                           \
        if (e_ != hipSuccess) return fail_hip(e_, what);  \
    } while (0)

struct DevSwitch {
    int prev = -1;
    explicit DevSwitch(int d) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != d) (void)hipSetDevice(d);
    }
    ~DevSwitch() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

float f16f(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t b;
    if (e == 0) {
        if (!m) b = s;
        else {  // subnormal: normalise
            int sh = 0;
            uint32_t mm = m;
            while (!(mm & 1024)) { mm <<= 1; ++sh; }
            b = s | ((uint32_t)(113 - sh) << 23) | ((mm & 1023) << 13);
        }
    } else if (e == 31) {
        b = s | 0x7F800000u | (m << 13);
    } else {
        b = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

// A 1-D (or (rows, d) 2-D) f16 / f32 array of the bundle as f32, appended
// to host staging at `dst` (n values).
int vec_f32(const frq_bundle* b, const std::string& name, size_t n, float* dst) {
    char dt[16];
    size_t shape[4], nd = 4, grp = 0, bytes = 0;
    const void* data = nullptr;
    if (int rc = frq_bundle_array(b, name.c_str(), dt, sizeof dt, shape, &nd, &grp, &data, &bytes)) return rc;
    size_t cnt = 1;
    for (size_t i = 0; i < nd; ++i) cnt *= shape[i];
    const std::string t = dt;
    if (cnt != n || (t != "f16" && t != "f32") || bytes != n * (t == "f16" ? 2 : 4))
        return set_error(FRQ_ERR_FORMAT, "array " + name + ": expected " + std::to_string(n) + " f16/f32 values");
    if (t == "f32") {
        std::memcpy(dst, data, n * 4);
    } else {
        const uint16_t* hsrc = static_cast<const uint16_t*>(data);
        for (size_t i = 0; i < n; ++i) dst[i] = f16f(hsrc[i]);
    }
    return FRQ_OK;
}

int check_lin(const frq_w* w, size_t k, size_t n, const std::string& name) {
    int dt = 0;
    size_t wn = 0, wk = 0, g = 0;
    if (int rc = frq_w_info(w, &dt, &wn, &wk, &g)) return rc;
    if (dt != FRQ_DT_I8 && dt != FRQ_DT_I4 && dt != FRQ_DT_Q4A)
        return set_error(FRQ_ERR_DTYPE, name + ": not an int8 / int4 / q4a linear");
    if (wk != k || wn != n)
        return set_error(FRQ_ERR_FORMAT, name + ": shape (" + std::to_string(wk) + ", " + std::to_string(wn) +
                                             "), expected (" + std::to_string(k) + ", " + std::to_string(n) + ")");
    return FRQ_OK;
}

size_t attn_pstride(const frq_gpt2* g) { return (std::max(g->npos, 2 * g->hd) + 3) & ~(size_t)3; }
size_t attn_lds(const frq_gpt2* g) { return (((g->hd + 3) & ~(size_t)3) + 2 * attn_pstride(g)) * sizeof(float); }

// One forward block (m rows at device position cur; rel: the row's token
// is the previous argmax) through the head: the argmax token and cur += m.
int gpt2_block(frq_ctx* c, frq_gpt2* g, size_t m, int rel, int P, float* logits_out) {
    hipStream_t s = (hipStream_t)frq_get_stream(c);
    const int d = (int)g->d, H = (int)g->H, hd = (int)g->hd;
    const Weight& wt = *weight_of(g->wte);
    const float rs = sqrtf((float)hd);
    auto ln = [&](const float* y, const float* bias, const float* gg, const float* bb, int rows, int row0) {
        resid_ln_kernel<<<dim3(rows), dim3(NT), 2 * g->d * sizeof(float), s>>>(g->x, y, bias, gg, bb, g->a, d,
                                                                              row0);
        return hipGetLastError();
    };
    // Bundle::mm over m rows; m > 16 through the MFMA GEMM with the exact
    // epilogue, else in chunks of 8..16 rows (the bit-exact multi-row path;
    // every row is quantised and reduced on its own, so the chunks give the
    // whole product's rows)
    auto mm = [&](frq_w* w, const float* in, size_t K, float* o, size_t N) -> int {
        if (m <= 16) return frq_mm_dev(c, w, in, m, o);
        if (i8_rows_exact_ok(w, m)) return mm_i8_rows_exact(c, w, in, m, o);
        const size_t nch = (m + 15) / 16;
        size_t r0 = 0;
        for (size_t i = 0; i < nch; ++i) {
            const size_t rows = m / nch + (i < m % nch ? 1 : 0);
            if (int rc = frq_mm_dev(c, w, in + r0 * K, rows, o + r0 * N)) return rc;
            r0 += rows;
        }
        return FRQ_OK;
    };
    embed_kernel<<<dim3((unsigned)m), dim3(NT), 0, s>>>(wt.rowp, wt.rpitch, g->wpe, d, rel ? g->tok : g->ids, rel,
                                                        P, g->cur, g->x);
    GCHK(hipGetLastError(), "launch embed");
    GCHK(ln(nullptr, nullptr, g->ln_of(0, 0), g->ln_of(0, 1), (int)m, 0), "launch layernorm");
    for (size_t l = 0; l < g->L; ++l) {
        if (int rc = mm(g->lin[4 * l], g->a, g->d, g->qkv, 3 * g->d)) return rc;
        float* kc = g->kv8 ? nullptr : g->kc + l * g->npos * g->d;
        float* vc = g->kv8 ? nullptr : g->vc + l * g->npos * g->d;
        int8_t* kq = g->kv8 ? g->kq + l * g->npos * g->d : nullptr;
        int8_t* vq = g->kv8 ? g->vq + l * g->npos * g->d : nullptr;
        float* ks = g->kv8 ? g->ks + l * g->npos * g->H : nullptr;
        float* vs = g->kv8 ? g->vs + l * g->npos * g->H : nullptr;
        const dim3 ag((unsigned)H, (unsigned)m);
        const size_t lds = attn_lds(g);
        const int np = (int)attn_pstride(g);
        if (m == 1) {  // decode: bias, cache append and attention in one launch per head
            if (g->kv8)
                attn_kernel<true, true><<<ag, dim3(NT), lds, s>>>(g->qkv, g->bias_of(l, 0), d, H, hd, g->cur, kc,
                                                                  vc, kq, vq, ks, vs, rs, np, g->att);
            else
                attn_kernel<false, true><<<ag, dim3(NT), lds, s>>>(g->qkv, g->bias_of(l, 0), d, H, hd, g->cur, kc,
                                                                   vc, kq, vq, ks, vs, rs, np, g->att);
        } else {
            if (g->kv8)
                qkv_kernel<true><<<dim3((unsigned)m), dim3(NT), 0, s>>>(g->qkv, g->bias_of(l, 0), d, H, hd, g->cur,
                                                                        kc, vc, kq, vq, ks, vs);
            else
                qkv_kernel<false><<<dim3((unsigned)m), dim3(NT), 0, s>>>(g->qkv, g->bias_of(l, 0), d, H, hd, g->cur,
                                                                         kc, vc, kq, vq, ks, vs);
            GCHK(hipGetLastError(), "launch qkv");
            if (g->kv8)
                attn_kernel<true, false><<<ag, dim3(NT), lds, s>>>(g->qkv, nullptr, d, H, hd, g->cur, kc, vc, kq, vq,
                                                                   ks, vs, rs, np, g->att);
            else
                attn_kernel<false, false><<<ag, dim3(NT), lds, s>>>(g->qkv, nullptr, d, H, hd, g->cur, kc, vc, kq,
                                                                    vq, ks, vs, rs, np, g->att);
        }
        GCHK(hipGetLastError(), "launch attention");
        if (int rc = mm(g->lin[4 * l + 1], g->att, g->d, g->y, g->d)) return rc;
        GCHK(ln(g->y, g->bias_of(l, 1), g->ln_of(l, 2), g->ln_of(l, 3), (int)m, 0), "launch layernorm");
        if (int rc = mm(g->lin[4 * l + 2], g->a, g->d, g->hm, 4 * g->d)) return rc;
        const size_t tot = m * 4 * g->d;
        const unsigned gb = (unsigned)std::min<size_t>((tot + NT - 1) / NT, 4096);
        bias_gelu_kernel<<<dim3(gb), dim3(NT), 0, s>>>(g->hm, g->bias_of(l, 2), 4 * d, tot, gelu_c());
        GCHK(hipGetLastError(), "launch gelu");
        if (int rc = mm(g->lin[4 * l + 3], g->hm, 4 * g->d, g->y, g->d)) return rc;
        if (l + 1 < g->L)
            GCHK(ln(g->y, g->bias_of(l, 3), g->ln_of(l + 1, 0), g->ln_of(l + 1, 1), (int)m, 0), "launch layernorm");
        else  // only the last row feeds the head: its residual and ln_f
            GCHK(ln(g->y, g->bias_of(l, 3), g->lnf_g, g->lnf_b, 1, (int)m - 1), "launch layernorm");
    }
    float* lg = logits_out ? logits_out : g->logits;
    GCHK(launch_rowdot_argmax(wt, g->a + (m - 1) * g->d, lg, g->best, ctx_err(c), s), "launch rowdot");
    argmax_done_kernel<<<dim3(1), dim3(64), 0, s>>>(g->best, g->cur, (int)m, P, g->tok);
    GCHK(hipGetLastError(), "launch argmax");
    return FRQ_OK;
}

int gpt2_check(frq_ctx* c, frq_gpt2* g) {
    if (!c) return set_error(FRQ_ERR_ARG, "null context");
    if (!g) return set_error(FRQ_ERR_ARG, "null model");
    if (ctx_device(c) != g->device) return set_error(FRQ_ERR_ARG, "model lives on another device");
    return FRQ_OK;
}

// Generate: prefill the prompt, then n_new - 1 decode steps (a captured
// graph replayed per step when allowed).  logits (n_new, vocab) host,
// nullable.
int gpt2_run(frq_ctx* c, frq_gpt2* g, const int64_t* prompt, size_t P, size_t n_new, int64_t* out, float* logits) {
    if (int rc = gpt2_check(c, g)) return rc;
    if (!P || !n_new) return set_error(FRQ_ERR_ARG, "empty prompt or no tokens asked for");
    if (!prompt || !out) return set_error(FRQ_ERR_ARG, "null prompt / output");
    if (P + n_new - 1 > g->npos)
        return set_error(FRQ_ERR_ARG, "position " + std::to_string(P + n_new - 2) + " beyond n_positions " +
                                          std::to_string(g->npos) + " (the reference panics on the wpe row)");
    for (size_t i = 0; i < P; ++i)
        if (prompt[i] < 0 || (size_t)prompt[i] >= g->vocab)
            return set_error(FRQ_ERR_ARG, "token id " + std::to_string(prompt[i]) + " beyond the vocabulary");
    DevSwitch dv(g->device);
    hipStream_t s = (hipStream_t)frq_get_stream(c);
    float* lgd = nullptr;
    if (logits) GCHK(hipMalloc(&lgd, n_new * g->vocab * sizeof(float)), "hipMalloc(logits)");
    struct Free {
        float* p;
        ~Free() { if (p) (void)hipFree(p); }
    } fr{lgd};
    GCHK(hipMemcpyAsync(g->ids, prompt, P * sizeof(int64_t), hipMemcpyHostToDevice, s), "hipMemcpyAsync(prompt)");
    GCHK(hipMemsetAsync(g->cur, 0, sizeof(int), s), "hipMemsetAsync(cur)");
    if (int rc = gpt2_block(c, g, P, 0, (int)P, lgd)) return rc;
    const bool graph = g->graphs && !logits && n_new > 2 && s != nullptr;
    if (graph) {
        hipGraph_t gr = nullptr;
        hipGraphExec_t ex = nullptr;
        GCHK(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
        const int rc = gpt2_block(c, g, 1, 1, (int)P, nullptr);
        const hipError_t e = hipStreamEndCapture(s, &gr);
        if (rc) { if (gr) (void)hipGraphDestroy(gr); return rc; }
        GCHK(e, "hipStreamEndCapture");
        hipError_t ei = hipGraphInstantiate(&ex, gr, nullptr, nullptr, 0);
        (void)hipGraphDestroy(gr);
        GCHK(ei, "hipGraphInstantiate");
        hipError_t el = hipSuccess;
        for (size_t t = 1; t < n_new && el == hipSuccess; ++t) el = hipGraphLaunch(ex, s);
        (void)hipGraphExecDestroy(ex);
        GCHK(el, "hipGraphLaunch");
    } else {
        for (size_t t = 1; t < n_new; ++t)
            if (int rc = gpt2_block(c, g, 1, 1, (int)P, lgd ? lgd + t * g->vocab : nullptr)) return rc;
    }
    GCHK(hipMemcpyAsync(out, g->tok, n_new * sizeof(int64_t), hipMemcpyDeviceToHost, s), "hipMemcpyAsync(tokens)");
    if (logits)
        GCHK(hipMemcpyAsync(logits, lgd, n_new * g->vocab * sizeof(float), hipMemcpyDeviceToHost, s),
             "hipMemcpyAsync(logits)");
    return frq_sync(c);  // NaN activations / logits -> FRQ_ERR_NAN
}

}  // namespace

extern "C" {

int frq_gpt2_load(frq_ctx* c, const frq_bundle* b, int kv_int8, frq_gpt2** out) {
    if (!out) return set_error(FRQ_ERR_ARG, "null output handle");
    *out = nullptr;
    if (!c || !b) return set_error(FRQ_ERR_ARG, "null context / bundle");
    char arch[32];
    int64_t cfg[8];
    size_t nc = 8, nf = 0;
    if (int rc = frq_bundle_header(b, arch, sizeof arch, cfg, &nc, nullptr, &nf)) return rc;
    if (std::string(arch) != "gpt2") return set_error(FRQ_ERR_FORMAT, std::string("not a gpt2 bundle: ") + arch);
    if (nc < 5) return set_error(FRQ_ERR_FORMAT, "gpt2 config needs [n_layer, n_head, n_embd, n_positions, vocab]");
    for (int i = 0; i < 5; ++i)
        if (cfg[i] <= 0) return set_error(FRQ_ERR_FORMAT, "gpt2 config entries must be positive");
    auto g = std::make_unique<frq_gpt2>();
    g->device = ctx_device(c);
    g->L = cfg[0]; g->H = cfg[1]; g->d = cfg[2]; g->npos = cfg[3]; g->vocab = cfg[4];
    g->kv8 = kv_int8 ? 1 : 0;
    if (g->d % g->H) return set_error(FRQ_ERR_FORMAT, "n_embd not a multiple of n_head");
    g->hd = g->d / g->H;
    // a head's scores are one a.dot block (hd <= MM_KC): a single FMA chain
    if (g->hd % 4 || g->hd > (size_t)MM_KC || g->d > 2048 || attn_lds(g.get()) > 64 * 1024 || g->npos > (1u << 20))
        return set_error(FRQ_ERR_ARG, "gpt2 shape outside this build's kernels (head dim % 4 and <= 256, "
                                      "n_embd <= 2048, n_positions within 64 KB of scores)");
    const size_t L = g->L, d = g->d;
    // linears and the row table
    static const char* names[4] = {"attn.c_attn", "attn.c_proj", "mlp.c_fc", "mlp.c_proj"};
    const size_t kin[4] = {d, d, d, 4 * d}, nout[4] = {3 * d, d, 4 * d, d};
    for (size_t l = 0; l < L; ++l)
        for (int j = 0; j < 4; ++j) {
            const std::string nm = "h" + std::to_string(l) + "." + names[j] + ".weight";
            frq_w* w = nullptr;
            if (int rc = frq_bundle_weight(c, b, nm.c_str(), &w)) return rc;
            g->lin.push_back(w);
            if (int rc = check_lin(w, kin[j], nout[j], nm)) return rc;
        }
    if (int rc = frq_bundle_weight(c, b, "wte", &g->wte)) return rc;
    {
        int dt = 0;
        size_t n = 0, k = 0, gg = 0;
        (void)frq_w_info(g->wte, &dt, &n, &k, &gg);
        if (dt != FRQ_DT_F16 || n != g->vocab || k != d)
            return set_error(FRQ_ERR_FORMAT, "wte: expected an f16 (vocab, n_embd) table");
    }
    // host staging of the f32 vectors: wpe, ln_f, ln (4 per layer), bias (9d per layer)
    const size_t nvec = g->npos * d + 2 * d + 4 * L * d + 9 * L * d;
    std::vector<float> hv(nvec);
    float* p = hv.data();
    if (int rc = vec_f32(b, "wpe", g->npos * d, p)) return rc;
    p += g->npos * d;
    if (int rc = vec_f32(b, "ln_f.weight", d, p)) return rc;
    if (int rc = vec_f32(b, "ln_f.bias", d, p + d)) return rc;
    p += 2 * d;
    for (size_t l = 0; l < L; ++l) {
        const std::string pre = "h" + std::to_string(l) + ".";
        const char* lns[4] = {"ln_1.weight", "ln_1.bias", "ln_2.weight", "ln_2.bias"};
        for (int j = 0; j < 4; ++j)
            if (int rc = vec_f32(b, pre + lns[j], d, p + j * d)) return rc;
        p += 4 * d;
    }
    for (size_t l = 0; l < L; ++l) {
        const std::string pre = "h" + std::to_string(l) + ".";
        size_t off = 0;
        for (int j = 0; j < 4; ++j) {
            if (int rc = vec_f32(b, pre + names[j] + ".bias", nout[j], p + off)) return rc;
            off += nout[j];
        }
        p += 9 * d;
    }
    // device memory: vectors, cache, activations
    const size_t N = g->npos, V = g->vocab, H = g->H;
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off += round_up(bytes, 256); return o; };
    const size_t o_vec = take(nvec * 4);
    size_t o_kc = 0, o_vc = 0, o_ks = 0, o_vs = 0;
    if (g->kv8) {
        o_kc = take(L * N * d); o_vc = take(L * N * d);
        o_ks = take(L * N * H * 4); o_vs = take(L * N * H * 4);
    } else {
        o_kc = take(L * N * d * 4); o_vc = take(L * N * d * 4);
    }
    const size_t o_x = take(N * d * 4), o_a = take(N * d * 4), o_qkv = take(N * 3 * d * 4), o_att = take(N * d * 4),
                 o_y = take(N * d * 4), o_h = take(N * 4 * d * 4), o_lg = take(V * 4), o_cur = take(4), o_best = take(8),
                 o_tok = take(N * 8), o_ids = take(N * 8);
    DevSwitch dv(g->device);
    hipStream_t s = (hipStream_t)frq_get_stream(c);
    GCHK(hipMalloc(&g->mem, off), "hipMalloc(gpt2)");
    char* m = g->mem;
    GCHK(hipMemsetAsync(m, 0, off, s), "hipMemsetAsync(gpt2)");
    GCHK(hipMemcpyAsync(m + o_vec, hv.data(), nvec * 4, hipMemcpyHostToDevice, s), "hipMemcpyAsync(vectors)");
    float* vec = reinterpret_cast<float*>(m + o_vec);
    g->wpe = vec;
    g->lnf_g = vec + N * d;
    g->lnf_b = g->lnf_g + d;
    g->ln = g->lnf_b + d;
    g->bias = g->ln + 4 * L * d;
    if (g->kv8) {
        g->kq = reinterpret_cast<int8_t*>(m + o_kc); g->vq = reinterpret_cast<int8_t*>(m + o_vc);
        g->ks = reinterpret_cast<float*>(m + o_ks); g->vs = reinterpret_cast<float*>(m + o_vs);
    } else {
        g->kc = reinterpret_cast<float*>(m + o_kc); g->vc = reinterpret_cast<float*>(m + o_vc);
    }
    g->x = reinterpret_cast<float*>(m + o_x); g->a = reinterpret_cast<float*>(m + o_a);
    g->qkv = reinterpret_cast<float*>(m + o_qkv); g->att = reinterpret_cast<float*>(m + o_att);
    g->y = reinterpret_cast<float*>(m + o_y); g->hm = reinterpret_cast<float*>(m + o_h);
    g->logits = reinterpret_cast<float*>(m + o_lg); g->cur = reinterpret_cast<int*>(m + o_cur);
    g->best = reinterpret_cast<unsigned long long*>(m + o_best);
    g->tok = reinterpret_cast<int64_t*>(m + o_tok); g->ids = reinterpret_cast<int64_t*>(m + o_ids);
    GCHK(hipStreamSynchronize(s), "hipStreamSynchronize");  // hv is released on return
    *out = g.release();
    return FRQ_OK;
}

void frq_gpt2_free(frq_gpt2* g) { delete g; }

int frq_gpt2_info(const frq_gpt2* g, size_t* n_layer, size_t* n_head, size_t* d, size_t* n_pos, size_t* vocab) {
    if (!g) return set_error(FRQ_ERR_ARG, "null model");
    if (n_layer) *n_layer = g->L;
    if (n_head) *n_head = g->H;
    if (d) *d = g->d;
    if (n_pos) *n_pos = g->npos;
    if (vocab) *vocab = g->vocab;
    return FRQ_OK;
}

int frq_libm_f32(frq_ctx* c, int fn, const float* x, size_t n, float* out) {
    if (fn < 0 || fn > 3) return set_error(FRQ_ERR_ARG, "fn: 0 expf, 1 expm1f, 2 tanhf, 3 expf (branch-free form)");
    if (!n) return FRQ_OK;
    if (!x || !out) return set_error(FRQ_ERR_ARG, "null input / output");
    if (!c) {
        for (size_t i = 0; i < n; ++i) out[i] = libm_fn(fn, x[i]);
        return FRQ_OK;
    }
    DevSwitch dv(ctx_device(c));
    hipStream_t s = (hipStream_t)frq_get_stream(c);
    float* dx = nullptr;
    GCHK(hipMalloc(&dx, 2 * n * sizeof(float)), "hipMalloc(libm)");
    struct Free {
        float* p;
        ~Free() { (void)hipFree(p); }
    } fr{dx};
    GCHK(hipMemcpyAsync(dx, x, n * sizeof(float), hipMemcpyHostToDevice, s), "hipMemcpyAsync");
    const unsigned grid = (unsigned)std::min<size_t>((n + NT - 1) / NT, 8192);
    libm_kernel<<<dim3(grid), dim3(NT), 0, s>>>(fn, dx, n, dx + n);
    GCHK(hipGetLastError(), "launch libm");
    GCHK(hipMemcpyAsync(out, dx + n, n * sizeof(float), hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
    GCHK(hipStreamSynchronize(s), "hipStreamSynchronize");
    return FRQ_OK;
}

int frq_gpt2_set_graphs(frq_gpt2* g, int on) {
    if (!g) return set_error(FRQ_ERR_ARG, "null model");
    g->graphs = on ? 1 : 0;
    return FRQ_OK;
}

int frq_gpt2_generate(frq_ctx* c, frq_gpt2* g, const int64_t* prompt, size_t n_prompt, size_t n_new,
                      int64_t* out, float* logits) {
    return gpt2_run(c, g, prompt, n_prompt, n_new, out, logits);
}

int frq_gpt2_predict(frq_ctx* c, frq_gpt2* g, const int64_t* ids, size_t n, int64_t* token, float* logits) {
    return gpt2_run(c, g, ids, n, 1, token, logits);
}

}  // extern "C"
