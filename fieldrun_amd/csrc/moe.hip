// moe.hip — routed MoE expert layer (gfx950).
//
// Restates the routed branch of /root/reference/src/qwen3moe.rs:120-158
// (act SiLU) and the expert part of src/gemma4.rs:131-187 (act gelu_tanh,
// packed gate_up, per_expert_scale), with the experts' matmuls as in
// expert_f32 / expert_mm (src/bundle.rs:404-461): W8A32, w = q * scale[j]
// exactly in f32, then an f32 GEMM.
//
// Pipeline (all on the device, no host round trip):
//   route     one wave per token: max, exp, sequential sum, divide
//             (softmax_rows, qwen3moe.rs:42-52), then k rounds of a wave
//             arg-max by (p desc, expert asc) == the reference's stable
//             sort_by + truncate (129-130), renorm over the top-k in that
//             order (131), gemma4: p / sum * per_expert_scale[e] (158).
//   dispatch  one workgroup: per-expert counts, offsets, and each (token,
//             slot) pair's row in the expert-sorted permutation, tokens in
//             ascending order within an expert (a per-expert token bitmap
//             gives the rank); plus the list of (expert, row0) GEMM tiles.
//   gemm      grouped GEMM over the tile list: rows gathered through the
//             permutation, weights dequantised while staged into LDS, a
//             sequential-k FMA chain per output (the oracle's sgemm order).
//   act       h = silu(g) * u   or   gelu_tanh(g[:mi]) * g[mi:].
//   combine   out[t,:] = sum over t's experts in ascending expert id of
//             w * down (mul then add from +0): the reference adds in HashMap
//             order, which is random per process; ascending id is one of
//             its orders.
#include "frq_internal.h"

namespace frq {

namespace {

constexpr int GBM = 32, GBN = 64, GKC = 32;

struct MoeWs {
    int32_t* sel;      // [T*k]
    float* w;          // [T*k]
    int32_t* cnt;      // [E]
    int32_t* off;      // [E+1]
    int32_t* pos;      // [T*k]   row of (t, slot) in the permutation
    int32_t* ptok;     // [T*k]   token of permuted row
    int32_t* tile_e;   // [ntile_max]
    int32_t* tile_r;   // [ntile_max]
    int32_t* ntile;    // [1]
    float* g;          // [T*k, gw]
    float* u;          // [T*k, mi]
    float* h;          // [T*k, mi]
    float* dn;         // [T*k, d]
};

size_t ntile_max(size_t T, size_t k, size_t E) { return T * k / GBM + E + 1; }

MoeWs moe_view(void* base, const MoeBank& b, size_t T, size_t k) {
    const size_t P = T * k, E = b.n_exp, nt = ntile_max(T, k, E);
    char* p = (char*)base;
    MoeWs v;
    auto take = [&](size_t bytes) { char* r = p; p += round_up(bytes, 256); return r; };
    v.sel = (int32_t*)take(P * 4);
    v.w = (float*)take(P * 4);
    v.cnt = (int32_t*)take(E * 4);
    v.off = (int32_t*)take((E + 1) * 4);
    v.pos = (int32_t*)take(P * 4);
    v.ptok = (int32_t*)take(P * 4);
    v.tile_e = (int32_t*)take(nt * 4);
    v.tile_r = (int32_t*)take(nt * 4);
    v.ntile = (int32_t*)take(4);
    v.g = (float*)take(P * b.gw * 4);
    v.u = (float*)take(P * b.mi * 4);
    v.h = (float*)take(P * b.mi * 4);
    v.dn = (float*)take(P * b.d * 4);
    return v;
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float gelu_tanh(float x) {
    const float c = sqrtf(2.0f / 3.14159274101257324f);
    return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

// ---- routing: one wave per token ----------------------------------------
__global__ __launch_bounds__(256) void route_kernel(
    const float* __restrict__ logits, int T, int E, int topk, int norm_topk,
    const float* __restrict__ pes, int32_t* __restrict__ sel,
    float* __restrict__ wout, int* __restrict__ err) {
    extern __shared__ float sp[];  // [4][E]
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wv;
    const bool active = t < T;
    float* p = sp + wv * E;
    const float* row = logits + (size_t)(active ? t : 0) * E;
    float m = -INFINITY;
    int bad = 0;
    for (int e = lane; e < E && active; e += 64) {
        const float v = row[e];
        bad |= (v != v);
        m = fmaxf(m, v);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        m = fmaxf(m, __shfl_xor(m, off, 64));
        bad |= __shfl_xor(bad, off, 64);
    }
    // sort_by(partial_cmp().unwrap()) panics on NaN: raise err; the token
    // gets experts 0..k-1 with weight 0 so the rest of the pipeline stays in
    // bounds (the call reports FRQ_ERR_NAN)
    if (active && bad && lane == 0) {
        atomicOr(err, 1);
        for (int i = 0; i < topk; ++i) {
            sel[(size_t)t * topk + i] = i;
            wout[(size_t)t * topk + i] = 0.0f;
        }
    }
    const bool go = active && !bad;
    for (int e = lane; e < E && go; e += 64) p[e] = expf(row[e] - m);
    __syncthreads();
    float s = 0.0f;  // sequential sum in expert order, as the reference
    for (int e = 0; e < E && go; ++e) s = s + p[e];
    __syncthreads();
    for (int e = lane; e < E && go; e += 64) p[e] = p[e] / s;
    __syncthreads();
    // k rounds of arg-max by (p desc, e asc); taken experts get p = -1
    float denom = -0.0f;
    for (int i = 0; i < topk; ++i) {
        float bv = -2.0f;
        int be = 0x7FFFFFFF;
        for (int e = lane; e < E && go; e += 64) {
            const float v = p[e];
            if (v > bv || (v == bv && e < be)) { bv = v; be = e; }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const int oe = __shfl_xor(be, off, 64);
            if (ov > bv || (ov == bv && oe < be)) { bv = ov; be = oe; }
        }
        __syncthreads();
        if (go && lane == 0) {
            sel[(size_t)t * topk + i] = be;
            wout[(size_t)t * topk + i] = bv;  // p for now
            p[be] = -1.0f;
        }
        __syncthreads();
        denom = denom + bv;
    }
    if (go && lane == 0) {
        const bool renorm = norm_topk || pes != nullptr;
        for (int i = 0; i < topk; ++i) {
            const float pv = wout[(size_t)t * topk + i];
            float wv2 = renorm ? pv / denom : pv;
            if (pes) wv2 = wv2 * pes[sel[(size_t)t * topk + i]];
            wout[(size_t)t * topk + i] = wv2;
        }
    }
}

// ---- dispatch: one workgroup of 1024 threads ------------------------------
constexpr int TC = 1024;  // tokens per bitmap chunk

__global__ __launch_bounds__(1024) void dispatch_kernel(
    const int32_t* __restrict__ sel, int T, int topk, int E,
    MoeWs ws) {
    extern __shared__ uint32_t sm[];
    const int nwc = TC / 32;
    uint32_t* bm = sm;                     // [E][nwc]
    uint32_t* run = sm + (size_t)E * nwc;  // [E] running count
    uint32_t* pre = run + E;               // [E][nwc] prefix popcounts
    uint32_t* offl = pre + (size_t)E * nwc;  // [E] expert row offsets
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += 1024) run[e] = 0;
    __syncthreads();
    // pass 1: counts
    for (int i = tid; i < T * topk; i += 1024) {
        const int e = sel[i];
        if (e >= 0 && e < E) atomicAdd(&run[e], 1u);
    }
    __syncthreads();
    if (tid == 0) {
        int acc = 0, nt = 0;
        for (int e = 0; e < E; ++e) {
            const int c = (int)run[e];
            ws.cnt[e] = c;
            ws.off[e] = acc;
            offl[e] = (uint32_t)acc;
            for (int r = 0; r < c; r += GBM) { ws.tile_e[nt] = e; ws.tile_r[nt] = r; ++nt; }
            acc += c;
        }
        ws.off[E] = acc;
        ws.ntile[0] = nt;
    }
    __syncthreads();
    for (int e = tid; e < E; e += 1024) run[e] = 0;
    __syncthreads();
    // pass 2: ranks, chunk by chunk of TC tokens
    for (int t0 = 0; t0 < T; t0 += TC) {
        const int tn = min(TC, T - t0);
        for (int i = tid; i < E * nwc; i += 1024) bm[i] = 0;
        __syncthreads();
        for (int i = tid; i < tn * topk; i += 1024) {
            const int tt = i / topk, e = sel[(size_t)t0 * topk + i];
            if (e >= 0 && e < E) atomicOr(&bm[(size_t)e * nwc + (tt >> 5)], 1u << (tt & 31));
        }
        __syncthreads();
        for (int e = tid; e < E; e += 1024) {
            uint32_t acc = run[e];
            for (int w = 0; w < nwc; ++w) {
                pre[(size_t)e * nwc + w] = acc;
                acc += __popc(bm[(size_t)e * nwc + w]);
            }
            run[e] = acc;
        }
        __syncthreads();
        for (int i = tid; i < tn * topk; i += 1024) {
            const int tt = i / topk, e = sel[(size_t)t0 * topk + i];
            if (e < 0 || e >= E) continue;
            const uint32_t word = bm[(size_t)e * nwc + (tt >> 5)];
            const uint32_t rank = pre[(size_t)e * nwc + (tt >> 5)] + __popc(word & ((1u << (tt & 31)) - 1u));
            const int prow = (int)offl[e] + (int)rank;
            ws.pos[(size_t)t0 * topk + i] = prow;
            ws.ptok[prow] = t0 + tt;
        }
        __syncthreads();
    }
}

// ---- grouped W8A32 GEMM: Y[prow, :] = X[row(prow), :] . (q[e] * s[e]) ------
// X rows: gather ? x[ptok[prow]] : xin[prow]; weights (E, K, N) i8 row-major.
__global__ __launch_bounds__(256) void grouped_gemm_kernel(
    const float* __restrict__ xin, int gather, const int32_t* __restrict__ ptok,
    const int8_t* __restrict__ q, const float* __restrict__ qs, int K, int N,
    const int32_t* __restrict__ off, const int32_t* __restrict__ cnt,
    const int32_t* __restrict__ tile_e, const int32_t* __restrict__ tile_r,
    const int32_t* __restrict__ ntile, float* __restrict__ y) {
    __shared__ float As[GKC][GBM + 4];
    __shared__ float Bs[GKC][GBN];
    const int tix = blockIdx.x;
    if (tix >= ntile[0]) return;
    const int e = tile_e[tix], r0 = tile_r[tix];
    const int rows = min(GBM, cnt[e] - r0);
    const int n0 = blockIdx.y * GBN;
    const int tid = threadIdx.x;
    const int tr = tid / 16, tc = tid % 16;   // 16 x 16 threads: 2 rows x 4 cols
    const int8_t* qe = q + (size_t)e * K * N;
    const float* se = qs + (size_t)e * N;
    const int pbase = off[e] + r0;
    float acc[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
    for (int k0 = 0; k0 < K; k0 += GKC) {
        // stage A^T (GKC x GBM) and dequantised B (GKC x GBN)
        for (int i = tid; i < GKC * GBM; i += 256) {
            const int r = i / GKC, kk = i % GKC;
            float v = 0.0f;
            if (r < rows && k0 + kk < K) {
                const int prow = pbase + r;
                const float* xr = gather ? xin + (size_t)ptok[prow] * K : xin + (size_t)prow * K;
                v = xr[k0 + kk];
            }
            As[kk][r] = v;
        }
        for (int i = tid; i < GKC * GBN; i += 256) {
            const int kk = i / GBN, c = i % GBN;
            float v = 0.0f;
            if (k0 + kk < K && n0 + c < N)
                v = (float)qe[(size_t)(k0 + kk) * N + n0 + c] * se[n0 + c];
            Bs[kk][c] = v;
        }
        __syncthreads();
        const int kn = min(GKC, K - k0);
        for (int kk = 0; kk < kn; ++kk) {
            const float a0 = As[kk][tr * 2], a1 = As[kk][tr * 2 + 1];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float b = Bs[kk][tc * 4 + c];
                acc[0][c] = __builtin_fmaf(a0, b, acc[0][c]);
                acc[1][c] = __builtin_fmaf(a1, b, acc[1][c]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int rr = tr * 2 + r;
        if (rr >= rows) continue;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int j = n0 + tc * 4 + c;
            if (j < N) y[(size_t)(pbase + rr) * N + j] = acc[r][c];
        }
    }
}

__global__ void act_kernel(const float* __restrict__ g, const float* __restrict__ u,
                           int act, int mi, int gw, const int32_t* __restrict__ off,
                           int E, float* __restrict__ h) {
    const int P = off[E];
    const size_t total = (size_t)P * mi;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / mi, c = i % mi;
        if (act == FRQ_ACT_SILU)
            h[i] = silu(g[r * gw + c]) * u[i];
        else
            h[i] = gelu_tanh(g[r * gw + c]) * g[r * gw + c + mi];
    }
}

__global__ void combine_kernel(const float* __restrict__ dn, const int32_t* __restrict__ sel,
                               const float* __restrict__ w, const int32_t* __restrict__ pos,
                               int topk, int d, float* __restrict__ out) {
    const int t = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= d) return;
    // the token's slots in ascending expert id (experts within a token are
    // distinct: top-k of a permutation)
    const int32_t* st = sel + (size_t)t * topk;
    float acc = 0.0f;
    int last = -1;
    for (int i = 0; i < topk; ++i) {
        int best = -1, be = 0x7FFFFFFF;
        for (int q = 0; q < topk; ++q) {
            const int ev = st[q];
            if (ev > last && ev < be) { be = ev; best = q; }
        }
        if (best < 0) break;
        last = be;
        acc = acc + w[(size_t)t * topk + best] * dn[(size_t)pos[(size_t)t * topk + best] * d + c];
    }
    out[(size_t)t * d + c] = acc;
}

}  // namespace

size_t moe_ws_bytes(const MoeBank& b, size_t T, size_t topk) {
    const size_t P = T * topk, E = b.n_exp, nt = ntile_max(T, topk, E);
    auto r = [](size_t x) { return round_up(x, 256); };
    return r(P * 4) * 4 + r(E * 4) + r((E + 1) * 4) + r(nt * 4) * 2 + r(4) +
           r(P * b.gw * 4) + r(P * b.mi * 4) * 2 + r(P * b.d * 4);
}

hipError_t launch_moe_route(const float* logits, size_t T, size_t E,
                            size_t topk, int norm_topk, const float* pes,
                            int32_t* sel, float* w, int* err, hipStream_t s) {
    const size_t lds = 4 * E * sizeof(float);
    route_kernel<<<dim3((unsigned)((T + 3) / 4)), dim3(256), lds, s>>>(
        logits, (int)T, (int)E, (int)topk, norm_topk, pes, sel, w, err);
    return hipGetLastError();
}

hipError_t launch_moe(const MoeBank& b, const float* x, size_t T,
                      const float* logits, size_t topk, int norm_topk,
                      const float* pes, float* out, void* wsp, int* err,
                      hipStream_t s) {
    if (T == 0) return hipSuccess;
    MoeWs ws = moe_view(wsp, b, T, topk);
    const int E = (int)b.n_exp, d = (int)b.d, mi = (int)b.mi, gw = (int)b.gw;
    hipError_t e = launch_moe_route(logits, T, b.n_exp, topk, norm_topk, pes, ws.sel, ws.w, err, s);
    if (e != hipSuccess) return e;
    const size_t dlds = ((size_t)E * (TC / 32) * 2 + 2 * E) * sizeof(uint32_t);
    dispatch_kernel<<<dim3(1), dim3(1024), dlds, s>>>(ws.sel, (int)T, (int)topk, E, ws);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const unsigned nt = (unsigned)ntile_max(T, topk, b.n_exp);
    grouped_gemm_kernel<<<dim3(nt, (unsigned)((gw + GBN - 1) / GBN)), dim3(256), 0, s>>>(
        x, 1, ws.ptok, b.gate, b.gate_s, d, gw, ws.off, ws.cnt, ws.tile_e, ws.tile_r, ws.ntile, ws.g);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (b.act == FRQ_ACT_SILU) {
        grouped_gemm_kernel<<<dim3(nt, (unsigned)((mi + GBN - 1) / GBN)), dim3(256), 0, s>>>(
            x, 1, ws.ptok, b.up, b.up_s, d, mi, ws.off, ws.cnt, ws.tile_e, ws.tile_r, ws.ntile, ws.u);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    act_kernel<<<dim3(1024), dim3(256), 0, s>>>(ws.g, ws.u, b.act, mi, gw, ws.off, E, ws.h);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    grouped_gemm_kernel<<<dim3(nt, (unsigned)((d + GBN - 1) / GBN)), dim3(256), 0, s>>>(
        ws.h, 0, ws.ptok, b.down, b.down_s, mi, d, ws.off, ws.cnt, ws.tile_e, ws.tile_r, ws.ntile, ws.dn);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    combine_kernel<<<dim3((unsigned)((d + 255) / 256), (unsigned)T), dim3(256), 0, s>>>(
        ws.dn, ws.sel, ws.w, ws.pos, (int)topk, d, out);
    return hipGetLastError();
}

// expert_mm for one expert: a single tile list built on the host.
__global__ void expert_mm_kernel(const float* __restrict__ x, int m, const int8_t* __restrict__ q,
                                 const float* __restrict__ s, int K, int N, float* __restrict__ y) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    const int i = blockIdx.y;
    if (j >= N || i >= m) return;
    float acc = 0.0f;
    for (int k = 0; k < K; ++k)
        acc = __builtin_fmaf(x[(size_t)i * K + k], (float)q[(size_t)k * N + j] * s[j], acc);
    y[(size_t)i * N + j] = acc;
}

hipError_t launch_expert_mm(const int8_t* q, const float* s, size_t inp,
                            size_t out, const float* x, size_t m, float* y,
                            hipStream_t st) {
    if (m == 0) return hipSuccess;
    expert_mm_kernel<<<dim3((unsigned)((out + 255) / 256), (unsigned)m), dim3(256), 0, st>>>(
        x, (int)m, q, s, (int)inp, (int)out, y);
    return hipGetLastError();
}

}  // namespace frq
