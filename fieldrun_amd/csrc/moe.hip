// moe.hip — routed MoE expert layer (gfx950).
//
// Restates the routed branch of /root/reference/src/qwen3moe.rs:120-158
// (act SiLU) and the expert part of src/gemma4.rs:131-187 (act gelu_tanh,
// packed gate_up, per_expert_scale), with the experts' matmuls as in
// expert_f32 / expert_mm (src/bundle.rs:404-461): W8A32, y = x . (q * s[j]).
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
//             gives the rank); plus the list of (expert, row0) tiles.
//   digits    each token row of x as X = round(x / s), s = max|x| /
//             (127 * 2^16), |X| <= 127 * 2^16, split into three int8 digits
//             X = d2*2^16 + d1*2^8 + d0 (a 24-bit fixed point per row).
//   gemm      grouped GEMM over the tile list on v_mfma_i32_16x16x64_i8: the
//             A rows of a token group are its tokens' three digit rows, B is
//             the expert's weight in the blocked MFMA-operand layout (built
//             at upload), so C_d = D_d . Q is exact in int32 over all of K
//             (|C| < 127 * 127 * K) and y = s * (C2*2^16 + C1*2^8 + C0) * s[j].
//             The rounding of x to 24 bits keeps y within ~1e-7 of
//             max|x| * sum|q*s|; a row with a non-finite or extreme value
//             takes expert_mm's own f32 sum (a.dot's blocked order).
//   act       h = silu(g) * u   or   gelu_tanh(g[:mi]) * g[mi:], written
//             directly as the digits (and f32 copy) the down GEMM reads.
//   combine   out[t,:] = sum over t's experts in ascending expert id of
//             w * down (mul then add from +0): the reference adds in HashMap
//             order, which is random per process; ascending id is one of
//             its orders.
#include "frq_internal.h"
#include "libm_f32.h"

#include <algorithm>

namespace frq {

namespace {

constexpr float XMAXD = 8323072.0f;  // 127 * 2^16: |X| of a 24-bit row digit triple

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
    int8_t* xd;        // [T][3][kpd] digits of x
    float* xso;        // [T]      their scales (-1: exact row)
    float* g;          // [T*k, gw]
    float* u;          // [T*k, mi]
    float* h;          // [T*k, mi]
    int8_t* hd;        // [T*k][3][kpm] digits of h
    float* hso;        // [T*k]
    float* dn;         // [T*k, d]
};

// Tiles of tr rows per expert: sum over experts of ceil(cnt / tr) is at most
// T*k / tr plus one per active expert.
size_t ntile_max(size_t T, size_t k, size_t E, size_t tr) {
    const size_t P = T * k;
    return P / tr + (E < P ? E : P) + 1;
}

size_t moe_tile_rows(size_t T) { return T <= 4 ? 4 : 32; }

MoeWs moe_view(void* base, const MoeBank& b, size_t T, size_t k) {
    const size_t P = T * k, E = b.n_exp, nt = ntile_max(T, k, E, moe_tile_rows(T));
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
    v.xd = (int8_t*)take(T * 3 * b.kpd);
    v.xso = (float*)take(T * 4);
    v.g = (float*)take(P * b.gw * 4);
    v.u = (float*)take(P * b.mi * 4);
    v.h = (float*)take(P * b.mi * 4);
    v.hd = (int8_t*)take(P * 3 * b.kpm);
    v.hso = (float*)take(P * 4);
    v.dn = (float*)take(P * b.d * 4);
    return v;
}

// y_j = x . (q[:, j] * s) over K in a.dot's order (expert_mm's x.dot(&wv):
// MM_KC-long k blocks, each an FMA chain from +0, added in order), q an
// (in, out) int8 matrix with row pitch ldq: the exact rows, whose digits
// cannot carry the activations.
__device__ __forceinline__ float exact_col(const float* __restrict__ x, const int8_t* __restrict__ q, int ldq, int j,
                                           float s, int K) {
    float c = 0.0f;
    for (int k0 = 0; k0 < K; k0 += MM_KC) {
        float ab = 0.0f;
        for (int k = k0; k < min(K, k0 + MM_KC); ++k) ab = __builtin_fmaf(x[k], (float)q[(size_t)k * ldq + j] * s, ab);
        c = c + ab;
    }
    return c;
}

// The gates and the softmax use the restated glibc expf / fdlibm tanhf
// (libm_f32.h), which Rust's f32::exp / f32::tanh reach on the reference's
// host, so route weights and gated activations are the reference's bits.
// (frq_expf_sel: frq_expf's value for every input, with selects for its
// special cases instead of branches)
__device__ __forceinline__ float silu(float x) { return x / (1.0f + libm::frq_expf_sel(-x)); }

__device__ __forceinline__ float gelu_tanh(float x) {
    const float c = sqrtf(2.0f / 3.14159274101257324f);
    return 0.5f * x * (1.0f + libm::frq_tanhf(c * (x + 0.044715f * x * x * x)));
}

// ---- routing: one wave per token ----------------------------------------
// Wave-wide max of a float (every lane gets it), VALU lane exchanges only.
__device__ __forceinline__ float wave_fmax(float v) {
    v = fmaxf(v, __uint_as_float(xshfl<1>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(xshfl<2>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(xshfl<4>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(xshfl<8>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(xshfl<16>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(xshfl<32>(__float_as_uint(v))));
    return v;
}

// A row has no probabilities the reference can sort when a logit is NaN or
// the max is +-inf (inf - inf in an exponent makes every p NaN): its
// partial_cmp().unwrap() panics.  The picks are then experts 0..k-1 with
// weight 0, and the caller raises the error.
__device__ __forceinline__ void route_fail(int topk, int* pe, float* pw) {
    for (int i = threadIdx.x & 63; i < topk; i += 64) { pe[i] = i; pw[i] = 0.0f; }
    wave_sync();
}

// The sequential sum p[0] + ... + p[E-1] from +0 (the reference's order),
// the same chain in every lane; reads batched ahead of it where p is
// 16-byte aligned.
__device__ __forceinline__ float route_sum(const float* p, int E) {
    if ((reinterpret_cast<uintptr_t>(p) & 15) == 0) return lds_seq_sum(p, E, 0.0f);
    float s = 0.0f;
    for (int e = 0; e < E; ++e) s = s + p[e];
    return s;
}

// Renormalised weights, one pick per lane (each the same operations as a
// sequential pass): p / denom (when renormalising) then * per_expert_scale.
__device__ __forceinline__ void route_weights(int topk, int norm_topk, const float* __restrict__ pes,
                                              float denom, const int* pe, float* pw) {
    const bool renorm = norm_topk || pes != nullptr;
    for (int i = threadIdx.x & 63; i < topk; i += 64) {
        float w = renorm ? pw[i] / denom : pw[i];
        if (pes) w = w * pes[pe[i]];
        pw[i] = w;
    }
    wave_sync();
}

// Routing of one token by one wave, E <= 64 * NC: the probabilities stay
// in registers (expert lane + 64 c in chunk c); softmax (max, exp,
// sequential sum, divide), then k rounds of arg-max by (p desc, expert
// asc): the wave max of p, and the lowest expert holding it from one
// ballot per chunk (chunks ascend in expert id).  p: E floats of LDS (the
// sum's operand); picks go to pe / pw (k entries of LDS, pick order).
// Returns true (uniformly) for a row the reference cannot sort.
template <int NC>
__device__ bool route_wave_r(const float* __restrict__ row, int E, int topk, int norm_topk,
                             const float* __restrict__ pes, float* p, int* pe, float* pw) {
    const int lane = threadIdx.x & 63;
    float v[NC];
    float m = -INFINITY;
    bool nan = false;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int e = lane + 64 * c;
        v[c] = e < E ? row[e] : -INFINITY;
        nan |= v[c] != v[c];
        m = fmaxf(m, v[c]);
    }
    m = wave_fmax(m);
    if (__builtin_amdgcn_ballot_w64(nan) != 0 || !(fabsf(m) <= 3.40282347e38f)) {
        route_fail(topk, pe, pw);
        return true;
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int e = lane + 64 * c;
        if (e < E) {
            v[c] = libm::frq_expf(v[c] - m);
            p[e] = v[c];
        }
    }
    wave_sync();
    const float s = route_sum(p, E);
    // taken experts become -1, lanes past E -2: both below every p >= +0
#pragma unroll
    for (int c = 0; c < NC; ++c) v[c] = lane + 64 * c < E ? v[c] / s : -2.0f;
    float denom = -0.0f;
    for (int i = 0; i < topk; ++i) {
        float bl = v[0];
#pragma unroll
        for (int c = 1; c < NC; ++c) bl = fmaxf(bl, v[c]);
        const float bv = wave_fmax(bl);
        int be = -1;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const unsigned long long msk = __builtin_amdgcn_ballot_w64(v[c] == bv);
            if (be < 0 && msk != 0) be = 64 * c + __builtin_ctzll(msk);
        }
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (be == lane + 64 * c) v[c] = -1.0f;
        if (lane == 0) {
            pe[i] = be;
            pw[i] = bv;
        }
        denom = denom + bv;
    }
    wave_sync();
    route_weights(topk, norm_topk, pes, denom, pe, pw);
    return false;
}

// Any E: the probabilities in LDS p (E floats), arg-max rounds over them.
__device__ bool route_wave_lds(const float* __restrict__ row, int E, int topk, int norm_topk,
                               const float* __restrict__ pes, float* p, int* pe, float* pw) {
    const int lane = threadIdx.x & 63;
    float m = -INFINITY;
    bool nan = false;
    for (int e = lane; e < E; e += 64) {
        const float v = row[e];
        nan |= v != v;
        m = fmaxf(m, v);
    }
    m = wave_fmax(m);
    if (__builtin_amdgcn_ballot_w64(nan) != 0 || !(fabsf(m) <= 3.40282347e38f)) {
        route_fail(topk, pe, pw);
        return true;
    }
    for (int e = lane; e < E; e += 64) p[e] = libm::frq_expf(row[e] - m);
    wave_sync();
    const float s = route_sum(p, E);
    wave_sync();
    for (int e = lane; e < E; e += 64) p[e] = p[e] / s;
    wave_sync();
    // k rounds of arg-max by (p desc, e asc); taken experts get p = -1
    float denom = -0.0f;
    for (int i = 0; i < topk; ++i) {
        float bv = -2.0f;
        int be = 0x7FFFFFFF;
        for (int e = lane; e < E; e += 64) {
            const float v = p[e];
            if (v > bv || (v == bv && e < be)) { bv = v; be = e; }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const int oe = __shfl_xor(be, off, 64);
            if (ov > bv || (ov == bv && oe < be)) { bv = ov; be = oe; }
        }
        if (lane == 0) {
            pe[i] = be;
            pw[i] = bv;
            p[be] = -1.0f;
        }
        wave_sync();
        denom = denom + bv;
    }
    route_weights(topk, norm_topk, pes, denom, pe, pw);
    return false;
}

// Routing of one token by one wave (see route_wave_r); picks in pick order.
__device__ bool route_wave(const float* __restrict__ row, int E, int topk, int norm_topk,
                           const float* __restrict__ pes, float* p, int* pe, float* pw) {
    if (E <= 64) return route_wave_r<1>(row, E, topk, norm_topk, pes, p, pe, pw);
    if (E <= 128) return route_wave_r<2>(row, E, topk, norm_topk, pes, p, pe, pw);
    if (E <= 256) return route_wave_r<4>(row, E, topk, norm_topk, pes, p, pe, pw);
    return route_wave_lds(row, E, topk, norm_topk, pes, p, pe, pw);
}

// One wave per token (4 per workgroup); every step stays inside the wave.
__global__ __launch_bounds__(256) void route_kernel(
    const float* __restrict__ logits, int T, int E, int topk, int norm_topk,
    const float* __restrict__ pes, int32_t* __restrict__ sel,
    float* __restrict__ wout, int* __restrict__ err) {
    extern __shared__ __attribute__((aligned(16))) float sp[];  // [4][E] probabilities, [4][topk] picks (expert, w)
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wv;
    if (t >= T) return;  // whole waves only
    int* pe = reinterpret_cast<int*>(sp + 4 * E) + wv * topk;
    float* pw = sp + 4 * E + 4 * topk + wv * topk;
    const bool bad = route_wave(logits + (size_t)t * E, E, topk, norm_topk, pes, sp + wv * E, pe, pw);
    if (bad && lane == 0) atomicOr(err, 1);
    for (int i = lane; i < topk; i += 64) {
        sel[(size_t)t * topk + i] = pe[i];
        wout[(size_t)t * topk + i] = pw[i];
    }
}

// ---- dispatch: one workgroup of 1024 threads ------------------------------
constexpr int TC = 1024;  // tokens per bitmap chunk

__global__ __launch_bounds__(1024) void dispatch_kernel(
    const int32_t* __restrict__ sel, int T, int topk, int E, int tr,
    MoeWs ws) {
    extern __shared__ uint32_t sm[];
    const int nwc = (min(T, TC) + 31) / 32;  // bitmap words per expert and chunk
    uint32_t* bm = sm;                     // [E][nwc]
    uint32_t* run = sm + (size_t)E * nwc;  // [E] running count
    uint32_t* pre = run + E;               // [E][nwc] prefix popcounts
    uint32_t* offl = pre + (size_t)E * nwc;  // [E] expert row offsets
    uint32_t* toff = offl + E;               // [E] expert tile offsets
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += 1024) run[e] = 0;
    __syncthreads();
    // pass 1: counts
    for (int i = tid; i < T * topk; i += 1024) {
        const int e = sel[i];
        if (e >= 0 && e < E) atomicAdd(&run[e], 1u);
    }
    __syncthreads();
    // row and tile offsets: exclusive scans over the experts by wave 0, 64
    // experts a step
    if (tid < 64) {
        int cr = 0, ct = 0;  // running totals of the steps before
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int e = e0 + tid;
            const int c = e < E ? (int)run[e] : 0, nt = (c + tr - 1) / tr;
            int ic = c, it = nt;  // inclusive scans
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int yc = __shfl_up(ic, o, 64), yt = __shfl_up(it, o, 64);
                if (tid >= o) { ic += yc; it += yt; }
            }
            if (e < E) {
                ws.cnt[e] = c;
                ws.off[e] = cr + ic - c;
                offl[e] = (uint32_t)(cr + ic - c);
                toff[e] = (uint32_t)(ct + it - nt);
            }
            cr += __shfl(ic, 63, 64);
            ct += __shfl(it, 63, 64);
        }
        if (tid == 0) {
            ws.off[E] = cr;
            ws.ntile[0] = ct;
        }
    }
    __syncthreads();
    // the tile list: (expert, first row) in ascending expert, then row
    for (int e = tid; e < E; e += 1024) {
        const int c = (int)run[e];
        int t = (int)toff[e];
        for (int r = 0; r < c; r += tr, ++t) { ws.tile_e[t] = e; ws.tile_r[t] = r; }
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

// ---- 24-bit row digits ------------------------------------------------------
// Digits of one f32 row v[0..K) into D[3][Kp] (d2, d1, d0; zero padding) and
// its scale; -1 when the row holds a non-finite value or its scale leaves
// [1e-30, 1e28] (|y| <= 127 * 127 * K * s must stay finite).  256 threads.
__device__ void row_digits(const float* __restrict__ v, int K, int Kp, int8_t* __restrict__ D,
                           float* __restrict__ so_out, float* red) {
    const int tid = threadIdx.x;
    float mx = 0.0f;
    int nf = 0;
    for (int k = tid; k < K; k += 256) {
        const float x = v[k];
        nf |= !(fabsf(x) <= 3.0e38f);
        mx = fmaxf(mx, fabsf(x));
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        nf |= __shfl_xor(nf, o, 64);
    }
    if ((tid & 63) == 0) { red[tid >> 6] = mx; red[4 + (tid >> 6)] = (float)nf; }
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    nf = (red[4] + red[5] + red[6] + red[7]) != 0.0f;
    const float s = mx > 0.0f ? mx / XMAXD : 1.0f;
    const bool ok = !nf && s >= 1.0e-30f && s <= 1.0e28f;
    const float r = 1.0f / s;  // any rounding of x / s keeps |x - s X| <= ~s/2
    for (int k = tid; k < Kp; k += 256) {
        int d2 = 0, d1 = 0, d0 = 0;
        if (ok && k < K) {
            float xf = rintf(v[k] * r);
            xf = fminf(fmaxf(xf, -XMAXD), XMAXD);
            const int X = (int)xf;
            d0 = (int)(int8_t)(X & 0xFF);
            const int X1 = (X - d0) >> 8;
            d1 = (int)(int8_t)(X1 & 0xFF);
            d2 = (X1 - d1) >> 8;
        }
        D[k] = (int8_t)d2;
        D[Kp + k] = (int8_t)d1;
        D[2 * Kp + k] = (int8_t)d0;
    }
    if (tid == 0) *so_out = ok ? s : -1.0f;
}

// row_digits over values produced by val(k), held in registers (thread
// tid takes k = tid + 256 i): one pass over the source, Kp <= 256 * NV.
template <int NV, typename F>
__device__ __forceinline__ void row_digits_r(F val, int K, int Kp, int8_t* __restrict__ D,
                                             float* __restrict__ so_out, float* red) {
    const int tid = threadIdx.x;
    float v[NV];
    float mx = 0.0f;
    bool nf = false;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int k = tid + 256 * i;
        v[i] = k < K ? val(k) : 0.0f;
        nf |= !(fabsf(v[i]) <= 3.0e38f);
        mx = fmaxf(mx, fabsf(v[i]));
    }
    mx = wave_fmax(mx);
    const bool wnf = __builtin_amdgcn_ballot_w64(nf) != 0;
    if ((tid & 63) == 0) { red[tid >> 6] = mx; red[4 + (tid >> 6)] = wnf ? 1.0f : 0.0f; }
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const bool anf = (red[4] + red[5] + red[6] + red[7]) != 0.0f;
    const float s = mx > 0.0f ? mx / XMAXD : 1.0f;
    const bool ok = !anf && s >= 1.0e-30f && s <= 1.0e28f;
    const float r = 1.0f / s;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int k = tid + 256 * i;
        if (k >= Kp) break;
        int d2 = 0, d1 = 0, d0 = 0;
        if (ok && k < K) {
            float xf = rintf(v[i] * r);
            xf = fminf(fmaxf(xf, -XMAXD), XMAXD);
            const int X = (int)xf;
            d0 = (int)(int8_t)(X & 0xFF);
            const int X1 = (X - d0) >> 8;
            d1 = (int)(int8_t)(X1 & 0xFF);
            d2 = (X1 - d1) >> 8;
        }
        D[k] = (int8_t)d2;
        D[Kp + k] = (int8_t)d1;
        D[2 * Kp + k] = (int8_t)d0;
    }
    if (tid == 0) *so_out = ok ? s : -1.0f;
}

constexpr int RD_NV = 8;  // register-held rows: Kp <= 2048

// row_digits_r with the fewest registers that hold the row (Kp <= 2048)
template <typename F>
__device__ __forceinline__ void row_digits_nv(F val, int K, int Kp, int8_t* __restrict__ D,
                                              float* __restrict__ so_out, float* red) {
    switch ((Kp + 255) / 256) {
        case 1: row_digits_r<1>(val, K, Kp, D, so_out, red); break;
        case 2: row_digits_r<2>(val, K, Kp, D, so_out, red); break;
        case 3: row_digits_r<3>(val, K, Kp, D, so_out, red); break;
        case 4: row_digits_r<4>(val, K, Kp, D, so_out, red); break;
        case 5: case 6: row_digits_r<6>(val, K, Kp, D, so_out, red); break;
        default: row_digits_r<8>(val, K, Kp, D, so_out, red); break;
    }
}

// One workgroup per token row of x.
__global__ __launch_bounds__(256) void x_digits_kernel(const float* __restrict__ x, int K, int Kp,
                                                       int8_t* __restrict__ D, float* __restrict__ so) {
    __shared__ float red[8];
    const int r = blockIdx.x;
    const float* xr = x + (size_t)r * K;
    if (Kp <= 256 * RD_NV)
        row_digits_nv([&](int k) { return xr[k]; }, K, Kp, D + (size_t)r * 3 * Kp, so + r, red);
    else
        row_digits(xr, K, Kp, D + (size_t)r * 3 * Kp, so + r, red);
}

// h = silu(g) * u  or  gelu_tanh(g[:mi]) * g[mi:], one workgroup per
// permuted row (rows >= off[E] are idle): the f32 row (for the exact path)
// and its digits.
__global__ __launch_bounds__(256) void act_digits_kernel(
    const float* __restrict__ g, const float* __restrict__ u, int act, int mi, int gw, int kpm,
    const int32_t* __restrict__ off, int E, float* __restrict__ h, int8_t* __restrict__ hd,
    float* __restrict__ hso) {
    __shared__ float red[8];
    const int r = blockIdx.x;
    if (r >= off[E]) return;  // uniform
    const float* gr = g + (size_t)r * gw;
    float* hr = h + (size_t)r * mi;
    if (kpm <= 256 * RD_NV) {
        row_digits_nv(
            [&](int c) {
                const float hv = act == FRQ_ACT_SILU ? silu(gr[c]) * u[(size_t)r * mi + c]
                                                     : gelu_tanh(gr[c]) * gr[c + mi];
                hr[c] = hv;
                return hv;
            },
            mi, kpm, hd + (size_t)r * 3 * kpm, hso + r, red);
        return;
    }
    for (int c = threadIdx.x; c < mi; c += 256)
        hr[c] = act == FRQ_ACT_SILU ? silu(gr[c]) * u[(size_t)r * mi + c] : gelu_tanh(gr[c]) * gr[c + mi];
    __syncthreads();
    row_digits(hr, mi, kpm, hd + (size_t)r * 3 * kpm, hso + r, red);
}

// ---- grouped digit GEMM: Y[prow, :] = X[src(prow), :] . (q[e] * s[e]) -------
// Workgroup = (tile of 4*TG rows of one expert, CB column blocks of 16);
// its KS waves split the k-blocks and add their int32 accumulators through
// LDS (exact in any order).  A operand of token group t: lane 16g + 4tl + d
// holds digit d of row 4t + tl, k-bytes 16g..16g+15 of the k-block; C lane
// l holds rows 4(l/16) + c, i.e. row 4t + l/16, digit c.  src = ptok[prow]
// when gather (rows of x), else prow (rows of h).
template <int TG, int CB, int KS>
__global__ __launch_bounds__(64 * KS) void moe_mm_kernel(
    const int8_t* __restrict__ D, const float* __restrict__ dso, int Kp, int gather,
    const int32_t* __restrict__ ptok, const int8_t* __restrict__ Wb, int Np,
    const float* __restrict__ wsc, int N, const float* __restrict__ xf, int K,
    const int8_t* __restrict__ wkn, const int32_t* __restrict__ off,
    const int32_t* __restrict__ cnt, const int32_t* __restrict__ tile_e,
    const int32_t* __restrict__ tile_r, const int32_t* __restrict__ ntile,
    float* __restrict__ y) {
    constexpr int TR = 4 * TG;
    __shared__ v4i red[KS > 1 ? KS - 1 : 1][TG][CB][64];
    const int tix = blockIdx.x;
    if (tix >= ntile[0]) return;  // uniform
    const int e = tile_e[tix], r0 = tile_r[tix];
    const int rows = min(TR, cnt[e] - r0);
    const int pbase = off[e] + r0;
    const int nb0 = blockIdx.y * CB;
    const int lane = threadIdx.x & 63;
    const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nkb = Kp / 64;
    const int kb0 = nkb * ks / KS, kb1 = nkb * (ks + 1) / KS;
    const int rr = lane & 15, tl = rr >> 2, dg = rr & 3, kq = lane >> 4;
    const int8_t* arow[TG];
    bool aval[TG];
#pragma unroll
    for (int t = 0; t < TG; ++t) {
        const int i = 4 * t + tl;
        aval[t] = i < rows && dg < 3;
        const int prow = pbase + min(i, rows - 1);
        const int src = gather ? ptok[prow] : prow;
        arow[t] = D + ((size_t)src * 3 + (dg < 3 ? dg : 0)) * Kp + 16 * kq;
    }
    const int8_t* wb = Wb + (size_t)e * Np * Kp + (size_t)nb0 * 1024 + lane * 16;
    const size_t kstride = (size_t)(Np / 16) * 1024;
    v4i acc[TG][CB];
#pragma unroll
    for (int t = 0; t < TG; ++t)
#pragma unroll
        for (int c = 0; c < CB; ++c) acc[t][c] = v4i{0, 0, 0, 0};
    // U k-blocks per step, all of their loads issued before the MFMAs
    constexpr int U = (TG + CB <= 2) ? 8 : 2;
    for (int kb = kb0; kb < kb1; kb += U) {
        v4i av[U][TG], bv[U][CB];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool in = kb + u < kb1;
#pragma unroll
            for (int t = 0; t < TG; ++t)
                av[u][t] = (in && aval[t]) ? *reinterpret_cast<const v4i*>(arow[t] + (size_t)(kb + u) * 64)
                                           : v4i{0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c < CB; ++c)
                bv[u][c] = in ? *reinterpret_cast<const v4i*>(wb + (size_t)(kb + u) * kstride + (size_t)c * 1024)
                              : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int t = 0; t < TG; ++t)
#pragma unroll
                for (int c = 0; c < CB; ++c)
                    acc[t][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[u][t], bv[u][c], acc[t][c], 0, 0, 0);
    }
    if (KS > 1) {
        if (ks > 0) {
#pragma unroll
            for (int t = 0; t < TG; ++t)
#pragma unroll
                for (int c = 0; c < CB; ++c) red[ks - 1][t][c][lane] = acc[t][c];
        }
        __syncthreads();
        if (ks > 0) return;
#pragma unroll
        for (int q = 0; q < KS - 1; ++q)
#pragma unroll
            for (int t = 0; t < TG; ++t)
#pragma unroll
                for (int c = 0; c < CB; ++c) acc[t][c] += red[q][t][c][lane];
    }
    // y = s * (C2 * 2^16 + C1 * 2^8 + C0) * wsc[e, j]; rows whose digits do not
    // carry them take expert_mm's own sum x . (q * s), a.dot's order
    const int col = lane & 15, tok = lane >> 4;
    const float* __restrict__ se = wsc + (size_t)e * N;
#pragma unroll
    for (int t = 0; t < TG; ++t) {
        const int i = 4 * t + tok;
        if (i >= rows) continue;
        const int prow = pbase + i;
        const int src = gather ? ptok[prow] : prow;
        const float so = dso[src];
#pragma unroll
        for (int c = 0; c < CB; ++c) {
            const int j = (nb0 + c) * 16 + col;
            if (j >= N) continue;
            float v;
            if (so >= 0.0f) {
                const v4i a4 = acc[t][c];
                v = so * ((float)a4[0] * 65536.0f + ((float)a4[1] * 256.0f + (float)a4[2])) * se[j];
            } else {
                v = exact_col(xf + (size_t)src * K, wkn + (size_t)e * K * N, N, j, se[j], K);
            }
            y[(size_t)prow * N + j] = v;
        }
    }
}

// ---- expert-stationary grouped digit GEMM (batched rows) -------------------
// Workgroup = (tile of up to 32 permuted rows of one expert, 128 columns):
// the expert's 128-column weight block streams from HBM once per tile, each
// of the 4 waves taking 32 columns (two 16-column blocks); the tile's digit
// rows pass through LDS GM_KC k-blocks at a time (double-buffered), and
// every A operand read from LDS feeds two MFMAs.  The A items and B operands of
// k-block kb sit in register slot kb % GM_BP from their load until use, so
// both stream GM_BP k-blocks ahead (the wait counter is in order: A, needed
// first, must not trail B).  Every load is unconditional, from a clamped
// address, so the waits stay exact.  A operand of row group g: lane
// 16 kq + 4 tl + d holds digit d of row 4 g + tl, k-bytes 16 kq..16 kq + 15
// of the k-block (LDS keeps the 48 lanes d < 3; d = 3 reads a copy of
// d = 2, whose product row acc[3] is not used); C lane l holds row
// 4 g + l / 16, digit c in acc[c], column l % 16.  Output as
// moe_mm_kernel's.  NGT = row groups the tile's rows need (4 or 8); 32-row
// tiles and a ring 3 deep fit a wave in 160 registers, three workgroups a
// CU (the MFMA issue waits on latency: occupancy is what hides it).
constexpr int GM_TR = 32;  // rows a tile
constexpr int GM_BP = 3;   // k-blocks of A and B in flight a wave
constexpr int GM_KC = 1;   // k-blocks a barrier (GM_BP a multiple; 2 needs 260 registers: one wave a SIMD, slower)
constexpr int GM_NS = (GM_TR / 4) * 48;        // A slots a k-block
constexpr int GM_AS = GM_KC * GM_NS + 256;     // A slots a buffer (+ one spare a thread)

struct GmmArgs {
    const int8_t* D;
    const float* dso;
    int Kp, Np, N, K;
    const int8_t* Wb;
    const float* wsc;
    const float* xf;
    const int8_t* wkn;
    float* y;
};

template <int NGT>
__device__ __forceinline__ void gmm_body(const GmmArgs& A, v4i (*As)[GM_AS], const int* srcs, int e,
                                         int rows, int pbase, int cg) {
    constexpr int NIT = 48 * NGT, UA = (NIT + 255) / 256;  // A items a k-block, a thread
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nkb = A.Kp / 64;
    const int8_t* asrc[UA];
    int adst[UA];
#pragma unroll
    for (int u = 0; u < UA; ++u) {
        const int it = tid + 256 * u, kq = it & 3, rd = it >> 2, i = rd / 3, dg = rd - 3 * i;
        const bool on = it < NIT;
        asrc[u] = A.D + ((size_t)srcs[on ? min(i, rows - 1) : 0] * 3 + (on ? dg : 0)) * A.Kp + 16 * kq;
        adst[u] = on ? (i >> 2) * 48 + kq * 12 + (i & 3) * 3 + dg : -1;
    }
    const int cb0 = cg * 8 + 2 * wave, ncb = A.Np / 16;  // this wave's column blocks
    const int8_t* wb0 = A.Wb + (size_t)e * A.Np * A.Kp + (size_t)min(cb0, ncb - 1) * 1024 + lane * 16;
    const int8_t* wb1 = A.Wb + (size_t)e * A.Np * A.Kp + (size_t)min(cb0 + 1, ncb - 1) * 1024 + lane * 16;
    const size_t ks = (size_t)ncb * 1024;
    v4i ar[GM_BP][UA], bq[GM_BP][2];
    // k-blocks past the last (the loop runs whole rounds of GM_BP) multiply
    // a zero B operand
    auto ld = [&](int sl, int kb) {
        const size_t k = (size_t)min(kb, nkb - 1);
#pragma unroll
        for (int u = 0; u < UA; ++u) ar[sl][u] = *reinterpret_cast<const v4i*>(asrc[u] + k * 64);
        const v4i b0 = *reinterpret_cast<const v4i*>(wb0 + k * ks);
        const v4i b1 = *reinterpret_cast<const v4i*>(wb1 + k * ks);
        const v4i z = v4i{0, 0, 0, 0};
        bq[sl][0] = kb < nkb ? b0 : z;
        bq[sl][1] = kb < nkb ? b1 : z;
    };
    // k-block q of a buffer's GM_KC; items past the tile's go to a spare slot
    auto sta = [&](int sl, int buf, int q) {
#pragma unroll
        for (int u = 0; u < UA; ++u) As[buf][adst[u] >= 0 ? q * GM_NS + adst[u] : GM_KC * GM_NS + tid] = ar[sl][u];
    };
    v4i acc[NGT][2];
#pragma unroll
    for (int g = 0; g < NGT; ++g) acc[g][0] = acc[g][1] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int sl = 0; sl < GM_BP; ++sl) ld(sl, sl);
#pragma unroll
    for (int q = 0; q < GM_KC; ++q) sta(q, 0, q);
    const int rr = lane & 15, tl = rr >> 2, dgl = rr & 3, kql = lane >> 4;
    const int aidx = kql * 12 + tl * 3 + (dgl < 3 ? dgl : 2);
    // chunks of GM_KC k-blocks; chunk ch's A in As[ch & 1]
    for (int kb0 = 0; kb0 < nkb; kb0 += GM_BP) {
#pragma unroll
        for (int c = 0; c < GM_BP / GM_KC; ++c) {
            const int kbc = kb0 + c * GM_KC, ch = kbc / GM_KC;
            __syncthreads();  // As[ch & 1] written by every wave, As[~ch & 1] read
            const v4i* ab = As[ch & 1];
            // every A read issued before the MFMAs (one LDS latency a
            // chunk; the scheduler would pair reads with their MFMAs)
            v4i av[GM_KC][NGT];
#pragma unroll
            for (int q = 0; q < GM_KC; ++q)
#pragma unroll
                for (int g = 0; g < NGT; ++g) av[q][g] = ab[q * GM_NS + g * 48 + aidx];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < GM_KC; ++q)
#pragma unroll
                for (int g = 0; g < NGT; ++g) {
                    const int sl = c * GM_KC + q;
                    acc[g][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[q][g], bq[sl][0], acc[g][0], 0, 0, 0);
                    acc[g][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[q][g], bq[sl][1], acc[g][1], 0, 0, 0);
                }
            // the next chunk's A into the other buffer; this chunk's slots are
            // then spent (their A stored a chunk ago, their B used now): reload
            if (kbc + GM_KC < nkb) {
#pragma unroll
                for (int q = 0; q < GM_KC; ++q) sta(((c + 1) * GM_KC + q) % GM_BP, (ch + 1) & 1, q);
            }
#pragma unroll
            for (int q = 0; q < GM_KC; ++q) ld(c * GM_KC + q, kbc + q + GM_BP);
        }
    }
    // y = s * (C2 * 2^16 + C1 * 2^8 + C0) * wsc[e, j]; rows whose digits do not
    // carry them take expert_mm's own sum x . (q * s), a.dot's order
    const int col = lane & 15, tok = lane >> 4;
    const float* __restrict__ se = A.wsc + (size_t)e * A.N;
#pragma unroll
    for (int g = 0; g < NGT; ++g) {
        const int i = 4 * g + tok;
        if (i < rows) {  // predicated, not continue: acc stays statically indexed
            const int prow = pbase + i, src = srcs[i];
            const float so = A.dso[src];
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int j = (cb0 + c) * 16 + col;
                if (j < A.N) {
                    float v;
                    if (so >= 0.0f) {
                        const v4i a4 = acc[g][c];
                        v = so * ((float)a4[0] * 65536.0f + ((float)a4[1] * 256.0f + (float)a4[2])) * se[j];
                    } else {
                        const float* xr = A.xf + (size_t)src * A.K;
                        v = exact_col(xr, A.wkn + (size_t)e * A.K * A.N, A.N, j, se[j], A.K);
                    }
                    A.y[(size_t)prow * A.N + j] = v;
                }
            }
        }
    }
}

// A1 (ncg1 = 0: none) is a second linear over the same rows (up beside
// gate): column groups ncg0 .. ncg0 + ncg1 - 1 of a tile are its.
__global__ __launch_bounds__(256, 3) void moe_gmm_kernel(GmmArgs A0, GmmArgs A1, int ncg1, int gather,
                                                         const int32_t* __restrict__ ptok,
                                                      const int32_t* __restrict__ off,
                                                      const int32_t* __restrict__ cnt,
                                                      const int32_t* __restrict__ tile_e,
                                                      const int32_t* __restrict__ tile_r,
                                                      const int32_t* __restrict__ ntile) {
    __shared__ v4i As[2][GM_AS];
    __shared__ int srcs[GM_TR];
    // XCD-aware order: workgroup id goes to XCD id % 8, and XCD x runs
    // tiles x, x + 8, ... with all ncg column groups of a tile in a row, so
    // the tile's digit rows are fetched into that XCD's L2 once
    const int ncg0 = (A0.Np / 16 + 7) / 8, ncg = ncg0 + ncg1;
    const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
    const int tix = xcd + 8 * (j / ncg), cgt = j % ncg;
    const bool second = cgt >= ncg0;  // uniform
    const GmmArgs& A = second ? A1 : A0;
    const int cg = second ? cgt - ncg0 : cgt;
    if (tix >= ntile[0]) return;  // uniform
    const int e = tile_e[tix], r0 = tile_r[tix];
    const int rows = min(GM_TR, cnt[e] - r0);
    const int pbase = off[e] + r0;
    const int tid = threadIdx.x;
    if (tid < GM_TR) {
        const int prow = pbase + min(tid, rows - 1);
        srcs[tid] = gather ? ptok[prow] : prow;
    }
    __syncthreads();
    if (rows <= 16) gmm_body<4>(A, As, srcs, e, rows, pbase, cg);
    else gmm_body<8>(A, As, srcs, e, rows, pbase, cg);
}

// ---- decode (T == 1): three launches ---------------------------------------
// (the form for shapes the two-launch decode below does not take: gelu with
// mi % 16 != 0, mi > 1024, k > 16)
// K1: every workgroup (slot s of the k picks in ascending expert id, 16
// columns of gate or up) routes the token in its wave 0 and builds the
// token's digit row in LDS itself (a few KB from L2, no launch in between),
// then runs the digit GEMM of moe_mm_kernel<1,1,4> for its expert and
// columns; workgroup (0,0) publishes the sorted picks (ws.sel / ws.w) and
// the row count the act kernel reads.
__global__ __launch_bounds__(256) void moe_dec_gu_kernel(
    const float* __restrict__ x, int d, int kpd, const float* __restrict__ logits, int E, int topk,
    int norm_topk, const float* __restrict__ pes, const int8_t* __restrict__ gate_b, int gwp,
    const float* __restrict__ gate_s, int gw, const int8_t* __restrict__ gate,
    const int8_t* __restrict__ up_b, int mip, const float* __restrict__ up_s, int mi,
    const int8_t* __restrict__ up, int nbg, float* __restrict__ g, float* __restrict__ u, MoeWs ws,
    int* __restrict__ err) {
    constexpr int KS = 4;
    extern __shared__ __attribute__((aligned(16))) float dsm[];
    float* p = dsm;                                       // [E]
    int* pe = reinterpret_cast<int*>(dsm + E);            // [topk] picks, pick order
    float* pw = dsm + E + topk;
    int* se = reinterpret_cast<int*>(dsm + E + 2 * topk);  // [topk] ascending expert id
    float* sw = dsm + E + 3 * topk;
    float* red = dsm + E + 4 * topk;                       // [8]
    float* so_l = red + 8;                                 // [1]
    int* bad_l = reinterpret_cast<int*>(red + 9);
    int8_t* Dl = reinterpret_cast<int8_t*>(dsm + ((E + 4 * topk + 10 + 3) & ~3));  // [3][kpd]
    __shared__ v4i rv[KS - 1][64];

    const int slot = blockIdx.x, cbk = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (wave == 0) {
        const bool bad = route_wave(logits, E, topk, norm_topk, pes, p, pe, pw);
        for (int i = lane; i < topk; i += 64) {
            int r = 0;
            for (int j = 0; j < topk; ++j) r += pe[j] < pe[i];
            se[r] = pe[i];
            sw[r] = pw[i];
        }
        if (lane == 0) *bad_l = bad;
    }
    row_digits(x, d, kpd, Dl, so_l, red);
    __syncthreads();
    if (slot == 0 && cbk == 0) {
        if (tid < topk) { ws.sel[tid] = se[tid]; ws.w[tid] = sw[tid]; }
        if (tid == 0) {
            ws.off[E] = topk;
            if (*bad_l) atomicOr(err, 1);
        }
    }
    const bool isg = cbk < nbg;
    const int e = se[slot];
    const int8_t* __restrict__ Wb = isg ? gate_b : up_b;
    const int Np = isg ? gwp : mip, N = isg ? gw : mi, nb0 = isg ? cbk : cbk - nbg;
    const int nkb = kpd / 64, kb0 = nkb * wave / KS, kb1 = nkb * (wave + 1) / KS;
    const int rr = lane & 15, dg = rr & 3, kq = lane >> 4;
    const bool aval = rr < 3;  // token 0, digits 0..2
    const int8_t* arow = Dl + (dg < 3 ? dg : 0) * kpd + 16 * kq;
    const int8_t* wb = Wb + (size_t)e * Np * kpd + (size_t)nb0 * 1024 + lane * 16;
    const size_t kstride = (size_t)(Np / 16) * 1024;
    v4i acc = v4i{0, 0, 0, 0};
    constexpr int U = 8;
    for (int kb = kb0; kb < kb1; kb += U) {
        v4i av[U], bv[U];
#pragma unroll
        for (int q = 0; q < U; ++q) {
            const bool in = kb + q < kb1;
            av[q] = (in && aval) ? *reinterpret_cast<const v4i*>(arow + (size_t)(kb + q) * 64) : v4i{0, 0, 0, 0};
            bv[q] = in ? *reinterpret_cast<const v4i*>(wb + (size_t)(kb + q) * kstride) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int q = 0; q < U; ++q) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[q], bv[q], acc, 0, 0, 0);
    }
    if (wave > 0) rv[wave - 1][lane] = acc;
    __syncthreads();
    if (wave > 0 || lane >= 16) return;
#pragma unroll
    for (int q = 0; q < KS - 1; ++q) acc += rv[q][lane];
    // lanes 0..15: row 0 (the token), digits in acc[0..2], column lane
    const int j = nb0 * 16 + lane;
    if (j >= N) return;
    const float so = *so_l, sj = (isg ? gate_s : up_s)[(size_t)e * N + j];
    float v;
    if (so >= 0.0f) {
        v = so * ((float)acc[0] * 65536.0f + ((float)acc[1] * 256.0f + (float)acc[2])) * sj;
    } else {
        v = exact_col(x, (isg ? gate : up) + (size_t)e * d * N, N, j, sj, d);
    }
    (isg ? g : u)[(size_t)slot * N + j] = v;
}

// K3: down GEMM of all k rows and the combine, one wave per slot (ascending
// expert id) and 16 output columns per workgroup; the combine adds the
// slots' w * down in that order from +0, as combine_kernel does.
__global__ __launch_bounds__(1024) void moe_dec_down_kernel(
    const int8_t* __restrict__ hd, const float* __restrict__ hso, int kpm, const float* __restrict__ h,
    int mi, const int8_t* __restrict__ down_b, int dp, const float* __restrict__ down_s,
    const int8_t* __restrict__ down, int d, const int32_t* __restrict__ sel, const float* __restrict__ wsel,
    int topk, float* __restrict__ out) {
    __shared__ float vs[16][16];
    const int tid = threadIdx.x, lane = tid & 63;
    const int slot = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb0 = blockIdx.x;
    const int e = sel[slot];
    const int nkb = kpm / 64;
    const int rr = lane & 15, dg = rr & 3, kq = lane >> 4;
    const bool aval = rr < 3;
    const int8_t* arow = hd + ((size_t)slot * 3 + (dg < 3 ? dg : 0)) * kpm + 16 * kq;
    const int8_t* wb = down_b + (size_t)e * dp * kpm + (size_t)nb0 * 1024 + lane * 16;
    const size_t kstride = (size_t)(dp / 16) * 1024;
    v4i acc = v4i{0, 0, 0, 0};
    constexpr int U = 8;
    for (int kb = 0; kb < nkb; kb += U) {
        v4i av[U], bv[U];
#pragma unroll
        for (int q = 0; q < U; ++q) {
            const bool in = kb + q < nkb;
            av[q] = (in && aval) ? *reinterpret_cast<const v4i*>(arow + (size_t)(kb + q) * 64) : v4i{0, 0, 0, 0};
            bv[q] = in ? *reinterpret_cast<const v4i*>(wb + (size_t)(kb + q) * kstride) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int q = 0; q < U; ++q) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[q], bv[q], acc, 0, 0, 0);
    }
    const int j = nb0 * 16 + lane;
    if (lane < 16 && j < d) {
        const float so = hso[slot], sj = down_s[(size_t)e * d + j];
        float v;
        if (so >= 0.0f) {
            v = so * ((float)acc[0] * 65536.0f + ((float)acc[1] * 256.0f + (float)acc[2])) * sj;
        } else {
            v = exact_col(h + (size_t)slot * mi, down + (size_t)e * mi * d, d, j, sj, mi);
        }
        vs[slot][lane] = v;
    }
    __syncthreads();
    if (tid < 16 && nb0 * 16 + tid < d) {
        float a = 0.0f;
        for (int q = 0; q < topk; ++q) a = a + wsel[q] * vs[q][tid];
        out[nb0 * 16 + tid] = a;
    }
}

// ---- decode (T == 1): two launches ----------------------------------------
// D1: workgroup (slot s of the k picks in ascending expert id, 16 columns
// of h).  Wave 0 routes the token while waves 1..3 take max|x| of its row;
// then every wave issues its share (a quarter of K) of the expert's two
// weight blocks, gate and up (or the two halves of the packed gate_up),
// before the token's digit row is formed in LDS, so the row's second pass
// over x overlaps the weight stream.  The two digit GEMMs end in wave 0,
// whose lanes 0..15 write h = act(g) * u for their columns.  Workgroup
// (0, 0) publishes the picks in ascending expert id (ws.sel / ws.w).
// Matrix a holds g (columns 0..mi), matrix b holds u at column boff.
constexpr int DEC_U = 8;  // k-blocks per wave and load batch

__global__ __launch_bounds__(256) void moe_dec_gua_kernel(
    const float* __restrict__ x, int d, int kpd, const float* __restrict__ logits, int E, int topk,
    int norm_topk, const float* __restrict__ pes, const int8_t* __restrict__ a_b, int npa,
    const float* __restrict__ a_s, int na, const int8_t* __restrict__ a_q,
    const int8_t* __restrict__ b_b, int npb, const float* __restrict__ b_s, int nbw,
    const int8_t* __restrict__ b_q, int boff, int act, int mi, float* __restrict__ h, MoeWs ws,
    int* __restrict__ err) {
    constexpr int KS = 4;
    extern __shared__ __attribute__((aligned(16))) float dsm[];
    float* p = dsm;                                        // [E]
    int* pe = reinterpret_cast<int*>(dsm + E);             // [topk] picks, pick order
    float* pw = dsm + E + topk;
    int* se = reinterpret_cast<int*>(dsm + E + 2 * topk);  // [topk] ascending expert id
    float* sw = dsm + E + 3 * topk;
    float* red = dsm + E + 4 * topk;                       // [8]
    int* bad_l = reinterpret_cast<int*>(red + 9);
    int8_t* Dl = reinterpret_cast<int8_t*>(dsm + ((E + 4 * topk + 10 + 3) & ~3));  // [3][kpd]
    __shared__ v4i rv[KS - 1][2][64];

    const int slot = blockIdx.x, cbk = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (wave == 0) {
        const bool bad = route_wave(logits, E, topk, norm_topk, pes, p, pe, pw);
        for (int i = lane; i < topk; i += 64) {
            int r = 0;
            for (int j = 0; j < topk; ++j) r += pe[j] < pe[i];
            se[r] = pe[i];
            sw[r] = pw[i];
        }
        if (lane == 0) *bad_l = bad;
    } else {
        float mx = 0.0f;
        bool nf = false;
        for (int k = tid - 64; k < d; k += 192) {
            const float xv = x[k];
            nf |= !(fabsf(xv) <= 3.0e38f);
            mx = fmaxf(mx, fabsf(xv));
        }
        mx = wave_fmax(mx);
        const bool wnf = __builtin_amdgcn_ballot_w64(nf) != 0;
        if (lane == 0) {
            red[wave - 1] = mx;
            red[4 + wave - 1] = wnf ? 1.0f : 0.0f;
        }
    }
    __syncthreads();
    if (slot == 0 && cbk == 0) {
        if (tid < topk) { ws.sel[tid] = se[tid]; ws.w[tid] = sw[tid]; }
        if (tid == 0 && *bad_l) atomicOr(err, 1);
    }
    const int e = se[slot];
    const int nkb = kpd / 64, kb0 = nkb * wave / KS, kb1 = nkb * (wave + 1) / KS;
    const int rr = lane & 15, dg = rr & 3, kq = lane >> 4;
    const bool aval = rr < 3;  // token 0, digits 0..2
    const int8_t* wa = a_b + (size_t)e * npa * kpd + (size_t)cbk * 1024 + lane * 16;
    const int8_t* wb = b_b + (size_t)e * npb * kpd + (size_t)(boff / 16 + cbk) * 1024 + lane * 16;
    const size_t ksa = (size_t)(npa / 16) * 1024, ksb = (size_t)(npb / 16) * 1024;
    v4i ba[DEC_U], bb[DEC_U];
    auto ldw = [&](int kb) {
#pragma unroll
        for (int q = 0; q < DEC_U; ++q) {
            const bool in = kb + q < kb1;
            ba[q] = in ? *reinterpret_cast<const v4i*>(wa + (size_t)(kb + q) * ksa) : v4i{0, 0, 0, 0};
            bb[q] = in ? *reinterpret_cast<const v4i*>(wb + (size_t)(kb + q) * ksb) : v4i{0, 0, 0, 0};
        }
    };
    // this thread's x channels for the digit row first: vector loads retire
    // in issue order, so the digits then wait on these, not on the weights
    constexpr int XR = 8;  // registers: kpd <= 2048
    const bool xreg = kpd <= 256 * XR;
    float xk[XR];
#pragma unroll
    for (int i = 0; i < XR; ++i) {
        const int k = tid + 256 * i;
        xk[i] = (xreg && k < d) ? x[k] : 0.0f;
    }
    __builtin_amdgcn_sched_barrier(0);
    ldw(kb0);
    const int j = cbk * 16 + lane;
    const bool jout = wave == 0 && lane < 16 && j < mi;
    const float sa = jout ? a_s[(size_t)e * na + j] : 0.0f;
    const float sb = jout ? b_s[(size_t)e * nbw + boff + j] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);
    // the token's digit row (as row_digits), from the maxima of waves 1..3
    const float mxx = fmaxf(fmaxf(red[0], red[1]), red[2]);
    const bool xnf = (red[4] + red[5] + red[6]) != 0.0f;
    const float sx = mxx > 0.0f ? mxx / XMAXD : 1.0f;
    const bool ok = !xnf && sx >= 1.0e-30f && sx <= 1.0e28f;
    const float rx = 1.0f / sx;
    auto digit = [&](int k, float xv) {
        int d2 = 0, d1 = 0, d0 = 0;
        if (ok && k < d) {
            float xf = rintf(xv * rx);
            xf = fminf(fmaxf(xf, -XMAXD), XMAXD);
            const int X = (int)xf;
            d0 = (int)(int8_t)(X & 0xFF);
            const int X1 = (X - d0) >> 8;
            d1 = (int)(int8_t)(X1 & 0xFF);
            d2 = (X1 - d1) >> 8;
        }
        Dl[k] = (int8_t)d2;
        Dl[kpd + k] = (int8_t)d1;
        Dl[2 * kpd + k] = (int8_t)d0;
    };
    if (xreg) {
#pragma unroll
        for (int i = 0; i < XR; ++i)
            if (tid + 256 * i < kpd) digit(tid + 256 * i, xk[i]);
    } else {
        for (int k = tid; k < kpd; k += 256) digit(k, k < d ? x[k] : 0.0f);
    }
    __syncthreads();
    const int8_t* arow = Dl + (dg < 3 ? dg : 0) * kpd + 16 * kq;
    v4i acca = v4i{0, 0, 0, 0}, accb = v4i{0, 0, 0, 0};
    for (int kb = kb0; kb < kb1; kb += DEC_U) {
        v4i av[DEC_U];
#pragma unroll
        for (int q = 0; q < DEC_U; ++q)
            av[q] = (kb + q < kb1 && aval) ? *reinterpret_cast<const v4i*>(arow + (size_t)(kb + q) * 64)
                                           : v4i{0, 0, 0, 0};
#pragma unroll
        for (int q = 0; q < DEC_U; ++q) {
            acca = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[q], ba[q], acca, 0, 0, 0);
            accb = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[q], bb[q], accb, 0, 0, 0);
        }
        if (kb + DEC_U < kb1) ldw(kb + DEC_U);
    }
    if (wave > 0) {
        rv[wave - 1][0][lane] = acca;
        rv[wave - 1][1][lane] = accb;
    }
    __syncthreads();
    if (wave > 0 || lane >= 16) return;
#pragma unroll
    for (int q = 0; q < KS - 1; ++q) {
        acca += rv[q][0][lane];
        accb += rv[q][1][lane];
    }
    // lanes 0..15: the token's digit sums in acc[0..2], column lane
    if (!jout) return;
    float ga, gb;
    if (ok) {
        ga = sx * ((float)acca[0] * 65536.0f + ((float)acca[1] * 256.0f + (float)acca[2])) * sa;
        gb = sx * ((float)accb[0] * 65536.0f + ((float)accb[1] * 256.0f + (float)accb[2])) * sb;
    } else {
        ga = exact_col(x, a_q + (size_t)e * d * na, na, j, sa, d);
        gb = exact_col(x, b_q + (size_t)e * d * nbw, nbw, boff + j, sb, d);
    }
    h[(size_t)slot * mi + j] = act == FRQ_ACT_SILU ? silu(ga) * gb : gelu_tanh(ga) * gb;
}

// D2: down GEMM of all k rows and the combine; wave s takes slot s
// (ascending expert id), each workgroup 16 output columns.  Every wave
// issues its expert's first weight batch, then forms its row's digits (as
// row_digits) from h in its own LDS slab, four channels a lane and step;
// the combine adds the slots' w * down in ascending expert id from +0, as
// combine_kernel does.
constexpr int DEC_HV = 4;   // h quads a lane: kpm <= 1024
constexpr int DEC_DU = 16;  // k-blocks a load batch: all of kpm <= 1024

__global__ __launch_bounds__(1024) void moe_dec_dn_kernel(
    const float* __restrict__ h, int mi, int kpm, const int8_t* __restrict__ down_b, int dp,
    const float* __restrict__ down_s, const int8_t* __restrict__ down, int d,
    const int32_t* __restrict__ sel, const float* __restrict__ wsel, int topk,
    float* __restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) uint32_t dw[];  // [topk][3][kpm / 4]
    __shared__ float vs[16][16];
    const int tid = threadIdx.x, lane = tid & 63;
    const int slot = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb0 = blockIdx.x;
    // the row's values first (lane takes channels 4 lane + 256 i .. + 3):
    // vector loads retire in issue order, so the digits then wait on these
    // and not on the weight stream issued after them
    const float* hr = h + (size_t)slot * mi;
    float hv[DEC_HV][4];
#pragma unroll
    for (int i = 0; i < DEC_HV; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int k = 256 * i + 4 * lane + c;
            hv[i][c] = k < mi ? hr[k] : 0.0f;
        }
    __builtin_amdgcn_sched_barrier(0);
    const int e = sel[slot];
    const int nkb = kpm / 64;
    const int8_t* wb = down_b + (size_t)e * dp * kpm + (size_t)nb0 * 1024 + lane * 16;
    const size_t kstride = (size_t)(dp / 16) * 1024;
    v4i bv[DEC_DU];
    auto ldw = [&](int kb) {
#pragma unroll
        for (int q = 0; q < DEC_DU; ++q)
            bv[q] = kb + q < nkb ? *reinterpret_cast<const v4i*>(wb + (size_t)(kb + q) * kstride)
                                 : v4i{0, 0, 0, 0};
    };
    ldw(0);
    const int j = nb0 * 16 + lane;
    const bool jout = lane < 16 && j < d;
    const float sj = jout ? down_s[(size_t)e * d + j] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);
    // the row's digits
    float mx = 0.0f;
    bool nf = false;
#pragma unroll
    for (int i = 0; i < DEC_HV; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            nf |= !(fabsf(hv[i][c]) <= 3.0e38f);
            mx = fmaxf(mx, fabsf(hv[i][c]));
        }
    mx = wave_fmax(mx);
    nf = __builtin_amdgcn_ballot_w64(nf) != 0;
    const float so = mx > 0.0f ? mx / XMAXD : 1.0f;
    const bool ok = !nf && so >= 1.0e-30f && so <= 1.0e28f;
    const float r = 1.0f / so;
    uint32_t* dr = dw + (size_t)slot * 3 * (kpm / 4);
#pragma unroll
    for (int i = 0; i < DEC_HV; ++i) {
        const int k4 = 64 * i + lane;  // word of 4 channels
        if (4 * k4 >= kpm) break;
        uint32_t w2 = 0, w1 = 0, w0 = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            int d2 = 0, d1 = 0, d0 = 0;
            if (ok && 4 * k4 + c < mi) {
                float xf = rintf(hv[i][c] * r);
                xf = fminf(fmaxf(xf, -XMAXD), XMAXD);
                const int X = (int)xf;
                d0 = (int)(int8_t)(X & 0xFF);
                const int X1 = (X - d0) >> 8;
                d1 = (int)(int8_t)(X1 & 0xFF);
                d2 = (X1 - d1) >> 8;
            }
            w2 |= (uint32_t)(d2 & 0xFF) << (8 * c);
            w1 |= (uint32_t)(d1 & 0xFF) << (8 * c);
            w0 |= (uint32_t)(d0 & 0xFF) << (8 * c);
        }
        dr[k4] = w2;
        dr[kpm / 4 + k4] = w1;
        dr[2 * (kpm / 4) + k4] = w0;
    }
    wave_sync();
    const int rr = lane & 15, dg = rr & 3, kq = lane >> 4;
    const bool aval = rr < 3;
    const int8_t* arow = reinterpret_cast<const int8_t*>(dr) + (size_t)(dg < 3 ? dg : 0) * kpm + 16 * kq;
    v4i acc = v4i{0, 0, 0, 0};
    for (int kb = 0; kb < nkb; kb += DEC_DU) {
#pragma unroll
        for (int q0 = 0; q0 < DEC_DU; q0 += 4) {  // A operands four at a time (VGPR budget)
            v4i av[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                av[q] = (kb + q0 + q < nkb && aval)
                            ? *reinterpret_cast<const v4i*>(arow + (size_t)(kb + q0 + q) * 64)
                            : v4i{0, 0, 0, 0};
#pragma unroll
            for (int q = 0; q < 4; ++q)
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[q], bv[q0 + q], acc, 0, 0, 0);
        }
        if (kb + DEC_DU < nkb) ldw(kb + DEC_DU);
    }
    if (jout) {
        float v;
        if (ok) {
            v = so * ((float)acc[0] * 65536.0f + ((float)acc[1] * 256.0f + (float)acc[2])) * sj;
        } else {
            v = exact_col(hr, down + (size_t)e * mi * d, d, j, sj, mi);
        }
        vs[slot][lane] = v;
    }
    __syncthreads();
    if (tid < 16 && nb0 * 16 + tid < d) {
        float a = 0.0f;
        for (int q = 0; q < topk; ++q) a = a + wsel[q] * vs[q][tid];
        out[nb0 * 16 + tid] = a;
    }
}

// out[t, :] = sum over t's slots in ascending expert id of w * down, from
// +0.  Workgroup (column block, token): the token's k slots are ranked by
// expert id into LDS (experts within a token are distinct: top-k of a
// permutation), then every thread adds its column's k terms in that order.
constexpr int CMB_K = 256;  // slots a token

__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ dn, const int32_t* __restrict__ sel,
                                                      const float* __restrict__ w, const int32_t* __restrict__ pos,
                                                      int topk, int d, float* __restrict__ out) {
    __shared__ int srow[CMB_K];
    __shared__ float swt[CMB_K];
    const int t = blockIdx.y;
    const int32_t* st = sel + (size_t)t * topk;
    for (int i = threadIdx.x; i < topk; i += 256) {
        const int ev = st[i];
        int r = 0;
        for (int q = 0; q < topk; ++q) r += st[q] < ev;
        srow[r] = pos[(size_t)t * topk + i];
        swt[r] = w[(size_t)t * topk + i];
    }
    __syncthreads();
    if ((d & 3) == 0) {  // four columns a thread, each in the same order
        const int c4 = blockIdx.x * 256 + threadIdx.x;
        if (4 * c4 >= d) return;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int i = 0; i < topk; ++i) {
            const float4 v = reinterpret_cast<const float4*>(dn + (size_t)srow[i] * d)[c4];
            const float wi = swt[i];
            acc.x = acc.x + wi * v.x;
            acc.y = acc.y + wi * v.y;
            acc.z = acc.z + wi * v.z;
            acc.w = acc.w + wi * v.w;
        }
        reinterpret_cast<float4*>(out + (size_t)t * d)[c4] = acc;
        return;
    }
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= d) return;
    float acc = 0.0f;
    for (int i = 0; i < topk; ++i) acc = acc + swt[i] * dn[(size_t)srow[i] * d + c];
    out[(size_t)t * d + c] = acc;
}

// ---- experts stored in other dtypes (i4, q4a, f16, f32) ---------------------
// expert_f32 (src/bundle.rs:404-454) forms W[k, j] of every arm in f32 before
// x.dot(&wv): i4 s4 * scale[j, k / g], q4a scale * u4 + min (a mul then an
// add), f16 the exact upcast, f32 as stored.  The kernels below read the
// stored bytes and form the same values in registers.
struct ExpView {
    const void* raw;
    const uint16_t* sc;
    const uint16_t* mn;
    int in, out, g, ng, rb;  // rb: bytes a packed row
    size_t per, sper;        // raw elements (bytes for i4 / q4a) and scales an expert
};

ExpView exp_view(const MoeBank& b, const ExpMat& m) {
    ExpView v;
    v.raw = m.raw; v.sc = m.sc; v.mn = m.mn;
    v.in = (int)m.in; v.out = (int)m.out;
    v.g = (int)(b.g ? b.g : 1);
    v.ng = (int)((m.in + v.g - 1) / v.g);
    v.rb = (int)((m.in + 1) / 2);
    v.per = (b.dtype == FRQ_DT_I4 || b.dtype == FRQ_DT_Q4A) ? m.out * (size_t)v.rb : m.in * m.out;
    v.sper = m.out * (size_t)v.ng;
    return v;
}

template <int DT>
__device__ __forceinline__ float wval(const ExpView& v, size_t e, int k, int j) {
    if constexpr (DT == FRQ_DT_F32) {
        return reinterpret_cast<const float*>(v.raw)[e * v.per + (size_t)k * v.out + j];
    } else if constexpr (DT == FRQ_DT_F16) {
        return h2f(reinterpret_cast<const uint16_t*>(v.raw)[e * v.per + (size_t)k * v.out + j]);
    } else {
        const uint8_t byte = reinterpret_cast<const uint8_t*>(v.raw)[e * v.per + (size_t)j * v.rb + (k >> 1)];
        const int nib = (k & 1) ? (byte >> 4) : (byte & 15);
        const size_t gi = e * v.sper + (size_t)j * v.ng + k / v.g;
        if constexpr (DT == FRQ_DT_I4) return (float)((nib ^ 8) - 8) * h2f(v.sc[gi]);
        else return h2f(v.sc[gi]) * (float)nib + h2f(v.mn[gi]);
    }
}

// x . W_e[:, j] in a.dot's order (MM_KC-long k blocks, each an FMA chain
// from +0, added in order).
template <int DT>
__device__ float exact_ex(const float* __restrict__ x, const ExpView& v, size_t e, int j) {
    float c = 0.0f;
    for (int k0 = 0; k0 < v.in; k0 += MM_KC) {
        float ab = 0.0f;
        for (int k = k0; k < min(v.in, k0 + MM_KC); ++k) ab = __builtin_fmaf(x[k], wval<DT>(v, e, k, j), ab);
        c = c + ab;
    }
    return c;
}

// expert_mm of one expert: a thread per (row, output column).
template <int DT>
__global__ __launch_bounds__(256) void expert_mm_ex_kernel(const float* __restrict__ x, int m, ExpView v, int e,
                                                           float* __restrict__ y) {
    const int j = blockIdx.x * 256 + threadIdx.x, i = blockIdx.y;
    if (j >= v.out || i >= m) return;
    y[(size_t)i * v.out + j] = exact_ex<DT>(x + (size_t)i * v.in, v, (size_t)e, j);
}

// Grouped expert matmul over the tile list in expert_mm's own order, for any
// stored dtype: workgroup (tile of up to GM_TR rows of one expert, 64
// output columns); a lane per column, wave w the tile's rows w, w + 4, ...;
// the tile's x rows pass through LDS one a.dot block at a time, each weight
// value formed once for all of the wave's rows.  src = ptok[prow] when gather
// (rows of x), else prow.
constexpr int EX_RW = GM_TR / 4;  // rows a wave

template <int DT>
__global__ __launch_bounds__(256) void moe_ex_kernel(ExpView v, const float* __restrict__ x, int gather,
                                                     const int32_t* __restrict__ ptok,
                                                     const int32_t* __restrict__ off,
                                                     const int32_t* __restrict__ cnt,
                                                     const int32_t* __restrict__ tile_e,
                                                     const int32_t* __restrict__ tile_r,
                                                     const int32_t* __restrict__ ntile, float* __restrict__ y) {
    __shared__ float xs[GM_TR][MM_KC + 1];
    __shared__ int srcs[GM_TR];
    const int tix = blockIdx.x;
    if (tix >= ntile[0]) return;  // uniform
    const int e = tile_e[tix], r0 = tile_r[tix];
    const int rows = min(GM_TR, cnt[e] - r0), pbase = off[e] + r0;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < GM_TR) {
        const int prow = pbase + min(tid, rows - 1);
        srcs[tid] = gather ? ptok[prow] : prow;
    }
    const int j = blockIdx.y * 64 + lane, jc = min(j, v.out - 1);
    const int K = v.in;
    float tot[EX_RW], acc[EX_RW];
#pragma unroll
    for (int u = 0; u < EX_RW; ++u) tot[u] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += MM_KC) {
        const int kn = min(MM_KC, K - k0);
        __syncthreads();  // srcs written / the previous block's xs read
        for (int idx = tid; idx < rows * kn; idx += 256) {
            const int r = idx / kn, kk = idx - r * kn;
            xs[r][kk] = x[(size_t)srcs[r] * K + k0 + kk];
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < EX_RW; ++u) acc[u] = 0.0f;
        for (int kk = 0; kk < kn; ++kk) {
            const float w = wval<DT>(v, (size_t)e, k0 + kk, jc);
#pragma unroll
            for (int u = 0; u < EX_RW; ++u) {
                const int r = wave + 4 * u;
                if (r < rows) acc[u] = __builtin_fmaf(xs[r][kk], w, acc[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < EX_RW; ++u) tot[u] = tot[u] + acc[u];
    }
    if (j < v.out) {
#pragma unroll
        for (int u = 0; u < EX_RW; ++u) {
            const int r = wave + 4 * u;
            if (r < rows) y[(size_t)(pbase + r) * v.out + j] = tot[u];
        }
    }
}

// ---- int4 experts on the int8 MFMA ------------------------------------------
// Expert-stationary grouped digit GEMM for i4 banks with g % 32 == 0:
// workgroup (tile of up to GM_TR rows of one expert, 128 output columns), 4
// waves x two 16-column blocks.  Per group quad (128 inputs) the tile's
// digit rows (24-bit fixed point per row, as the int8 bank's) pass through
// LDS, laid out as the v_mfma_i32_16x16x32_i8 A operands in lane order:
// token group t, group gi, lane 16 q + 4 tl + d holds digit d of row
// 4 t + tl, inputs 8 q .. 8 q + 7 of the group (the d == 3 slots stay zero),
// so a wave's operand is one linear 512-byte LDS read.  B is one 16-byte
// load a lane and block (the quad's four groups of q4e), each 4-byte group
// word sign-extended into eight int8 values in input order.  A group gives
// the exact integer dots C_d of the three digits, and their combination
// G = C2 * 2^16 + C1 * 2^8 + C0 is exact in int32 (|C2| <= 32 * 127 * 8,
// |C1|, |C0| <= 32 * 128 * 8: |G| < 2^31); the f32 sum over the groups is
// acc += scale[j, g] * G and y = so * acc.  The next quad's A and B loads
// are in flight during the MFMAs.  Rows whose digits cannot carry the
// activations take expert_mm's own order over the stored nibbles.
constexpr int I4_AS = 8 * 4 * 64;  // A slots (8 bytes) of a quad: t, gi, lane

struct I4Args {
    const int8_t* D;     // digit rows [src][3][Kp]
    const float* dso;    // their scales (-1: exact row)
    int Kp, nrb, ng4, N, K;
    const uint8_t* q4e;
    const uint16_t* s4e;
    ExpView raw;
    const float* xf;     // f32 rows (exact rows)
    float* y;
};

// The eight nibbles of a q4e group word (input 8 q + b in the low, 8 q + 4 + b
// in the high half of byte b) as sign-extended int8 in input order: per byte
// with y = x ^ 8, ((y + 0x78) ^ 0x80) is x as a signed nibble, and y + 0x78
// <= 0x87 never carries into the next byte.
__device__ __forceinline__ long i4_bop(uint32_t w) {
    const uint32_t y = w ^ 0x88888888u;
    const uint32_t lo = ((y & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
    const uint32_t hi = (((y >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
    return (long)(((unsigned long long)hi << 32) | lo);
}


template <int NGT>
__device__ __forceinline__ void i4_body(const I4Args& A, uint2 (*As)[I4_AS], const int* srcs, int e, int rows,
                                        int pbase, int cg) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int cb0 = cg * 8 + 2 * wave;  // this wave's two 16-column blocks (clamped loads past the last)
    const size_t eb = (size_t)e * A.nrb;
    const uint8_t* qb0 = A.q4e + (eb + min(cb0, A.nrb - 1)) * A.ng4 * 1024 + lane * 16;
    const uint8_t* qb1 = A.q4e + (eb + min(cb0 + 1, A.nrb - 1)) * A.ng4 * 1024 + lane * 16;
    const uint16_t* sb0 = A.s4e + (eb + min(cb0, A.nrb - 1)) * A.ng4 * 64 + (lane & 15) * 4;
    const uint16_t* sb1 = A.s4e + (eb + min(cb0 + 1, A.nrb - 1)) * A.ng4 * 64 + (lane & 15) * 4;
    // A staging: item = (row, digit, 16-byte chunk of the quad), two 8-byte
    // operand pieces each (q and q + 1 of group ch / 2)
    constexpr int NIT = 24 * 4 * NGT, UA = (NIT + 255) / 256;
    const int8_t* asrc[UA];
    int adst[UA];
#pragma unroll
    for (int u = 0; u < UA; ++u) {
        const int it = min(tid + 256 * u, NIT - 1), r = it / 24, dg = (it % 24) / 8, ch = it % 8;
        asrc[u] = A.D + ((size_t)srcs[min(r, rows - 1)] * 3 + dg) * A.Kp + 16 * ch;
        adst[u] = tid + 256 * u < NIT ? ((r >> 2) * 4 + (ch >> 1)) * 64 + 32 * (ch & 1) + 4 * (r & 3) + dg : -1;
    }
    // the d == 3 slots of both buffers: zero for good
    for (int i = tid; i < 2 * NGT * 4 * 16; i += 256) As[i / (NGT * 64)][(i % (NGT * 64)) * 4 + 3] = make_uint2(0u, 0u);
    uint4 an[UA], bn0, bn1, bc0, bc1;
    uint2 sn0, sn1, sc0, sc1;
    auto ldq = [&](int q4) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < UA; ++u) an[u] = *reinterpret_cast<const uint4*>(asrc[u] + (size_t)q4 * 128);
        bn0 = *reinterpret_cast<const uint4*>(qb0 + (size_t)q4 * 1024);
        bn1 = *reinterpret_cast<const uint4*>(qb1 + (size_t)q4 * 1024);
        sn0 = *reinterpret_cast<const uint2*>(sb0 + (size_t)q4 * 64);
        sn1 = *reinterpret_cast<const uint2*>(sb1 + (size_t)q4 * 64);
    };
    auto sta = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < UA; ++u)
            if (adst[u] >= 0) {
                As[buf][adst[u]] = make_uint2(an[u].x, an[u].y);
                As[buf][adst[u] + 16] = make_uint2(an[u].z, an[u].w);
            }
    };
    float acc[NGT][2];
#pragma unroll
    for (int t = 0; t < NGT; ++t) acc[t][0] = acc[t][1] = 0.0f;
    ldq(0);
    sta(0);
    bc0 = bn0; bc1 = bn1; sc0 = sn0; sc1 = sn1;
    __syncthreads();
    for (int q4 = 0; q4 < A.ng4; ++q4) {
        const int buf = q4 & 1;
        if (q4 + 1 < A.ng4) ldq(q4 + 1);
        long b0[4], b1[4];
        float f0[4], f1[4];
        {
            const uint32_t w0[4] = {bc0.x, bc0.y, bc0.z, bc0.w}, w1[4] = {bc1.x, bc1.y, bc1.z, bc1.w};
            const uint32_t s0[2] = {sc0.x, sc0.y}, s1[2] = {sc1.x, sc1.y};
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                b0[gi] = i4_bop(w0[gi]);
                b1[gi] = i4_bop(w1[gi]);
                f0[gi] = h2f((uint16_t)(s0[gi >> 1] >> (16 * (gi & 1))));
                f1[gi] = h2f((uint16_t)(s1[gi >> 1] >> (16 * (gi & 1))));
            }
        }
#pragma unroll
        for (int t = 0; t < NGT; ++t) {
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                uint2 a = As[buf][(t * 4 + gi) * 64 + lane];
                // the operand passes an ordered (volatile) point, so this
                // token group's MFMAs cannot be hoisted above the previous
                // group's sums: every MFMA of the quad in flight at once
                // would hold 64 result registers a token group
                asm volatile("" : "+v"(a.x), "+v"(a.y));
                const long aop = (long)(((unsigned long long)a.y << 32) | a.x);
                const v4i c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, b0[gi], v4i{0, 0, 0, 0}, 0, 0, 0);
                const v4i c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, b1[gi], v4i{0, 0, 0, 0}, 0, 0, 0);
                const int g0 = c0[0] * 65536 + c0[1] * 256 + c0[2], g1 = c1[0] * 65536 + c1[1] * 256 + c1[2];
                acc[t][0] = __builtin_fmaf(f0[gi], (float)g0, acc[t][0]);
                acc[t][1] = __builtin_fmaf(f1[gi], (float)g1, acc[t][1]);
            }
            asm volatile("" : "+v"(acc[t][0]), "+v"(acc[t][1]));
        }
        if (q4 + 1 < A.ng4) {
            sta(buf ^ 1);
            bc0 = bn0; bc1 = bn1; sc0 = sn0; sc1 = sn1;
        }
        __syncthreads();
    }
    const int col = lane & 15, tok = lane >> 4;
#pragma unroll
    for (int t = 0; t < NGT; ++t) {
        const int i = 4 * t + tok;
        if (i < rows) {
            const int prow = pbase + i, src = srcs[i];
            const float so = A.dso[src];
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int j = (cb0 + c) * 16 + col;
                if (j < A.N) {
                    const float v = so >= 0.0f ? so * acc[t][c]
                                               : exact_ex<FRQ_DT_I4>(A.xf + (size_t)src * A.K, A.raw, (size_t)e, j);
                    A.y[(size_t)prow * A.N + j] = v;
                }
            }
        }
    }
}

// i4_body<1> for tiles of at most 4 rows and at most I4_SQ quads (the
// decode): every quad's A operands are staged into LDS up front (one
// barrier, 2 KB a quad: token group 0 of the As layout, quad q at 256 q),
// and the B words and scales run I4_PF quads ahead in a register ring, so
// the loop waits on no load it has just issued and has no barrier; the
// operations and their order are i4_body's, so the values are the same bits.
constexpr int I4_SQ = 2 * I4_AS / 256, I4_PF = 4;

__device__ __forceinline__ void i4_body_s(const I4Args& A, uint2* As, const int* srcs, int e, int rows, int pbase,
                                          int cg) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int cb0 = cg * 8 + 2 * wave;
    const size_t eb = (size_t)e * A.nrb;
    const uint8_t* qb0 = A.q4e + (eb + min(cb0, A.nrb - 1)) * A.ng4 * 1024 + lane * 16;
    const uint8_t* qb1 = A.q4e + (eb + min(cb0 + 1, A.nrb - 1)) * A.ng4 * 1024 + lane * 16;
    const uint16_t* sb0 = A.s4e + (eb + min(cb0, A.nrb - 1)) * A.ng4 * 64 + (lane & 15) * 4;
    const uint16_t* sb1 = A.s4e + (eb + min(cb0 + 1, A.nrb - 1)) * A.ng4 * 64 + (lane & 15) * 4;
    const int ng4 = A.ng4;
    uint4 B0[I4_PF], B1[I4_PF];
    uint2 S0[I4_PF], S1[I4_PF];
    auto ldb = [&](int p, int q4) __attribute__((always_inline)) {
        const int q = min(q4, ng4 - 1);  // clamped: the loads stay unconditional
        B0[p] = *reinterpret_cast<const uint4*>(qb0 + (size_t)q * 1024);
        B1[p] = *reinterpret_cast<const uint4*>(qb1 + (size_t)q * 1024);
        S0[p] = *reinterpret_cast<const uint2*>(sb0 + (size_t)q * 64);
        S1[p] = *reinterpret_cast<const uint2*>(sb1 + (size_t)q * 64);
    };
#pragma unroll
    for (int p = 0; p < I4_PF; ++p) ldb(p, p);
    // A of every quad: item (quad, row < 4, digit, 16-byte chunk), as i4_body
    for (int it = tid; it < 96 * ng4; it += 256) {
        const int q4 = it / 96, rem = it - 96 * q4, r = rem / 24, dg = (rem % 24) / 8, ch = rem % 8;
        const uint4 a = *reinterpret_cast<const uint4*>(A.D + ((size_t)srcs[min(r, rows - 1)] * 3 + dg) * A.Kp +
                                                         (size_t)q4 * 128 + 16 * ch);
        const int dst = q4 * 256 + (ch >> 1) * 64 + 32 * (ch & 1) + 4 * r + dg;
        As[dst] = make_uint2(a.x, a.y);
        As[dst + 16] = make_uint2(a.z, a.w);
    }
    for (int i = tid; i < 64 * ng4; i += 256) As[4 * i + 3] = make_uint2(0u, 0u);  // the d == 3 slots
    __syncthreads();
    float acc0 = 0.0f, acc1 = 0.0f;
    for (int q0 = 0; q0 < ng4; q0 += I4_PF) {
#pragma unroll
        for (int p = 0; p < I4_PF; ++p) {
            const int q4 = q0 + p;
            if (q4 >= ng4) break;  // uniform
            const uint32_t w0[4] = {B0[p].x, B0[p].y, B0[p].z, B0[p].w}, w1[4] = {B1[p].x, B1[p].y, B1[p].z, B1[p].w};
            const uint32_t s0[2] = {S0[p].x, S0[p].y}, s1[2] = {S1[p].x, S1[p].y};
            long b0[4], b1[4];
            float f0[4], f1[4];
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                b0[gi] = i4_bop(w0[gi]);
                b1[gi] = i4_bop(w1[gi]);
                f0[gi] = h2f((uint16_t)(s0[gi >> 1] >> (16 * (gi & 1))));
                f1[gi] = h2f((uint16_t)(s1[gi >> 1] >> (16 * (gi & 1))));
            }
            ldb(p, q4 + I4_PF);  // this slot's next quad
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                const uint2 a = As[q4 * 256 + gi * 64 + lane];
                const long aop = (long)(((unsigned long long)a.y << 32) | a.x);
                const v4i c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, b0[gi], v4i{0, 0, 0, 0}, 0, 0, 0);
                const v4i c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, b1[gi], v4i{0, 0, 0, 0}, 0, 0, 0);
                const int g0 = c0[0] * 65536 + c0[1] * 256 + c0[2], g1 = c1[0] * 65536 + c1[1] * 256 + c1[2];
                acc0 = __builtin_fmaf(f0[gi], (float)g0, acc0);
                acc1 = __builtin_fmaf(f1[gi], (float)g1, acc1);
            }
        }
    }
    const int col = lane & 15, i = lane >> 4;
    if (i < rows) {
        const int prow = pbase + i, src = srcs[i];
        const float so = A.dso[src];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int j = (cb0 + c) * 16 + col;
            if (j < A.N) {
                const float v = so >= 0.0f ? so * (c ? acc1 : acc0)
                                           : exact_ex<FRQ_DT_I4>(A.xf + (size_t)src * A.K, A.raw, (size_t)e, j);
                A.y[(size_t)prow * A.N + j] = v;
            }
        }
    }
}

// A1 (ncg1 = 0: none) is a second matrix over the same rows (up beside gate).
__global__ __launch_bounds__(256) void moe_i4_kernel(I4Args A0, I4Args A1, int ncg1, int gather,
                                                     const int32_t* __restrict__ ptok,
                                                     const int32_t* __restrict__ off,
                                                     const int32_t* __restrict__ cnt,
                                                     const int32_t* __restrict__ tile_e,
                                                     const int32_t* __restrict__ tile_r,
                                                     const int32_t* __restrict__ ntile) {
    __shared__ uint2 As[2][I4_AS];
    __shared__ int srcs[GM_TR];
    // XCD-aware order (as moe_gmm_kernel): a tile's column groups on one XCD
    const int ncg0 = (A0.nrb + 7) / 8, ncg = ncg0 + ncg1;
    const int xcd = blockIdx.x & 7, jb = blockIdx.x >> 3;
    const int tix = xcd + 8 * (jb / ncg), cgt = jb % ncg;
    const bool second = cgt >= ncg0;  // uniform
    const int cg = second ? cgt - ncg0 : cgt;
    if (tix >= ntile[0]) return;  // uniform
    // the tile's expert and rows, wave-uniform (scalar, so the branches on
    // them stay scalar)
    const int e = __builtin_amdgcn_readfirstlane(tile_e[tix]), r0 = __builtin_amdgcn_readfirstlane(tile_r[tix]);
    const int rows = __builtin_amdgcn_readfirstlane(min(GM_TR, cnt[e] - r0));
    const int pbase = __builtin_amdgcn_readfirstlane(off[e] + r0);
    const int tid = threadIdx.x;
    if (tid < GM_TR) {
        const int prow = pbase + min(tid, rows - 1);
        srcs[tid] = gather ? ptok[prow] : prow;
    }
    __syncthreads();
    // each argument block read in place (a reference chosen between the two
    // at run time would copy both to scratch)
    auto run = [&](const I4Args& A) __attribute__((always_inline)) {
        if (rows <= 4 && A.ng4 <= I4_SQ) i4_body_s(A, &As[0][0], srcs, e, rows, pbase, cg);
        else if (rows <= 4) i4_body<1>(A, As, srcs, e, rows, pbase, cg);
        else if (rows <= 16) i4_body<4>(A, As, srcs, e, rows, pbase, cg);
        else i4_body<8>(A, As, srcs, e, rows, pbase, cg);
    };
    if (second) run(A1);
    else run(A0);
}

// ---- int4 decode (T == 1, SiLU): two launches -------------------------------
// The batched path's values (digit rows as row_digits, i4_body's group order
// and epilogue, act_digits's h, combine_kernel's order), so the same bits,
// in two launches instead of seven.  A lane's MFMA A operand is read from a
// compact digit row in LDS (rows dr[dg][k], dg 0..2 = d2, d1, d0; token row 0
// only, the other rows of the operand zero).
__device__ __forceinline__ long i4_dec_aop(const int8_t* dr, int kp, int q4, int gi, int lane) {
    const int dg = lane & 3, tl = (lane >> 2) & 3, qq = lane >> 4;
    if (tl != 0 || dg == 3) return 0;
    const uint2 a = *reinterpret_cast<const uint2*>(dr + (size_t)dg * kp + q4 * 128 + gi * 32 + 8 * qq);
    return (long)(((unsigned long long)a.y << 32) | a.x);
}

// the three digits of v at scale reciprocal r (row_digits), zero unless ok
__device__ __forceinline__ void i4_dec_digits(float v, float r, bool ok, int8_t* dr, int kp, int k) {
    int d2 = 0, d1 = 0, d0 = 0;
    if (ok) {
        float xf = rintf(v * r);
        xf = fminf(fmaxf(xf, -XMAXD), XMAXD);
        const int X = (int)xf;
        d0 = (int)(int8_t)(X & 0xFF);
        const int X1 = (X - d0) >> 8;
        d1 = (int)(int8_t)(X1 & 0xFF);
        d2 = (X1 - d1) >> 8;
    }
    dr[k] = (int8_t)d2;
    dr[kp + k] = (int8_t)d1;
    dr[2 * kp + k] = (int8_t)d0;
}

// i4_body's quad loop for one token row over two 16-column blocks (B words
// of block b at qb[b] / scales sb[b], I4_PF quads ahead in registers):
// acc[b] += scale * G over the groups in order.
__device__ __forceinline__ void i4_dec_loop(const uint8_t* const (&qb)[2], const uint16_t* const (&sb)[2],
                                            const int8_t* dr, int kp, int ng4, int lane, float (&acc)[2]) {
    uint4 B0[I4_PF], B1[I4_PF];
    uint2 S0[I4_PF], S1[I4_PF];
    auto ldb = [&](int p, int q4) __attribute__((always_inline)) {
        const int q = min(q4, ng4 - 1);
        B0[p] = *reinterpret_cast<const uint4*>(qb[0] + (size_t)q * 1024);
        B1[p] = *reinterpret_cast<const uint4*>(qb[1] + (size_t)q * 1024);
        S0[p] = *reinterpret_cast<const uint2*>(sb[0] + (size_t)q * 64);
        S1[p] = *reinterpret_cast<const uint2*>(sb[1] + (size_t)q * 64);
    };
#pragma unroll
    for (int p = 0; p < I4_PF; ++p) ldb(p, p);
    acc[0] = acc[1] = 0.0f;
    for (int q0 = 0; q0 < ng4; q0 += I4_PF) {
#pragma unroll
        for (int p = 0; p < I4_PF; ++p) {
            const int q4 = q0 + p;
            if (q4 >= ng4) break;  // uniform
            const uint32_t w0[4] = {B0[p].x, B0[p].y, B0[p].z, B0[p].w}, w1[4] = {B1[p].x, B1[p].y, B1[p].z, B1[p].w};
            const uint32_t s0[2] = {S0[p].x, S0[p].y}, s1[2] = {S1[p].x, S1[p].y};
            long b0[4], b1[4];
            float f0[4], f1[4];
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                b0[gi] = i4_bop(w0[gi]);
                b1[gi] = i4_bop(w1[gi]);
                f0[gi] = h2f((uint16_t)(s0[gi >> 1] >> (16 * (gi & 1))));
                f1[gi] = h2f((uint16_t)(s1[gi >> 1] >> (16 * (gi & 1))));
            }
            ldb(p, q4 + I4_PF);
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                const long aop = i4_dec_aop(dr, kp, q4, gi, lane);
                const v4i c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, b0[gi], v4i{0, 0, 0, 0}, 0, 0, 0);
                const v4i c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, b1[gi], v4i{0, 0, 0, 0}, 0, 0, 0);
                const int g0 = c0[0] * 65536 + c0[1] * 256 + c0[2], g1 = c1[0] * 65536 + c1[1] * 256 + c1[2];
                acc[0] = __builtin_fmaf(f0[gi], (float)g0, acc[0]);
                acc[1] = __builtin_fmaf(f1[gi], (float)g1, acc[1]);
            }
        }
    }
}

// I1: workgroup (slot s of the k picks in ascending expert id, 4 column
// blocks of h).  Wave 0 routes the token while waves 1..3 take max|x|; every
// thread then forms digits of x into LDS, and wave w runs the quad loop over
// gate and up column block 4 by + w, then lanes 0..15 write h = silu(g) * u.
// Workgroup (0, 0) publishes the picks (ws.sel / ws.w, ascending expert id).
__global__ __launch_bounds__(256) void moe_i4_dec_gu_kernel(
    const float* __restrict__ x, const float* __restrict__ logits, int E, int topk, int norm_topk,
    const float* __restrict__ pes, I4Args G, I4Args U, int mi, float* __restrict__ h, MoeWs ws,
    int* __restrict__ err) {
    extern __shared__ __attribute__((aligned(16))) float dsm[];
    float* p = dsm;                                        // [E]
    int* pe = reinterpret_cast<int*>(dsm + E);             // [topk] picks, pick order
    float* pw = dsm + E + topk;
    int* se = reinterpret_cast<int*>(dsm + E + 2 * topk);  // [topk] ascending expert id
    float* sw = dsm + E + 3 * topk;
    float* red = dsm + E + 4 * topk;                       // [8]
    int* bad_l = reinterpret_cast<int*>(red + 9);
    int8_t* dr = reinterpret_cast<int8_t*>(dsm + ((E + 4 * topk + 10 + 3) & ~3));  // [3][kp]
    const int slot = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int d = G.K, ng4 = G.ng4, kp = 128 * ng4;
    if (wave == 0) {
        const bool bad = route_wave(logits, E, topk, norm_topk, pes, p, pe, pw);
        for (int i = lane; i < topk; i += 64) {
            int r = 0;
            for (int j = 0; j < topk; ++j) r += pe[j] < pe[i];
            se[r] = pe[i];
            sw[r] = pw[i];
        }
        if (lane == 0) *bad_l = bad;
    } else {
        float mx = 0.0f;
        bool nf = false;
        for (int k = tid - 64; k < d; k += 192) {
            const float xv = x[k];
            nf |= !(fabsf(xv) <= 3.0e38f);
            mx = fmaxf(mx, fabsf(xv));
        }
        mx = wave_fmax(mx);
        const bool wnf = __builtin_amdgcn_ballot_w64(nf) != 0;
        if (lane == 0) {
            red[wave - 1] = mx;
            red[4 + wave - 1] = wnf ? 1.0f : 0.0f;
        }
    }
    __syncthreads();
    if (slot == 0 && blockIdx.y == 0) {
        if (tid < topk) { ws.sel[tid] = se[tid]; ws.w[tid] = sw[tid]; }
        if (tid == 0 && *bad_l) atomicOr(err, 1);
    }
    const int e = se[slot];
    const int cb = blockIdx.y * 4 + wave, cbc = min(cb, G.nrb - 1);
    const size_t eb = (size_t)e * G.nrb;
    const uint8_t* const qb[2] = {G.q4e + (eb + cbc) * ng4 * 1024 + lane * 16, U.q4e + (eb + cbc) * ng4 * 1024 + lane * 16};
    const uint16_t* const sb[2] = {G.s4e + (eb + cbc) * ng4 * 64 + (lane & 15) * 4,
                                   U.s4e + (eb + cbc) * ng4 * 64 + (lane & 15) * 4};
    // the token's digit row (x_digits_kernel's values)
    const float mxx = fmaxf(fmaxf(red[0], red[1]), red[2]);
    const bool xnf = (red[4] + red[5] + red[6]) != 0.0f;
    const float sx = mxx > 0.0f ? mxx / XMAXD : 1.0f;
    const bool ok = !xnf && sx >= 1.0e-30f && sx <= 1.0e28f;
    const float rx = 1.0f / sx;
    for (int k = tid; k < kp; k += 256) i4_dec_digits(k < d ? x[k] : 0.0f, rx, ok && k < d, dr, kp, k);
    __syncthreads();
    float acc[2];
    i4_dec_loop(qb, sb, dr, kp, ng4, lane, acc);
    const int j = cb * 16 + lane;
    if (lane < 16 && j < mi) {
        const float gv = ok ? sx * acc[0] : exact_ex<FRQ_DT_I4>(x, G.raw, (size_t)e, j);
        const float uv = ok ? sx * acc[1] : exact_ex<FRQ_DT_I4>(x, U.raw, (size_t)e, j);
        h[(size_t)slot * mi + j] = silu(gv) * uv;
    }
}

// I2: the down rows of all k slots and the combine: wave s takes slot s
// (ascending expert id), a workgroup two column blocks of the output; each
// wave forms its row's digits (row_digits's values, act_digits's scale) in
// its own LDS slab, runs the quad loop over its expert's two down blocks,
// and the first 32 threads add the slots' w * down in ascending expert id
// from +0 (combine_kernel's order).
__global__ __launch_bounds__(1024) void moe_i4_dec_dn_kernel(const float* __restrict__ h, int mi, I4Args D,
                                                             const int32_t* __restrict__ sel,
                                                             const float* __restrict__ wsel, int topk,
                                                             float* __restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) int8_t dsl[];  // [topk][3][kp]
    __shared__ float vs[16][32];
    const int tid = threadIdx.x, lane = tid & 63;
    const int slot = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ng4 = D.ng4, kp = 128 * ng4, dn = D.N;
    int8_t* dr = dsl + (size_t)slot * 3 * kp;
    const int e = sel[slot];
    const int cb0 = blockIdx.x * 2;
    const size_t eb = (size_t)e * D.nrb;
    const int c0 = min(cb0, D.nrb - 1), c1 = min(cb0 + 1, D.nrb - 1);
    const uint8_t* const qb[2] = {D.q4e + (eb + c0) * ng4 * 1024 + lane * 16, D.q4e + (eb + c1) * ng4 * 1024 + lane * 16};
    const uint16_t* const sb[2] = {D.s4e + (eb + c0) * ng4 * 64 + (lane & 15) * 4,
                                   D.s4e + (eb + c1) * ng4 * 64 + (lane & 15) * 4};
    const float* hr = h + (size_t)slot * mi;
    float mx = 0.0f;
    bool nf = false;
    for (int k = lane; k < mi; k += 64) {
        const float v = hr[k];
        nf |= !(fabsf(v) <= 3.0e38f);
        mx = fmaxf(mx, fabsf(v));
    }
    mx = wave_fmax(mx);
    nf = __builtin_amdgcn_ballot_w64(nf) != 0;
    const float so = mx > 0.0f ? mx / XMAXD : 1.0f;
    const bool ok = !nf && so >= 1.0e-30f && so <= 1.0e28f;
    const float r = 1.0f / so;
    for (int k = lane; k < kp; k += 64) i4_dec_digits(k < mi ? hr[k] : 0.0f, r, ok && k < mi, dr, kp, k);
    wave_sync();
    float acc[2];
    i4_dec_loop(qb, sb, dr, kp, ng4, lane, acc);
    if (lane < 16) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int j = (cb0 + c) * 16 + lane;
            if (j < dn) vs[slot][16 * c + lane] = ok ? so * acc[c] : exact_ex<FRQ_DT_I4>(hr, D.raw, (size_t)e, j);
        }
    }
    __syncthreads();
    if (tid < 32 && cb0 * 16 + tid < dn) {
        float a = 0.0f;
        for (int q = 0; q < topk; ++q) a = a + wsel[q] * vs[q][tid];
        out[cb0 * 16 + tid] = a;
    }
}

// (E, out, ceil(in/2)) i4 rows + (E, out, ceil(in/g)) f16 scales -> q4e / s4e.
__global__ void moe_i4_block_kernel(const uint8_t* __restrict__ raw, const uint16_t* __restrict__ sc, int E,
                                    int in, int out, int g, int nrb, int ng4, uint8_t* __restrict__ q4e,
                                    uint16_t* __restrict__ s4e) {
    const int rb_ = (in + 1) / 2, ng = (in + g - 1) / g;
    const size_t total = (size_t)E * nrb * ng4 * 64;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int L = (int)(i % 64), q = L >> 4, r = L & 15;
        const size_t blk = i / 64;
        const int g4 = (int)(blk % ng4);
        const size_t er = blk / ng4;
        const int rb = (int)(er % nrb), e = (int)(er / nrb), j = 16 * rb + r;
        uint32_t words[4];
        for (int gi = 0; gi < 4; ++gi) {
            const int k0 = 32 * (4 * g4 + gi) + 8 * q;
            uint32_t wd = 0;
            for (int b = 0; b < 4; ++b) {
                uint32_t lo = 0, hi = 0;
                if (j < out && k0 + b < in) {
                    const uint8_t by = raw[((size_t)e * out + j) * rb_ + ((k0 + b) >> 1)];
                    lo = ((k0 + b) & 1) ? (by >> 4) : (by & 15);
                }
                if (j < out && k0 + 4 + b < in) {
                    const uint8_t by = raw[((size_t)e * out + j) * rb_ + ((k0 + 4 + b) >> 1)];
                    hi = ((k0 + 4 + b) & 1) ? (by >> 4) : (by & 15);
                }
                wd |= (lo | (hi << 4)) << (8 * b);
            }
            words[gi] = wd;
            if (q == 0) {
                const int kg = 32 * (4 * g4 + gi);
                s4e[(blk * 16 + r) * 4 + gi] = (j < out && kg < in) ? sc[((size_t)e * out + j) * ng + kg / g] : 0;
            }
        }
        *reinterpret_cast<uint4*>(q4e + i * 16) = make_uint4(words[0], words[1], words[2], words[3]);
    }
}

}  // namespace

size_t moe_ws_bytes(const MoeBank& b, size_t T, size_t topk) {
    const size_t P = T * topk, E = b.n_exp, nt = ntile_max(T, topk, E, moe_tile_rows(T));
    auto r = [](size_t x) { return round_up(x, 256); };
    return r(P * 4) * 4 + r(E * 4) + r((E + 1) * 4) + r(nt * 4) * 2 + r(4) + r(T * 3 * b.kpd) +
           r(T * 4) + r(P * b.gw * 4) + r(P * b.mi * 4) * 2 + r(P * 3 * b.kpm) + r(P * 4) +
           r(P * b.d * 4);
}

hipError_t launch_moe_route(const float* logits, size_t T, size_t E,
                            size_t topk, int norm_topk, const float* pes,
                            int32_t* sel, float* w, int* err, hipStream_t s) {
    const size_t lds = 4 * (E + 2 * topk) * sizeof(float);
    route_kernel<<<dim3((unsigned)((T + 3) / 4)), dim3(256), lds, s>>>(
        logits, (int)T, (int)E, (int)topk, norm_topk, pes, sel, w, err);
    return hipGetLastError();
}

// One grouped digit GEMM: a few tokens (tiles of 4 rows) split K over 4
// waves per 16-column block; batches (tiles of 32 rows) run the
// expert-stationary kernel, 128 columns a workgroup.
static hipError_t moe_mm(bool dec, unsigned nt, const int8_t* D, const float* dso, size_t kp,
                         int gather, const MoeWs& ws, const int8_t* wb, size_t np, const float* wsc,
                         size_t n, const float* xf, size_t k, const int8_t* wkn, float* y,
                         hipStream_t s) {
    if (dec) {
        moe_mm_kernel<1, 1, 4><<<dim3(nt, (unsigned)(np / 16)), dim3(256), 0, s>>>(
            D, dso, (int)kp, gather, ws.ptok, wb, (int)np, wsc, (int)n, xf, (int)k, wkn, ws.off,
            ws.cnt, ws.tile_e, ws.tile_r, ws.ntile, y);
    } else {
        const GmmArgs ga{D, dso, (int)kp, (int)np, (int)n, (int)k, wb, wsc, xf, wkn, y};
        moe_gmm_kernel<<<dim3((unsigned)(8 * ((nt + 7) / 8) * ((np / 16 + 7) / 8))), dim3(256), 0, s>>>(
            ga, ga, 0, gather, ws.ptok, ws.off, ws.cnt, ws.tile_e, ws.tile_r, ws.ntile);
    }
    return hipGetLastError();
}

// The batched gate and up GEMMs in one launch (the same digit rows).
static hipError_t moe_gmm_pair(unsigned nt, const GmmArgs& g0, const GmmArgs& g1, const MoeWs& ws, hipStream_t s) {
    const int ncg0 = (g0.Np / 16 + 7) / 8, ncg1 = (g1.Np / 16 + 7) / 8;
    moe_gmm_kernel<<<dim3((unsigned)(8 * ((nt + 7) / 8) * (ncg0 + ncg1))), dim3(256), 0, s>>>(
        g0, g1, ncg1, 1, ws.ptok, ws.off, ws.cnt, ws.tile_e, ws.tile_r, ws.ntile);
    return hipGetLastError();
}

// One grouped matmul of a non-int8 bank matrix: the int4 MFMA kernel where
// the bank has the operand copy (g % 32 == 0), else expert_mm's own order.
static hipError_t moe_ex_mm(const MoeBank& b, const ExpMat& m, unsigned nt, int gather, const int8_t* D,
                            const float* dso, size_t kp, const float* xf, const MoeWs& ws, float* y,
                            const ExpMat* m2, float* y2, hipStream_t s) {
    const ExpView v = exp_view(b, m);
    if (m.q4e) {
        const int nrb = (int)((m.out + 15) / 16), ng4 = (int)((m.in + 127) / 128);
        const I4Args a{D, dso, (int)kp, nrb, ng4, (int)m.out, (int)m.in, m.q4e, m.s4e, v, xf, y};
        I4Args a2 = a;
        int ncg1 = 0;
        if (m2) {
            a2 = I4Args{D, dso, (int)kp, (int)((m2->out + 15) / 16), ng4, (int)m2->out, (int)m2->in, m2->q4e,
                        m2->s4e, exp_view(b, *m2), xf, y2};
            ncg1 = (a2.nrb + 7) / 8;
        }
        const int ncg = (nrb + 7) / 8 + ncg1;
        moe_i4_kernel<<<dim3((unsigned)(8 * ((nt + 7) / 8) * ncg)), dim3(256), 0, s>>>(
            a, a2, ncg1, gather, ws.ptok, ws.off, ws.cnt, ws.tile_e, ws.tile_r, ws.ntile);
        return hipGetLastError();
    }
    const dim3 grid(nt, (unsigned)((m.out + 63) / 64));
    switch (b.dtype) {
        case FRQ_DT_I4:
            moe_ex_kernel<FRQ_DT_I4><<<grid, dim3(256), 0, s>>>(v, xf, gather, ws.ptok, ws.off, ws.cnt, ws.tile_e,
                                                                ws.tile_r, ws.ntile, y);
            break;
        case FRQ_DT_Q4A:
            moe_ex_kernel<FRQ_DT_Q4A><<<grid, dim3(256), 0, s>>>(v, xf, gather, ws.ptok, ws.off, ws.cnt, ws.tile_e,
                                                                 ws.tile_r, ws.ntile, y);
            break;
        case FRQ_DT_F16:
            moe_ex_kernel<FRQ_DT_F16><<<grid, dim3(256), 0, s>>>(v, xf, gather, ws.ptok, ws.off, ws.cnt, ws.tile_e,
                                                                 ws.tile_r, ws.ntile, y);
            break;
        default:
            moe_ex_kernel<FRQ_DT_F32><<<grid, dim3(256), 0, s>>>(v, xf, gather, ws.ptok, ws.off, ws.cnt, ws.tile_e,
                                                                 ws.tile_r, ws.ntile, y);
            break;
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && m2) return moe_ex_mm(b, *m2, nt, gather, D, dso, kp, xf, ws, y2, nullptr, nullptr, s);
    return e;
}

// The routed layer over a non-int8 bank: route, dispatch, (int4: the x
// digit rows), gate and up, act (and the h digit rows), down, combine.
static hipError_t launch_moe_ex(const MoeBank& b, const float* x, size_t T, const float* logits, size_t topk,
                                int norm_topk, const float* pes, float* out, void* wsp, int* err, hipStream_t s) {
    MoeWs ws = moe_view(wsp, b, T, topk);
    const int E = (int)b.n_exp, d = (int)b.d, mi = (int)b.mi, gw = (int)b.gw;
    if (T == 1 && topk <= 16 && b.act == FRQ_ACT_SILU && b.mg.q4e && b.mu.q4e && b.md.q4e) {
        // int4 decode in two launches (route + digits + gate / up + act,
        // then the down rows + combine), where the digit rows fit in LDS
        const ExpMat &mg = b.mg, &mu = b.mu, &md = b.md;
        const int ng4g = (int)((mg.in + 127) / 128), ng4d = (int)((md.in + 127) / 128);
        const size_t lds1 = (size_t)((E + 4 * (int)topk + 10 + 3) & ~3) * 4 + 3 * 128 * (size_t)ng4g;
        const size_t lds2 = topk * 3 * 128 * (size_t)ng4d;
        if (mg.out == (size_t)mi && mu.out == (size_t)mi && mg.in == (size_t)d && md.in == (size_t)mi &&
            md.out == (size_t)d && lds1 <= 65536 && lds2 <= 65536) {
            const I4Args G{nullptr, nullptr, 0, (int)((mg.out + 15) / 16), ng4g, (int)mg.out, (int)mg.in,
                           mg.q4e, mg.s4e, exp_view(b, mg), x, nullptr};
            const I4Args U{nullptr, nullptr, 0, (int)((mu.out + 15) / 16), ng4g, (int)mu.out, (int)mu.in,
                           mu.q4e, mu.s4e, exp_view(b, mu), x, nullptr};
            const I4Args Dn{nullptr, nullptr, 0, (int)((md.out + 15) / 16), ng4d, (int)md.out, (int)md.in,
                            md.q4e, md.s4e, exp_view(b, md), ws.h, nullptr};
            moe_i4_dec_gu_kernel<<<dim3((unsigned)topk, (unsigned)((G.nrb + 3) / 4)), dim3(256), lds1, s>>>(
                x, logits, E, (int)topk, norm_topk, pes, G, U, mi, ws.h, ws, err);
            if (hipError_t e1 = hipGetLastError()) return e1;
            moe_i4_dec_dn_kernel<<<dim3((unsigned)((Dn.nrb + 1) / 2)), dim3((unsigned)(64 * topk)), lds2, s>>>(
                ws.h, mi, Dn, ws.sel, ws.w, (int)topk, out);
            return hipGetLastError();
        }
    }
    const size_t tr = moe_tile_rows(T);
    hipError_t e = launch_moe_route(logits, T, b.n_exp, topk, norm_topk, pes, ws.sel, ws.w, err, s);
    if (e != hipSuccess) return e;
    const size_t nwc = (std::min(T, (size_t)TC) + 31) / 32;
    const size_t dlds = ((size_t)E * nwc * 2 + 3 * E) * sizeof(uint32_t);
    dispatch_kernel<<<dim3(1), dim3(1024), dlds, s>>>(ws.sel, (int)T, (int)topk, E, (int)tr, ws);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const unsigned nt = (unsigned)ntile_max(T, topk, b.n_exp, tr);
    const bool mf = b.mg.q4e != nullptr;
    if (mf) {
        x_digits_kernel<<<dim3((unsigned)T), dim3(256), 0, s>>>(x, d, (int)b.kpd, ws.xd, ws.xso);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    const bool silu_ = b.act == FRQ_ACT_SILU;
    if ((e = moe_ex_mm(b, b.mg, nt, 1, ws.xd, ws.xso, b.kpd, x, ws, ws.g, silu_ ? &b.mu : nullptr, ws.u, s)) !=
        hipSuccess)
        return e;
    act_digits_kernel<<<dim3((unsigned)(T * topk)), dim3(256), 0, s>>>(
        ws.g, ws.u, b.act, mi, gw, (int)b.kpm, ws.off, E, ws.h, ws.hd, ws.hso);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = moe_ex_mm(b, b.md, nt, 0, ws.hd, ws.hso, b.kpm, ws.h, ws, ws.dn, nullptr, nullptr, s)) != hipSuccess)
        return e;
    combine_kernel<<<dim3((unsigned)(((d % 4 ? d : d / 4) + 255) / 256), (unsigned)T), dim3(256), 0, s>>>(
        ws.dn, ws.sel, ws.w, ws.pos, (int)topk, d, out);
    return hipGetLastError();
}

hipError_t launch_expert_mm_ex(const MoeBank& b, const ExpMat& mt, size_t e, const float* x, size_t m, float* y,
                               hipStream_t st) {
    if (m == 0) return hipSuccess;
    const ExpView v = exp_view(b, mt);
    const dim3 grid((unsigned)((mt.out + 255) / 256), (unsigned)m);
    switch (b.dtype) {
        case FRQ_DT_I4: expert_mm_ex_kernel<FRQ_DT_I4><<<grid, dim3(256), 0, st>>>(x, (int)m, v, (int)e, y); break;
        case FRQ_DT_Q4A: expert_mm_ex_kernel<FRQ_DT_Q4A><<<grid, dim3(256), 0, st>>>(x, (int)m, v, (int)e, y); break;
        case FRQ_DT_F16: expert_mm_ex_kernel<FRQ_DT_F16><<<grid, dim3(256), 0, st>>>(x, (int)m, v, (int)e, y); break;
        case FRQ_DT_F32: expert_mm_ex_kernel<FRQ_DT_F32><<<grid, dim3(256), 0, st>>>(x, (int)m, v, (int)e, y); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_moe_i4_block(ExpMat& mt, size_t E, size_t g, hipStream_t st) {
    const size_t nrb = (mt.out + 15) / 16, ng4 = (mt.in + 127) / 128;
    moe_i4_block_kernel<<<dim3(2048), dim3(256), 0, st>>>((const uint8_t*)mt.raw, mt.sc, (int)E, (int)mt.in,
                                                          (int)mt.out, (int)g, (int)nrb, (int)ng4, mt.q4e, mt.s4e);
    return hipGetLastError();
}

hipError_t launch_moe(const MoeBank& b, const float* x, size_t T,
                      const float* logits, size_t topk, int norm_topk,
                      const float* pes, float* out, void* wsp, int* err,
                      hipStream_t s) {
    if (T == 0) return hipSuccess;
    if (b.dtype != FRQ_DT_I8) return launch_moe_ex(b, x, T, logits, topk, norm_topk, pes, out, wsp, err, s);
    MoeWs ws = moe_view(wsp, b, T, topk);
    const int E = (int)b.n_exp, d = (int)b.d, mi = (int)b.mi, gw = (int)b.gw;
    const size_t tr = moe_tile_rows(T);
    const bool dec = tr == 4;
    const size_t gwp = round_up(b.gw, 16), mip = round_up(b.mi, 16), dp = round_up(b.d, 16);
    const bool gelu_split = b.act != FRQ_ACT_SILU && b.mi % 16 == 0;  // u at a block edge
    if (T == 1 && topk <= 16 && (b.act == FRQ_ACT_SILU || gelu_split) && b.kpm <= 256 * DEC_HV &&
        topk * 3 * b.kpm <= 65536) {
        // decode in two launches: route + digits + gate/up + act, then the
        // down digits + down GEMM + combine
        const bool silu_ = b.act == FRQ_ACT_SILU;
        const size_t nbh = (b.mi + 15) / 16;
        const size_t lds1 = ((size_t)((E + 4 * (int)topk + 10 + 3) & ~3)) * 4 + 3 * b.kpd;
        moe_dec_gua_kernel<<<dim3((unsigned)topk, (unsigned)nbh), dim3(256), lds1, s>>>(
            x, d, (int)b.kpd, logits, E, (int)topk, norm_topk, pes, b.gate_b, (int)gwp, b.gate_s, gw,
            b.gate, silu_ ? b.up_b : b.gate_b, (int)(silu_ ? mip : gwp), silu_ ? b.up_s : b.gate_s,
            silu_ ? mi : gw, silu_ ? b.up : b.gate, silu_ ? 0 : mi, b.act, mi, ws.h, ws, err);
        hipError_t e1 = hipGetLastError();
        if (e1 != hipSuccess) return e1;
        moe_dec_dn_kernel<<<dim3((unsigned)(dp / 16)), dim3((unsigned)(64 * topk)), topk * 3 * b.kpm, s>>>(
            ws.h, mi, (int)b.kpm, b.down_b, (int)dp, b.down_s, b.down, d, ws.sel, ws.w, (int)topk, out);
        return hipGetLastError();
    }
    if (T == 1 && topk <= 16) {
        // decode, three launches: route + digits + gate/up, act digits, down + combine
        const int nbg = (int)(gwp / 16), nbu = b.act == FRQ_ACT_SILU ? (int)(mip / 16) : 0;
        const size_t lds1 = ((size_t)((E + 4 * (int)topk + 10 + 3) & ~3)) * 4 + 3 * b.kpd;
        moe_dec_gu_kernel<<<dim3((unsigned)topk, (unsigned)(nbg + nbu)), dim3(256), lds1, s>>>(
            x, d, (int)b.kpd, logits, E, (int)topk, norm_topk, pes, b.gate_b, (int)gwp, b.gate_s, gw,
            b.gate, b.up_b, (int)mip, b.up_s, mi, b.up, nbg, ws.g, ws.u, ws, err);
        hipError_t e1 = hipGetLastError();
        if (e1 != hipSuccess) return e1;
        act_digits_kernel<<<dim3((unsigned)topk), dim3(256), 0, s>>>(
            ws.g, ws.u, b.act, mi, gw, (int)b.kpm, ws.off, E, ws.h, ws.hd, ws.hso);
        if ((e1 = hipGetLastError()) != hipSuccess) return e1;
        moe_dec_down_kernel<<<dim3((unsigned)(dp / 16)), dim3((unsigned)(64 * topk)), 0, s>>>(
            ws.hd, ws.hso, (int)b.kpm, ws.h, mi, b.down_b, (int)dp, b.down_s, b.down, d, ws.sel, ws.w,
            (int)topk, out);
        return hipGetLastError();
    }
    hipError_t e = launch_moe_route(logits, T, b.n_exp, topk, norm_topk, pes, ws.sel, ws.w, err, s);
    if (e != hipSuccess) return e;
    const size_t nwc = (std::min(T, (size_t)TC) + 31) / 32;
    const size_t dlds = ((size_t)E * nwc * 2 + 3 * E) * sizeof(uint32_t);
    dispatch_kernel<<<dim3(1), dim3(1024), dlds, s>>>(ws.sel, (int)T, (int)topk, E, (int)tr, ws);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    x_digits_kernel<<<dim3((unsigned)T), dim3(256), 0, s>>>(x, d, (int)b.kpd, ws.xd, ws.xso);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const unsigned nt = (unsigned)ntile_max(T, topk, b.n_exp, tr);
    if (!dec && b.act == FRQ_ACT_SILU) {
        const GmmArgs gg{ws.xd, ws.xso, (int)b.kpd, (int)gwp, (int)b.gw, (int)b.d, b.gate_b, b.gate_s, x, b.gate, ws.g};
        const GmmArgs gu{ws.xd, ws.xso, (int)b.kpd, (int)mip, (int)b.mi, (int)b.d, b.up_b, b.up_s, x, b.up, ws.u};
        if ((e = moe_gmm_pair(nt, gg, gu, ws, s)) != hipSuccess) return e;
    } else {
        if ((e = moe_mm(dec, nt, ws.xd, ws.xso, b.kpd, 1, ws, b.gate_b, gwp, b.gate_s, b.gw, x, b.d,
                        b.gate, ws.g, s)) != hipSuccess)
            return e;
        if (b.act == FRQ_ACT_SILU &&
            (e = moe_mm(dec, nt, ws.xd, ws.xso, b.kpd, 1, ws, b.up_b, mip, b.up_s, b.mi, x, b.d, b.up,
                        ws.u, s)) != hipSuccess)
            return e;
    }
    act_digits_kernel<<<dim3((unsigned)(T * topk)), dim3(256), 0, s>>>(
        ws.g, ws.u, b.act, mi, gw, (int)b.kpm, ws.off, E, ws.h, ws.hd, ws.hso);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = moe_mm(dec, nt, ws.hd, ws.hso, b.kpm, 0, ws, b.down_b, dp, b.down_s, b.d, ws.h, b.mi,
                    b.down, ws.dn, s)) != hipSuccess)
        return e;
    combine_kernel<<<dim3((unsigned)(((d % 4 ? d : d / 4) + 255) / 256), (unsigned)T), dim3(256), 0, s>>>(
        ws.dn, ws.sel, ws.w, ws.pos, (int)topk, d, out);
    return hipGetLastError();
}

// (K, N) (in, out) int8 expert weights -> blocked (Np, Kp) per expert
// (zero padding), the MFMA B-operand layout of the digit GEMM.
__global__ void moe_block_kernel(const int8_t* __restrict__ src, int E, int K, int N, int Kp,
                                 int Np, int8_t* __restrict__ dst) {
    const size_t per = (size_t)Np * Kp, total = (size_t)E * per;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t e = i / per, rem = i % per;
        const int n = (int)(rem / Kp), k = (int)(rem % Kp);
        const int8_t v = (n < N && k < K) ? src[e * (size_t)K * N + (size_t)k * N + n] : (int8_t)0;
        dst[e * per + blk_off((size_t)n, (size_t)k, (size_t)Np)] = v;
    }
}

hipError_t launch_moe_block(const int8_t* src, size_t E, size_t K, size_t N, size_t kp,
                            size_t np, int8_t* dst, hipStream_t s) {
    moe_block_kernel<<<dim3(2048), dim3(256), 0, s>>>(src, (int)E, (int)K, (int)N, (int)kp,
                                                      (int)np, dst);
    return hipGetLastError();
}

// expert_mm for one expert: a single tile list built on the host.
__global__ void expert_mm_kernel(const float* __restrict__ x, int m, const int8_t* __restrict__ q,
                                 const float* __restrict__ s, int K, int N, float* __restrict__ y) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    const int i = blockIdx.y;
    if (j >= N || i >= m) return;
    y[(size_t)i * N + j] = exact_col(x + (size_t)i * K, q, N, j, s[j], K);
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
