// frq_internal.h — shared definitions of the gfx950 kernel library.
//
// Device layouts (all in HBM, uploaded once):
//   int8 weight  wt   (Np, Kp) i8 row-major, K contiguous; Kp = K rounded up
//                     to 128 and Np = N rounded up to 256, padding zero.
//                wkn  (Kp, Np) i8 row-major: the bundle's (in, out) layout,
//                     read by the GEMM's outlier correction.
//                scale (Np) f32.
//   int4 weight  q4   (g == 32, K % 32 == 0) the MFMA layout: for 16-row
//                     block rb, group quad g4 and lane l = 16q + r, the 4
//                     bytes (k = 8q..8q+7) of row 16rb + r in each of the 4
//                     groups, 16 bytes at ((rb*ng4 + g4)*64 + l)*16; s4 the
//                     f16 scales (rb, g4, r, 4 groups).
//                q4raw/s4raw the bundle's (N, ceil(K/2)) rows and (N, ng)
//                     f16 scales (generic shapes and the exact fallback).
//                wblk (Np, Kp) i8 in the blocked MFMA-operand layout
//                     (blk_off below), read by the GEMM's main loop.
//   activations  a8   (Mp, Kp) i8 per call (workspace): row-major for the
//                     GEMV, blocked (blk_off, R = Mp) for the GEMM; sa (M)
//                     f32, oidx/oval (M, 32) u32/f32, outliers in ascending
//                     channel.
#pragma once

#include <algorithm>
#include <string>

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/frq.h"

#define FRQ_T 32            // OUTLIER_T (src/bundle.rs:309)
#define FRQ_KALIGN 128      // Kp alignment (a multiple of the GEMM k-step)
#define FRQ_NALIGN 256      // Np alignment (a multiple of every N tile)
#define FRQ_MALIGN 128      // Mp alignment of the a8 workspace (GEMM M tile)

namespace frq {

inline size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// IEEE binary16 -> binary32 on the host (exact; the arr1o upcast).
inline float h2f_host(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, ex = (h >> 10) & 0x1F, m = h & 0x3FF;
    uint32_t u;
    if (ex == 0) {
        if (!m) {
            u = s;
        } else {  // subnormal: m * 2^-24, exact in f32
            const float f = (float)m * 5.9604644775390625e-08f;
            u = __builtin_bit_cast(uint32_t, f) | s;
        }
    } else if (ex == 31) {
        u = s | 0x7F800000u | (m << 13);
    } else {
        u = s | ((ex + 112) << 23) | (m << 13);
    }
    return __builtin_bit_cast(float, u);
}

// Blocked MFMA-operand layout of an (R, Kp) int8 matrix (R % 16 == 0,
// Kp % 64 == 0): the v_mfma_i32_16x16x64_i8 operand of rows 16rb..16rb+15
// and k-bytes 64kb..64kb+63 is one contiguous 1 KB block in lane order
// (lane 16g + r holds row r, k-bytes 16g..16g+15), blocks k-block major.
__host__ __device__ inline size_t blk_off(size_t i, size_t k, size_t R) {
    return ((k >> 6) * (R >> 4) + (i >> 4)) * 1024 + ((((k & 63) >> 4) << 4) + (i & 15)) * 16 +
           (k & 15);
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

// 128-bit streaming (non-temporal) load of a weight chunk.
__device__ __forceinline__ int4 ntload16(const void* p) {
    const v4i v = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
    return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ v4i ntload_v4i(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
}
__device__ __forceinline__ uint4 ntload16u(const void* p) {
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Lane exchange v[lane ^ J] in VALU instructions only (no LDS crossbar):
// J = 1, 2 via DPP quad_perm; J = 4, 8 via DPP row_shl / row_shr (lane i
// reads i+J / i-J within a 16-lane row) selected by lane bit; J = 16, 32 via
// gfx950 v_permlane16_swap / v_permlane32_swap.
template <int J>
__device__ __forceinline__ uint32_t xshfl(uint32_t v) {
    const int lane = threadIdx.x & 63;
    if constexpr (J == 1) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
    } else if constexpr (J == 2) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
    } else if constexpr (J == 4 || J == 8) {
        const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x100 + J, 0xF, 0xF, false);
        const uint32_t dn = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x110 + J, 0xF, 0xF, false);
        return (lane & J) ? dn : up;
    } else if constexpr (J == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane & 16) ? p[0] : p[1];
    } else {
        static_assert(J == 32, "xor distance");
        const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane & 32) ? p[0] : p[1];
    }
}

template <int J>
__device__ __forceinline__ unsigned long long xshfl64(unsigned long long v) {
    const uint32_t lo = xshfl<J>((uint32_t)v), hi = xshfl<J>((uint32_t)(v >> 32));
    return ((unsigned long long)hi << 32) | lo;
}

// Orders a wave's LDS accesses before and after (no other wave waits).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// IEEE binary16 -> binary32 (exact).
__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// The summation order of one element of the reference's a.dot (ndarray
// 0.16.1 -> matrixmultiply 0.3.10 sgemm, Cargo.lock:1108, 1207): k is split
// into blocks of MM_KC = 256 (S_KC) in order; in each block the FMA
// micro-kernel chains the products from +0, k ascending; the first block's
// result is stored, each later one added (C = C + AB).  An FMA chain from +0
// never ends at -0, so C = +0 + AB_0 is AB_0 and one running sum from +0
// covers both steps.
constexpr int MM_KC = 256;

// That order over the indices [j0, n) of a product whose terms outside are
// exact zeros (masked keys with p = 0, padding): the block edges stay at
// multiples of MM_KC from 0, and chain(s, e) returns the FMA chain from +0
// over [s, e) (within one block).
template <typename F>
__device__ __forceinline__ float mm_blocks(int j0, int n, F chain) {
    float c = 0.0f;
    for (int s = j0; s < n;) {
        const int e = min(n, (s / MM_KC + 1) * MM_KC);
        c = c + chain(s, e);
        s = e;
    }
    return c;
}

// acc + p[0] + p[1] + ... + p[n-1] in index order, in the calling lane,
// over LDS (p 16-byte aligned): loads run one 32-value batch ahead of the
// adds (unconditional, the index clamped to the last batch) so the chain
// waits on the adds, not on LDS latency.
__device__ __forceinline__ float lds_seq_sum(const float* p, int n, float acc) {
    constexpr int B = 8;  // float4 per batch
    const int nb = n / (4 * B);
    const float4* p4 = reinterpret_cast<const float4*>(p);
    float4 b0[B], b1[B];
    auto ld = [&](float4 (&b)[B], int k) {
#pragma unroll
        for (int u = 0; u < B; ++u) b[u] = p4[k * B + u];
    };
    auto add = [&](const float4 (&b)[B]) {
#pragma unroll
        for (int u = 0; u < B; ++u) {
            acc = acc + b[u].x;
            acc = acc + b[u].y;
            acc = acc + b[u].z;
            acc = acc + b[u].w;
        }
    };
    // two batches a trip, both consumed unconditionally, the odd last batch
    // after the loop; the scheduling barriers keep each batch's loads where
    // they are issued, a batch ahead of their adds (the scheduler would
    // otherwise sink them down to the use)
    if (nb > 0) {
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
    for (int i = nb * 4 * B; i < n; ++i) acc = acc + p[i];
    return acc;
}

// lds_seq_sum with two chains in the calling lane: a0 and a1 each get
// p[0] + ... + p[n-1] added in index order (one LDS load feeds both).
__device__ __forceinline__ void lds_seq_sum2(const float* p, int n, float& a0, float& a1) {
    constexpr int B = 8;
    const int nb = n / (4 * B);
    const float4* p4 = reinterpret_cast<const float4*>(p);
    float4 b0[B], b1[B];
    auto ld = [&](float4 (&b)[B], int k) {
#pragma unroll
        for (int u = 0; u < B; ++u) b[u] = p4[k * B + u];
    };
    auto add = [&](const float4 (&b)[B]) {
#pragma unroll
        for (int u = 0; u < B; ++u) {
            a0 = a0 + b[u].x; a1 = a1 + b[u].x;
            a0 = a0 + b[u].y; a1 = a1 + b[u].y;
            a0 = a0 + b[u].z; a1 = a1 + b[u].z;
            a0 = a0 + b[u].w; a1 = a1 + b[u].w;
        }
    };
    if (nb > 0) {
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
    for (int i = nb * 4 * B; i < n; ++i) {
        a0 = a0 + p[i];
        a1 = a1 + p[i];
    }
}

// Direct-to-LDS load (global_load_lds, 16 bytes a lane): lane l's 16 bytes
// at g land at lds_base + 16 l (lds_base wave-uniform).  Counted by vmcnt;
// the data is in LDS once the count has dropped past the load.
typedef __attribute__((address_space(1))) void frq_gvoid_t;
typedef __attribute__((address_space(3))) void frq_lvoid_t;
__device__ __forceinline__ void dma16_lds(const void* g, void* lds_base) {
    __builtin_amdgcn_global_load_lds((frq_gvoid_t*)g, (frq_lvoid_t*)lds_base, 16, 0, 0);
}
// s_waitcnt vmcnt(N) (gfx9 encoding; expcnt / lgkmcnt not waited on)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// LDS floats of seq_sum_spec<NT>'s scratch.
constexpr int seq_sum_spec_scratch(int nt) { return 2 * ((nt / 64) * 128) + 6 * (nt / 64) + 4; }

// init + p[0] + p[1] + ... + p[n-1], the sequential f32 fold in index order
// (p in LDS, 16-byte aligned), bit-identical to lds_seq_sum, by all NT
// threads of the workgroup (every thread calls it and gets the result).
// The row is cut into S = 2 NT / 64 contiguous segments of a multiple of 32
// elements, one a half-wave.  Segment 0 is folded from init.  Segment k > 0
// is folded from 64 start values at once, two chains in each of the
// half-wave's 32 lanes: the f32 values within 32 steps (one unit in the
// last place each) either side of its estimate f32(init + the sum of the
// earlier segments), each segment summed in f32 by its half-wave and the
// sums added in double.  The true start of segment k is the fold's value at
// its first index, which differs from the estimate only by the accumulated
// rounding (a few dozen units in the last place at most on activation rows,
// typically fewer).  Wave 0 then resolves the chain: lane j computes, for
// every segment k, which candidate of segment k the end of segment k-1's
// candidate j selects (its index, or none), so that following the true
// candidates from segment 0 is one lane read a segment; where the true
// start is not among the candidates (rows whose rounding drifts further,
// constant rows, non-finite values) the remaining segments are folded again
// from the true value.  The result never depends on the estimates, only the
// time does.  NF < NT: only the first NF threads fold (S = 2 NF / 64), the
// others take part in the barriers only (the candidate chains are VALU
// work, 64 adds an element whatever S is, while the barriers and the
// resolve grow with S).
template <int NT, int NF = NT>
__device__ __forceinline__ float seq_sum_spec(const float* p, int n, float init, float* sc) {
    constexpr int S = 2 * (NF / 64), C = 64;
    static_assert(S <= 64, "a lane of wave 0 a segment");
    static_assert(NF <= NT && NF % 64 == 0, "whole waves of the workgroup");
    const int tid = threadIdx.x, lane = tid & 63, hl = lane & 31;
    const int k = 2 * (tid >> 6) + (lane >> 5);  // this half-wave's segment
    float* ends = sc;                                      // [S][C] candidate ends
    float* psum = sc + S * C;                              // [S] segment sums (estimates)
    uint32_t* est = reinterpret_cast<uint32_t*>(psum + S);  // [S] start estimates (f32 bits)
    float* res = psum + 2 * S;                             // [1] the result
    if (n < 256) {  // short: the plain chain
        if (tid == 0) res[0] = lds_seq_sum(p, n, init);
        __syncthreads();
        const float r = res[0];
        __syncthreads();
        return r;
    }
    const int L = ((n + S - 1) / S + 31) & ~31;  // segment length, whole 32-element batches
    const int lo = min(n, k * L), hi = min(n, lo + L);
    // the segment's sum by its half-wave (an estimate: any order will do)
    float ps = 0.0f;
    for (int i = lo + hl; i < hi; i += 32) ps += p[i];
    ps += __builtin_bit_cast(float, xshfl<16>(__builtin_bit_cast(uint32_t, ps)));
    ps += __builtin_bit_cast(float, xshfl<8>(__builtin_bit_cast(uint32_t, ps)));
    ps += __builtin_bit_cast(float, xshfl<4>(__builtin_bit_cast(uint32_t, ps)));
    ps += __builtin_bit_cast(float, xshfl<2>(__builtin_bit_cast(uint32_t, ps)));
    ps += __builtin_bit_cast(float, xshfl<1>(__builtin_bit_cast(uint32_t, ps)));
    if (hl == 0 && k < S) psum[k] = ps;
    __syncthreads();
    float pv[S];  // every segment's sum, read at once
#pragma unroll
    for (int kk = 0; kk < S; ++kk) pv[kk] = psum[kk];
    double pre = (double)init;
#pragma unroll
    for (int kk = 0; kk < S; ++kk)
        if (kk < k) pre += (double)pv[kk];
    const uint32_t eb = __float_as_uint((float)pre);
    const uint32_t ebn = __float_as_uint((float)(pre + (double)pv[k < S - 1 ? k : 0]));  // segment k+1's
    if (hl == 0 && k < S) est[k] = eb;
    float c0 = k == 0 ? init : __uint_as_float(eb + (uint32_t)hl - (uint32_t)(C / 2));
    float c1 = k == 0 ? init : __uint_as_float(eb + (uint32_t)hl);
    if (lo < hi) lds_seq_sum2(p + lo, hi - lo, c0, c1);
    if (k < S) {
        ends[k * C + hl] = c0;  // candidate start eb + hl - C/2
        ends[k * C + hl + C / 2] = c1;
    }
    // the candidate of segment k+1 that each of these ends selects (or -1)
    int* nxs = reinterpret_cast<int*>(ends + S * C) + 3 * S + 1;  // [S][C]
    auto sel = [&](float e) {
        const int64_t d = (int64_t)__float_as_uint(e) - (int64_t)ebn + C / 2;
        return d >= 0 && d < C ? (int)d : -1;
    };
    if (k + 1 < S) {
        nxs[(k + 1) * C + hl] = sel(c0);
        nxs[(k + 1) * C + hl + C / 2] = sel(c1);
    }
    __syncthreads();
    if (tid < 64) {
        // wave 0: lane j holds candidate j's end of every segment, and
        // nx[kk] = the candidate of segment kk that candidate j of segment
        // kk - 1 selects (or -1)
        float e[S];
        int nx[S];
#pragma unroll
        for (int kk = 0; kk < S; ++kk) e[kk] = ends[kk * C + lane];
#pragma unroll
        for (int kk = 1; kk < S; ++kk) nx[kk] = nxs[kk * C + lane];
        // follow the true candidates: segment 0's is any (all start at init)
        int d = 0, kk = 1;
#pragma unroll
        for (int j = 1; j < S; ++j) {
            if (kk == j) {
                const int dn = __builtin_amdgcn_readlane(nx[j], d);
                if (dn >= 0) {
                    d = dn;
                    ++kk;
                }
            }
        }
        float s = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e[kk - 1]), d));
        // from the first segment whose start was missed: folded again, or
        // its candidate where the refolded start is one
        for (; kk < S; ++kk) {
            const int64_t dd = (int64_t)__float_as_uint(s) - (int64_t)est[kk] + C / 2;
            const int lo2 = min(n, kk * L), hi2 = min(n, lo2 + L);
            if (dd >= 0 && dd < C) {
                const float ek = ends[kk * C + (int)dd];
                s = ek;
            } else if (lo2 < hi2) {
                s = lds_seq_sum(p + lo2, hi2 - lo2, s);
            }
        }
        if (tid == 0) res[0] = s;
    }
    __syncthreads();
    const float r = res[0];
    __syncthreads();  // the scratch may be reused by the caller
    return r;
}

// ---- weights -------------------------------------------------------------
struct Weight {
    int dtype = 0;           // FRQ_DT_*
    int device = 0;
    size_t n = 0, k = 0, g = 0;
    size_t np = 0, kp = 0;   // padded dims (int8)
    int8_t* wt = nullptr;    // int8 (Np, Kp)
    int8_t* wkn = nullptr;   // int8 (Kp, Np): the bundle's (in, out) layout
    int8_t* wblk = nullptr;  // int8 (Np, Kp) blocked (blk_off): the GEMM operand
    float* scale = nullptr;  // int8 scale (Np)
    uint8_t* q4 = nullptr;   // int4 MFMA layout, when i4_blocked
    uint16_t* s4 = nullptr;  // int4 f16 scales, MFMA layout
    uint8_t* q4raw = nullptr;   // int4 packed (N, ceil(K/2)) as stored
    uint16_t* s4raw = nullptr;  // int4 f16 scales (N, ceil(K/g)) as stored
    int i4_blocked = 0;      // 1 when the MFMA layout (g == 32) is built
    uint8_t* rowp = nullptr; // row tables: (n, k) rows, each padded to rpitch bytes
    size_t rpitch = 0;       //   (a multiple of 128); rowi8 scales in `scale`;
                             //   q4a: the q4raw row pitch (a multiple of 16)
    uint32_t* q4a_sm = nullptr;  // q4a: (N, ng) words, f16 scale | f16 min << 16
};

// One matrix (gate / gate_up, up or down) of every expert of a bank whose
// experts are not int8, as the bundle stores it (src/bundle.rs:404-454,
// src/convert.rs:174-260): f16 / f32 (E, in, out) row-major; i4 / q4a
// (E, out, ceil(in/2)) packed nibbles, even input index low, with f16 scales
// (and q4a mins) (E, out, ceil(in/g)).  An i4 matrix with g % 32 == 0 also
// has the MFMA operand copy q4e / s4e: per expert, 16-row block rb and group
// quad g4 (four 32-input groups) one 1 KB block, lane 16 q + r holding row
// 16 rb + r's nibbles of inputs 8 q .. 8 q + 7 of each of the four groups,
// four bytes a group with input 8 q + b in the low and 8 q + 4 + b in the
// high half of byte b (so a shift and a mask give 16 x the sign-extended
// values in input order); s4e the rows' f16 scales (rb, g4, r, 4), one per
// 32-input group (zero past in).
struct ExpMat {
    void* raw = nullptr;
    uint16_t* sc = nullptr;
    uint16_t* mn = nullptr;
    uint8_t* q4e = nullptr;
    uint16_t* s4e = nullptr;
    size_t in = 0, out = 0;
};

struct MoeBank {
    int device = 0;
    size_t n_exp = 0, d = 0, mi = 0;
    int act = 0;
    int dtype = FRQ_DT_I8;       // the experts' stored dtype
    size_t g = 0;                // i4 / q4a group
    ExpMat mg, mu, md;           // non-int8 banks: gate (or gate_up), up, down
    size_t gw = 0;               // gate width: mi (SiLU) or 2*mi (gate_up)
    int8_t* gate = nullptr;      // (E, d, gw) i8 (in,out) row-major per expert
    float* gate_s = nullptr;     // (E, gw)
    int8_t* up = nullptr;        // (E, d, mi)
    float* up_s = nullptr;       // (E, mi)
    int8_t* down = nullptr;      // (E, mi, d)
    float* down_s = nullptr;     // (E, d)
    // blocked MFMA-operand copies (blk_off, per expert (Np, Kp)): gate
    // (gw rows of d), up (mi rows of d), down (d rows of mi)
    size_t kpd = 0, kpm = 0;     // d and mi rounded up to 64
    int8_t* gate_b = nullptr;
    int8_t* up_b = nullptr;
    int8_t* down_b = nullptr;
};

// ---- kernel launchers (each returns hipError_t of the launch) ------------
// Activation quant of M rows of K f32 (row pitch K) into a8: row-major with
// pitch kp when mpb == 0, else blocked (blk_off) with R = mpb rows.
hipError_t launch_quant(const float* a, size_t m, size_t k, size_t kp,
                        int8_t* a8, float* sa, uint32_t* oidx, float* oval,
                        int* err, hipStream_t s, size_t mpb = 0);
// int8 GEMV for 1 <= m <= 4.
hipError_t launch_gemv_i8(const Weight& w, size_t m, const int8_t* a8,
                          const float* sa, const uint32_t* oidx,
                          const float* oval, float* out, int32_t* acc,
                          hipStream_t s);
// The whole int8 linear for one row (quant fused into the GEMV) when
// linear_m1_ok: K > 32, K % 4 == 0, a 16-byte aligned, Kp <= 20480.  a8o (Kp
// bytes, row-major) / sao / oio / ovo receive the quantisation when a8o is
// set; gmax caps the persistent grid (0: the default for the shape).
bool linear_m1_ok(const Weight& w, const float* a);
hipError_t launch_linear_m1(const Weight& w, const float* a, float* out, int32_t* acc,
                            int8_t* a8o, float* sao, uint32_t* oio, float* ovo, int* err,
                            hipStream_t s, int gmax = 0);
// The fused linear of a gated pair with the activation in its epilogue:
// w's rows interleaved in runs of hr (gated_rows: gate columns hr p ..
// hr p + hr - 1, then the same up columns), hr = linear_m1_rpp(Kp, N) / 2;
// out[c] = act(gate[c]) * up[c] for the N / 2 columns, act SiLU (silu) or
// gelu_tanh with constant gc, the separate activation kernel's values bit
// for bit.
int linear_m1_rpp(size_t kp, size_t n);
bool linear_m1_act_ok(const Weight& w, const float* a, int hr);
hipError_t launch_linear_m1_act(const Weight& w, const float* a, float* out, int hr, int silu, float gc, int* err,
                                hipStream_t s);
// Position of gate column c (up: + hr) in a gated pair interleaved in runs
// of hr (hr == 0: [gate | up], up at + half).
__host__ __device__ inline size_t gated_col(size_t c, size_t hr) { return hr ? 2 * hr * (c / hr) + c % hr : c; }
// int8 linear for 1 <= m <= 16 on row-major a8 (pitch kp) from the blocked
// weight copy; outputs bit-exact to the reference's M > 1 order.
hipError_t launch_skinny_i8(const Weight& w, size_t m, const int8_t* a8, const float* sa,
                            const uint32_t* oidx, const float* oval, float* out, int32_t* acc,
                            hipStream_t s);
// (valid rows of an (R, kp) row-major int8 matrix, pitch) -> blocked
// (blk_off, R rows); rows >= valid become zero.
hipError_t launch_blockify(const int8_t* src, size_t valid, size_t R, size_t kp,
                           size_t pitch, int8_t* dst, hipStream_t s);
// int8 MFMA GEMM for m > 16 on blocked a8 (R = round_up(m, 128)).
// ws: gemm_ws_bytes(m, kp, np) bytes of device workspace (the per-row-tile
// outlier union and correction operands, split-K partial tiles).
size_t gemm_ws_bytes(size_t m, size_t kp, size_t np);
hipError_t launch_gemm_i8(const Weight& w, size_t m, const int8_t* a8b,
                          const float* sa, const uint32_t* oidx,
                          const float* oval, float* out, int32_t* acc, void* ws,
                          hipStream_t s, bool acc_only = false);
// out = scale * (sa * acc + corr) from the GEMM's i32 sums with the
// reference's sequential outlier correction (the skinny kernel's order);
// acc_only above skips the GEMM's own approximate correction for this
hipError_t launch_i8_exact_epilogue(const Weight& w, size_t m, const float* sa, const uint32_t* oidx,
                                    const float* oval, const int32_t* acc, float* out, hipStream_t s);
// Context and weight internals, for engines built on the entry points: the
// context's device, its NaN error word (reported by frq_sync) and a
// weight's device layout.
int ctx_device(const frq_ctx* c);
// The device's compute units (hipDeviceAttributeMultiprocessorCount, cached).
int device_cus(int dev);
int* ctx_err(frq_ctx* c);
// The context workspace, grown to at least `bytes` (synchronises when it
// grows, so not under graph capture).
int ctx_ws(frq_ctx* c, size_t bytes, void** ws);
const Weight* weight_of(const frq_w* w);
// The int8 linear over m > 16 rows bit for bit as the skinny path gives it
// (the reference's M > 1 arm), in one pass: the MFMA GEMM's exact i32 sums
// and the sequential outlier correction.  i8_rows_exact_ok says whether the
// weight allows it (an int8 weight with its blocked copy, m > 16).
bool i8_rows_exact_ok(const frq_w* w, size_t m);
int mm_i8_rows_exact(frq_ctx* c, const frq_w* w, const float* d_a, size_t m, float* d_out);
// Sets the calling thread's frq_last_error() message and returns code.
int set_error(int code, const std::string& msg);
// The status of the calling thread's last failure.
int last_code();

// Row tables (FRQ_DT_F32 / F16 / ROWI8): bytes per padded row, and
// out[i] = dot(W[row i], x) for nout rows (cand == nullptr: rows 0..nout-1;
// else the candidate ids, invalid ones -inf).
size_t row_pitch(int dtype, size_t d);
hipError_t launch_rowdot(const Weight& w, const float* x, const int64_t* cand, size_t nout, float* out,
                         hipStream_t s);
// The full-table form that also folds the argmax (the last index of the
// largest value) into *best as (order-preserving value bits << 32 | row);
// *best must start at 0.  A NaN output sets *err.
hipError_t launch_rowdot_argmax(const Weight& w, const float* x, float* out, unsigned long long* best, int* err,
                                hipStream_t s);
hipError_t launch_rowdot_argmax_batch(const Weight& w, size_t nx, const float* x, size_t xs, float* xt, float* out,
                                      size_t os, unsigned long long* best, int* err, hipStream_t s);
// int4 linear (any m).
hipError_t launch_i4(const Weight& w, size_t m, const float* a, float* out,
                     float* wsf, hipStream_t s);
size_t i4_ws_floats(const Weight& w, size_t m);
// int4 at M == 1 in i4_dot_avx2's order (bit-exact) with coalesced loads, for
// K % 32 == 0 and g in {32, 64}; hipErrorNotSupported for other shapes.
hipError_t launch_i4_terms(const Weight& w, const float* a, float* out, hipStream_t s);
// int4 in the reference's orders for any m (M == 1 i4_dot_avx2, M > 1 the
// dequantise + sequential-k GEMM): the paths decode engines use.
hipError_t launch_i4_exact(const Weight& w, size_t m, const float* a, float* out, hipStream_t s);
// m rows each in the M == 1 order (i4_dot_avx2), weights read once.
// Batched decode rows (m independent rows, each in the M == 1 order):
// i4_rows_a4_ok says whether the weight takes the broadcast kernel, which
// reads its <= 16 rows in the a4 layout (launch_rows_to_a4: the rows
// interleaved by k-quads, i4_a4_floats(K) floats); launch_i4_m1_rows takes
// row-major rows and a4 scratch (or NULL: one M == 1 launch a row).
bool i4_rows_a4_ok(const Weight& w);
size_t i4_a4_floats(size_t k);
hipError_t launch_rows_to_a4(const float* a, size_t m, size_t k, float* a4, hipStream_t s);
hipError_t launch_i4_rows_a4(const Weight& w, size_t m, const float* a4, float* out, hipStream_t s);
hipError_t launch_i4_m1_rows(const Weight& w, size_t m, const float* a, float* out, float* a4, hipStream_t s);
// int4 (N, K/2) -> the MFMA layout (g == 32, K % 32 == 0); bytes of q4.
size_t i4_blocked_bytes(size_t n, size_t k);
hipError_t launch_i4_block(const uint8_t* raw, const uint16_t* sraw, size_t n,
                           size_t k, uint8_t* blk, uint16_t* sblk,
                           hipStream_t s);
// Affine int4 (q4a) linear (any m): packed rows in q4raw at pitch rpitch.
size_t q4a_pitch(size_t k);
hipError_t launch_q4a(const Weight& w, size_t m, const float* a, float* out, hipStream_t s);
// MoE.
size_t moe_ws_bytes(const MoeBank& b, size_t T, size_t topk);
hipError_t launch_moe(const MoeBank& b, const float* x, size_t T,
                      const float* logits, size_t topk, int norm_topk,
                      const float* pes, float* out, void* ws, int* err,
                      hipStream_t s);
hipError_t launch_moe_route(const float* logits, size_t T, size_t E,
                            size_t topk, int norm_topk, const float* pes,
                            int32_t* sel, float* w, int* err, hipStream_t s);
// (E, K, N) (in, out) int8 -> per expert blocked (np, kp) copies.
hipError_t launch_moe_block(const int8_t* src, size_t E, size_t K, size_t N, size_t kp,
                            size_t np, int8_t* dst, hipStream_t s);
hipError_t launch_expert_mm(const int8_t* q, const float* s, size_t inp,
                            size_t out, const float* x, size_t m, float* y,
                            hipStream_t st);
// expert_mm of expert e of a non-int8 bank matrix (dtype / g of the bank).
hipError_t launch_expert_mm_ex(const MoeBank& b, const ExpMat& mt, size_t e, const float* x, size_t m, float* y,
                               hipStream_t st);
// The i4 MFMA operand copy of an i4 bank matrix (mt.raw / mt.sc filled).
hipError_t launch_moe_i4_block(ExpMat& mt, size_t E, size_t g, hipStream_t st);

}  // namespace frq
