// quant_core.h — one row of the outlier-aware int8 activation quant held in
// registers by a 256-thread workgroup (gfx950).
//
// Restates the I8 arm's activation quant of Bundle::mm
// (/root/reference/src/bundle.rs:691, 699-708 == 732-743; OUTLIER_T 309):
//   t        = min(32, K)
//   bulk_max = the (t+1)-th largest |a| of the row (0 when t == K)
//   sa       = bulk_max > 0 ? bulk_max / 127 : 1          (IEEE f32 divide)
//   a8[k]    = clamp(round(a[k] / sa) as i32, -127, 127)  (round half away)
//   the t largest-|a| channels get a8 = 0 and are kept as (idx, a) outliers.
// Ties at |a| == bulk_max, which the reference leaves to
// select_nth_unstable_by, go to the lowest channel index; outliers are listed
// in ascending channel order.
//
// The routines here cover rows with K % 4 == 0 and 32 < K <= 4 NT NV4 for a
// workgroup of NT = 256, 512 or 1024 threads, the row held as
// v[i] = a[4 (tid + NT i) ..] (float4, entries past K ignored):
//   row_select:   1. each thread's max |a|;
//                 2. tau: with 4 waves the 33rd largest thread max (every
//                    wave sorts its 64 maxima with a bitonic network on DPP /
//                    permlane lane exchanges, and every wave merges the four
//                    lists keeping the top 64; 8 waves: the eight lists
//                    merged pairwise the same way); with 16 waves the 33rd
//                    largest of the waves' top-3 lane maxima.  At least t+1
//                    elements are >= tau, so bulk_max >= tau;
//                 3. the elements >= tau (a few dozen on real rows) are
//                    compacted into per-wave LDS regions with ballot + mbcnt
//                    as keys (|a|, -channel, sign); each key's rank is counted
//                    against the others (the four waves a quarter each, over
//                    LDS broadcasts, for up to 64 keys; thread per key for up
//                    to FCAP), and beyond that (constant rows) a radix select
//                    over the row in global memory gives bulk_max;
//                 4. the t outliers (|a| > bulk_max, then ties at bulk_max
//                    lowest channel first) are placed in channel order by
//                    counting lower channels among them, with their values,
//                    and marked in an LDS bitmap.
//   row_quantize: a8 = round(a / sa) from the registers, the quotient taken
//                 as a Markstein-corrected product with RN(1/sa) (an IEEE
//                 divide for rows with extreme sa), four to a word, outlier
//                 slots zero.
// The standalone quant kernel and the fused M == 1 linear both run these, so
// they produce the same bytes.  |a| is compared as its IEEE bit pattern, which
// orders non-negative floats.
#pragma once

#include "frq_internal.h"

namespace frq {
namespace qc {

constexpr int BLOCK = 256;
constexpr int NW = BLOCK / 64;
constexpr int FCAP = 2048;  // candidate keys ranked in LDS

__device__ __forceinline__ uint32_t absbits(float v) {
    return __float_as_uint(v) & 0x7FFFFFFFu;
}

// Exclusive scan of one uint per thread across the block; *total gets the sum.
template <int NT>
__device__ uint32_t block_excl_scan(uint32_t v, uint32_t* lds /*NT/64+1*/, uint32_t* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        uint32_t y = __shfl_up(incl, off, 64);
        if (lane >= off) incl += y;
    }
    if (lane == 63) lds[wave] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t run = 0;
        for (int w = 0; w < NT / 64; ++w) {
            uint32_t c = lds[w];
            lds[w] = run;
            run += c;
        }
        lds[NT / 64] = run;
    }
    __syncthreads();
    uint32_t r = lds[wave] + incl - v;
    *total = lds[NT / 64];
    __syncthreads();
    return r;
}

// Value of descending rank `rank` (0 = largest) among n non-negative float
// bit patterns given by get(i).  Four 8-bit MSB-first digit passes.
template <int NT, typename Get>
__device__ uint32_t radix_select_desc(Get get, int n, uint32_t rank, uint32_t* hist, uint32_t* bc) {
    uint32_t prefix = 0, mask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = threadIdx.x; i < 256; i += NT) hist[i] = 0;
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += NT) {
            uint32_t v = get(i);
            if ((v & mask) == prefix) atomicAdd(&hist[(v >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            const int lane = threadIdx.x;
            // lane owns digits 255-4l .. 252-4l (descending order)
            uint32_t h0 = hist[255 - 4 * lane], h1 = hist[254 - 4 * lane];
            uint32_t h2 = hist[253 - 4 * lane], h3 = hist[252 - 4 * lane];
            uint32_t s = h0 + h1 + h2 + h3, incl = s;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                uint32_t y = __shfl_up(incl, off, 64);
                if (lane >= off) incl += y;
            }
            uint32_t c = incl - s;
            if (c <= rank && rank < incl) {
                int d;
                if (rank < c + h0) {
                    d = 255 - 4 * lane;
                } else if (rank < c + h0 + h1) {
                    c += h0; d = 254 - 4 * lane;
                } else if (rank < c + h0 + h1 + h2) {
                    c += h0 + h1; d = 253 - 4 * lane;
                } else {
                    c += h0 + h1 + h2; d = 252 - 4 * lane;
                }
                bc[0] = (uint32_t)d;
                bc[1] = c;
            }
        }
        __syncthreads();
        prefix |= bc[0] << shift;
        mask |= 255u << shift;
        rank -= bc[1];
        __syncthreads();
    }
    return prefix;
}

// Bitonic networks across the 64-lane wave on VALU lane exchanges.
template <int J, int K, bool DESC, typename T, typename X>
__device__ __forceinline__ T bstage(T x, X xs) {
    const int lane = threadIdx.x & 63;
    const T y = xs(x);
    const bool lower = !(lane & J), dir = !(lane & K);
    const bool keep_big = DESC ? (lower == dir) : (lower != dir);
    return keep_big ? (x > y ? x : y) : (x < y ? x : y);
}

template <bool DESC, typename T, typename X1, typename X2, typename X4, typename X8, typename X16,
          typename X32>
__device__ __forceinline__ T bitonic64(T x, X1 s1, X2 s2, X4 s4, X8 s8, X16 s16, X32 s32) {
    x = bstage<1, 2, DESC>(x, s1);
    x = bstage<2, 4, DESC>(x, s2); x = bstage<1, 4, DESC>(x, s1);
    x = bstage<4, 8, DESC>(x, s4); x = bstage<2, 8, DESC>(x, s2); x = bstage<1, 8, DESC>(x, s1);
    x = bstage<8, 16, DESC>(x, s8); x = bstage<4, 16, DESC>(x, s4); x = bstage<2, 16, DESC>(x, s2);
    x = bstage<1, 16, DESC>(x, s1);
    x = bstage<16, 32, DESC>(x, s16); x = bstage<8, 32, DESC>(x, s8); x = bstage<4, 32, DESC>(x, s4);
    x = bstage<2, 32, DESC>(x, s2); x = bstage<1, 32, DESC>(x, s1);
    x = bstage<32, 64, DESC>(x, s32); x = bstage<16, 64, DESC>(x, s16); x = bstage<8, 64, DESC>(x, s8);
    x = bstage<4, 64, DESC>(x, s4); x = bstage<2, 64, DESC>(x, s2); x = bstage<1, 64, DESC>(x, s1);
    return x;
}

__device__ __forceinline__ uint32_t wave_sort_desc(uint32_t x) {
    return bitonic64<true>(x, xshfl<1>, xshfl<2>, xshfl<4>, xshfl<8>, xshfl<16>, xshfl<32>);
}
// Top 64 of two descending 64-lists, a in lane order and b reversed
// (lane l holds b[63-l]): max() forms a bitonic sequence, the half-cleaners
// sort it descending.
__device__ __forceinline__ uint32_t merge_top64(uint32_t a, uint32_t b_rev) {
    uint32_t c = max(a, b_rev);
    c = bstage<32, 64, true>(c, xshfl<32>);
    c = bstage<16, 64, true>(c, xshfl<16>);
    c = bstage<8, 64, true>(c, xshfl<8>);
    c = bstage<4, 64, true>(c, xshfl<4>);
    c = bstage<2, 64, true>(c, xshfl<2>);
    c = bstage<1, 64, true>(c, xshfl<1>);
    return c;
}

// round(q) half away from zero (Rust f32::round), clamped to [-127, 127];
// q finite.  trunc + exact fraction: |q - trunc(q)| is exact in f32.
__device__ __forceinline__ uint32_t rq8(float q) {
    const float t = __builtin_truncf(q);
    const float r = __builtin_fabsf(q - t) >= 0.5f ? t + __builtin_copysignf(1.0f, q) : t;
    return (uint32_t)(uint8_t)(int8_t)(int)__builtin_amdgcn_fmed3f(r, -127.0f, 127.0f);
}

// RN(a / sa) by r = RN(1/sa) and one FMA residual correction (Markstein).
__device__ __forceinline__ float qdiv_fast(float a, float sa, float r) {
    const float q = a * r;
    const float e = __builtin_fmaf(-q, sa, a);
    return __builtin_fmaf(e, r, q);
}

// Exact path for rows outside the fast path's range (IEEE divide; Rust `as
// i32` saturation maps NaN to 0).
__device__ __forceinline__ uint32_t q8_slow(float a, float sa) {
    const float x = __builtin_roundf(a / sa);
    return (x != x) ? 0u : (uint32_t)(uint8_t)(int8_t)(x < -127.0f ? -127 : (x > 127.0f ? 127 : (int)x));
}

// Candidate key of channel k with IEEE bits b: |a| in the high word, then
// 2^31 - 1 - k (lower channel first among equal magnitudes), then the sign
// bit, so keys order as (|a|, -k) and still carry a exactly.
__device__ __forceinline__ unsigned long long cand_key(uint32_t b, uint32_t k) {
    return ((unsigned long long)(b & 0x7FFFFFFFu) << 32) | ((0x7FFFFFFFu - k) << 1) | (b >> 31);
}
__device__ __forceinline__ uint32_t key_chan(unsigned long long key) {
    return 0x7FFFFFFFu - ((uint32_t)key >> 1);
}
__device__ __forceinline__ uint32_t key_bits(unsigned long long key) {
    return (uint32_t)(key >> 32) | ((uint32_t)key << 31);
}

// LDS of one row's selection by NT threads (besides the candidate keys and
// the bitmap, which the caller places so that it can reuse their space).
template <int NT>
struct RowLdsT {
    static constexpr int W = NT / 64;
    unsigned long long top[FRQ_T + 1];
    uint32_t hist[256];
    uint32_t scan[W + 1];
    uint32_t ws[W][64];
    uint32_t wn[W];
    uint32_t wcnt[W];
    uint32_t bc[2];
    uint32_t sel_i[FRQ_T];
    float sel_v[FRQ_T];
    uint32_t rank[64];
    uint32_t cch[64];
    unsigned long long ck[W][64];
};
using RowLds = RowLdsT<BLOCK>;

struct RowSel {
    float sa;
    bool fast;  // Markstein quotient valid for every element
    bool nan;   // the row holds a NaN (the reference panics)
};

// Steps 1-4 for the row a (K floats, K % 4 == 0, 32 < K <= 1024 NV4) held in
// v (entries past K/4 are ignored).  cand: FCAP keys of LDS; bitmap: nbw >= ceil(K/32) words of LDS, cleared
// here.  Ends with a barrier; then sel_i / sel_v hold the 32 outliers in
// channel order and bitmap marks them, and cand is free.  A NaN row returns
// nan (uniformly) with sel_i[q] = q, sel_v[q] = 0 and an empty bitmap.
template <int NV4, int NT = BLOCK>
__device__ RowSel row_select(const float* __restrict__ a, int K, const float4 (&v)[NV4], RowLdsT<NT>& L,
                             unsigned long long* cand, uint32_t* bitmap, int nbw) {
    constexpr int NW = NT / 64, BLOCK = NT;
    static_assert(NW == 4 || NW == 8 || NW == 16, "4, 8 or 16 waves");
    constexpr int TOPW = 3;  // lane maxima a wave contributes (16 waves)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K4 = K >> 2;
    uint32_t mx = 0;  // max |a| bits; NaN shows as > 0x7F800000
#pragma unroll
    for (int i = 0; i < NV4; ++i) {
        const uint32_t m4 = max(max(absbits(v[i].x), absbits(v[i].y)), max(absbits(v[i].z), absbits(v[i].w)));
        mx = max(mx, tid + BLOCK * i < K4 ? m4 : 0u);
    }
    // threshold tau, every element above the (t+1)-th largest |a| is >= tau.
    // 4 waves: tau = the 33rd largest thread maximum (at least 33 elements
    // are >= tau; for iid rows only a few dozen pass): every wave sorts its
    // 64 maxima, and after one barrier every wave merges the four lists
    // itself.  16 waves: tau = the 33rd largest of the waves' top-3 lane
    // maxima (48 distinct elements, sorted in every wave).  The NaN check
    // rides on the same barrier.
    const bool wnan = __builtin_amdgcn_ballot_w64(mx > 0x7F800000u) != 0;  // NaN bits
    const uint32_t srt = wave_sort_desc(mx);
    if (NW <= 8 || lane < TOPW) L.ws[wave][lane] = srt;
    if (lane == 0) L.wn[wave] = wnan;
    for (int w = tid; w < nbw; w += BLOCK) bitmap[w] = 0u;
    if (tid < 64) L.rank[tid] = 0u;
    __syncthreads();
    uint32_t anynan = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) anynan |= L.wn[w];
    if (anynan) {
        if (tid < FRQ_T) { L.sel_i[tid] = (uint32_t)tid; L.sel_v[tid] = 0.0f; }
        __syncthreads();
        return {1.0f, false, true};
    }
    uint32_t tau;
    if constexpr (NW == 4) {
        const uint32_t mx01 = merge_top64(L.ws[0][lane], L.ws[1][63 - lane]);
        const uint32_t mx23 = merge_top64(L.ws[2][lane], L.ws[3][63 - lane]);
        tau = __builtin_amdgcn_readlane(merge_top64(mx01, __shfl(mx23, 63 - lane, 64)), FRQ_T);
    } else if constexpr (NW == 8) {
        // the 33rd largest thread maximum, the eight lists merged pairwise
        const uint32_t mx01 = merge_top64(L.ws[0][lane], L.ws[1][63 - lane]);
        const uint32_t mx23 = merge_top64(L.ws[2][lane], L.ws[3][63 - lane]);
        const uint32_t mx45 = merge_top64(L.ws[4][lane], L.ws[5][63 - lane]);
        const uint32_t mx67 = merge_top64(L.ws[6][lane], L.ws[7][63 - lane]);
        const uint32_t mx03 = merge_top64(mx01, __shfl(mx23, 63 - lane, 64));
        const uint32_t mx47 = merge_top64(mx45, __shfl(mx67, 63 - lane, 64));
        tau = __builtin_amdgcn_readlane(merge_top64(mx03, __shfl(mx47, 63 - lane, 64)), FRQ_T);
    } else {
        // the 33rd largest of the waves' top-3 lane maxima: 48 distinct
        // elements, so at least 33 elements are >= it
        const uint32_t t3 = lane < TOPW * NW ? L.ws[lane / TOPW][lane % TOPW] : 0u;
        tau = __builtin_amdgcn_readlane(wave_sort_desc(t3), FRQ_T);
    }
    // compact candidates into per-wave regions of cand[] (FCAP/4 keys each),
    // offsets from ballots
    constexpr int WCAP = FCAP / NW;
    uint32_t wcount = 0;
#pragma unroll
    for (int i = 0; i < NV4; ++i) {
        const uint32_t b0 = __float_as_uint(v[i].x), b1 = __float_as_uint(v[i].y);
        const uint32_t b2 = __float_as_uint(v[i].z), b3 = __float_as_uint(v[i].w);
        const bool any = max(max(absbits(v[i].x), absbits(v[i].y)), max(absbits(v[i].z), absbits(v[i].w))) >= tau;
        if (__builtin_amdgcn_ballot_w64(any)) {  // rare: wave-uniform skip
            const uint32_t base = 4u * (uint32_t)(tid + BLOCK * i);
            const uint32_t bb[4] = {b0, b1, b2, b3};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const bool hit = (bb[c] & 0x7FFFFFFFu) >= tau && base + c < (uint32_t)K;
                const unsigned long long m = __builtin_amdgcn_ballot_w64(hit);
                const uint32_t below = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                const uint32_t slot = wcount + below;
                if (hit && slot < (uint32_t)WCAP) cand[wave * WCAP + slot] = cand_key(bb[c], base + c);
                wcount += (uint32_t)__builtin_popcountll(m);
            }
        }
    }
    if (lane == 0) L.wcnt[wave] = wcount;
    __syncthreads();
    // concatenate the four regions (keys are independent of order)
    uint32_t wc[NW], woff[NW + 1];  // wave-uniform: kept in SGPRs
    bool overflow = false;
    woff[0] = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        wc[w] = __builtin_amdgcn_readfirstlane(L.wcnt[w]);
        overflow |= wc[w] > (uint32_t)WCAP;
        woff[w + 1] = woff[w] + wc[w];
    }
    const uint32_t nc = overflow ? (uint32_t)FCAP + 1u : woff[NW];
    auto cand_at = [&](uint32_t i) -> unsigned long long {
        int w = 0;
#pragma unroll
        for (int x = 1; x < NW; ++x) w += i >= woff[x];
        return cand[w * WCAP + (i - woff[w])];
    };
    uint32_t bulk;
    if (nc <= (uint32_t)FCAP) {
        if (nc <= 64) {
            // rank of lane l's key among the nc (distinct) keys: wave w
            // counts the keys KPW w .. KPW w + KPW-1 above it, the counts
            // summed in LDS; ranks 0..32 go to top[]
            // (each wave gathers the keys into its own contiguous copy first,
            // so that its reads share one base; keys are > 0, and the slots
            // past nc hold 0)
            constexpr int KPW = 64 / NW;
            const bool valid = lane < (int)nc;
            const unsigned long long key = valid ? cand_at(lane) : 0ull;
            L.ck[wave][lane] = key;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            const unsigned long long* kq = &L.ck[__builtin_amdgcn_readfirstlane(wave)][KPW * __builtin_amdgcn_readfirstlane(wave)];
            uint32_t part = 0;
#pragma unroll
            for (int jj = 0; jj < KPW; ++jj) part += kq[jj] > key;
            if (valid && part) atomicAdd(&L.rank[lane], part);
            __syncthreads();
            if (wave == 0) {
                const uint32_t rank = L.rank[lane];
                if (valid && rank <= (uint32_t)FRQ_T) L.top[rank] = key;
            }
        } else {
            // exact rank of every candidate; the 33 largest keys land in top[]
            for (uint32_t i = tid; i < nc; i += BLOCK) {
                const unsigned long long key = cand_at(i);
                uint32_t rank = 0;
#pragma unroll
                for (int w = 0; w < NW; ++w)
                    for (uint32_t j = 0; j < wc[w]; ++j) rank += cand[w * WCAP + j] > key;
                if (rank <= (uint32_t)FRQ_T) L.top[rank] = key;
            }
            __syncthreads();
        }
        if (wave == 0) {
            // the 32 outliers in channel order: position = the number of
            // outliers on a lower channel (counted over LDS broadcasts)
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
            const unsigned long long key = L.top[lane < FRQ_T ? lane : 0];
            const uint32_t ch = lane < FRQ_T ? key_chan(key) : 0xFFFFFFFFu;
            L.cch[lane] = ch;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            uint32_t pos = 0;
#pragma unroll
            for (int j = 0; j < FRQ_T; j += 4) {
                const uint4 c4 = *reinterpret_cast<const uint4*>(&L.cch[j]);
                pos += (c4.x < ch) + (c4.y < ch) + (c4.z < ch) + (c4.w < ch);
            }
            if (lane < FRQ_T) {
                const uint32_t sk = min(ch, (uint32_t)(K - 1));
                L.sel_i[pos] = sk;
                L.sel_v[pos] = __uint_as_float(key_bits(key));
                atomicOr(&bitmap[sk >> 5], 1u << (sk & 31));
            }
        }
    } else {
        // many near-equal magnitudes (e.g. constant rows): exact select over
        // the row in global memory, outliers by ordered chunks
        bulk = radix_select_desc<BLOCK>([&](int i) { return absbits(a[i]); }, K, (uint32_t)FRQ_T,
                                        L.hist, L.bc);
        const int C = (K + BLOCK - 1) / BLOCK;
        const int lo = tid * C, hi = min(lo + C, K);
        uint32_t gt = 0, ties = 0;
        for (int k = lo; k < hi; ++k) {
            const uint32_t b = absbits(a[k]);
            gt += b > bulk;
            ties += b == bulk;
        }
        uint32_t gt_total, ties_total, sel_total;
        block_excl_scan<BLOCK>(gt, L.scan, &gt_total);
        const uint32_t tie_base = block_excl_scan<BLOCK>(ties, L.scan, &ties_total);
        const uint32_t need = gt_total < (uint32_t)FRQ_T ? (uint32_t)FRQ_T - gt_total : 0u;
        const uint32_t take = need > tie_base ? min(need - tie_base, ties) : 0u;
        uint32_t pos = block_excl_scan<BLOCK>(gt + take, L.scan, &sel_total);
        if (gt + take) {
            uint32_t seen = 0;
            for (int k = lo; k < hi; ++k) {
                const float x = a[k];
                const uint32_t b = absbits(x);
                bool s = b > bulk;
                if (b == bulk) { s = seen < take; seen++; }
                if (s && pos < (uint32_t)FRQ_T) {
                    L.sel_i[pos] = (uint32_t)k;
                    L.sel_v[pos] = x;
                    atomicOr(&bitmap[k >> 5], 1u << (k & 31));
                    pos++;
                }
            }
        }
    }
    __syncthreads();
    // the row's largest |a| is top[0] (the radix path takes the IEEE divide)
    uint32_t rowmax = 0xFFFFFFFFu;
    if (nc <= (uint32_t)FCAP) {
        bulk = (uint32_t)(L.top[FRQ_T] >> 32);
        rowmax = (uint32_t)(L.top[0] >> 32);
    }
    const float bulkf = __uint_as_float(bulk);
    const float sa = bulkf > 0.0f ? bulkf / 127.0f : 1.0f;
    // the Markstein correction needs no under/overflow in q*sa and the residual
    const bool fast = sa >= 1e-30f && sa <= 1e30f && rowmax < 0x7A800000u;  // |a| < 2^118
    return {sa, fast, false};
}

// Step 5: the quantised word of float4 i4 (channels 4 i4 .. 4 i4 + 3) goes to
// st(i4, word), bytes in channel order, outlier slots zero; i4 < K/4 only.
template <int NV4, int NT = BLOCK, typename St>
__device__ __forceinline__ void row_quantize(const float4 (&v)[NV4], int K4, const uint32_t* bitmap,
                                             float sa, bool fast, St st) {
    constexpr int BLOCK = NT;
    const int tid = threadIdx.x;
    const float r = 1.0f / sa;
#pragma unroll
    for (int i = 0; i < NV4; ++i) {
        const int i4 = tid + BLOCK * i;
        if (i4 < K4) {
            const int base = 4 * i4;
            const uint32_t bw = bitmap[base >> 5] >> (base & 31);
            uint32_t w;
            if (fast) {
                w = rq8(qdiv_fast(v[i].x, sa, r)) | (rq8(qdiv_fast(v[i].y, sa, r)) << 8) |
                    (rq8(qdiv_fast(v[i].z, sa, r)) << 16) | (rq8(qdiv_fast(v[i].w, sa, r)) << 24);
            } else {
                w = q8_slow(v[i].x, sa) | (q8_slow(v[i].y, sa) << 8) | (q8_slow(v[i].z, sa) << 16) |
                    (q8_slow(v[i].w, sa) << 24);
            }
            const uint32_t keep = ((bw & 1u) ? 0u : 0xFFu) | ((bw & 2u) ? 0u : 0xFF00u) |
                                  ((bw & 4u) ? 0u : 0xFF0000u) | ((bw & 8u) ? 0u : 0xFF000000u);
            st(i4, w & keep);
        }
    }
}

// The row a (K floats, 16-byte aligned) into v: float4 tid + 256 i.  Entries
// past K/4 repeat the last float4 (clamped addresses, no branches, so that
// loads issued after these need not wait for them); row_select and
// row_quantize ignore them.
template <int NV4, int NT = BLOCK>
__device__ __forceinline__ void row_load(const float* __restrict__ a, int K4, float4 (&v)[NV4]) {
    constexpr int BLOCK = NT;
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NV4; ++i) v[i] = reinterpret_cast<const float4*>(a)[min(tid + BLOCK * i, K4 - 1)];
}

}  // namespace qc
}  // namespace frq
