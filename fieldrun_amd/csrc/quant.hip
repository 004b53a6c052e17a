// quant.hip — outlier-aware per-token int8 activation quant (gfx950).
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
// in ascending channel order.  A NaN in a row with t < K is the reference's
// partial_cmp().unwrap() panic: the kernel raises *err.
//
// One workgroup per row.  The (t+1)-th largest is found without sorting:
//   1. each thread's max |a| (coalesced sweep);
//   2. tau0 = the (t+1)-th largest thread max (LDS radix select over BLOCK
//      values).  At least t+1 elements are >= tau0, so bulk_max >= tau0;
//   3. elements >= tau0 (typically a few dozen) are compacted into LDS and
//      an 8-bit-digit radix select over them yields bulk_max exactly; if more
//      than CAP survive (e.g. constant rows) the select runs over the whole
//      row from global memory instead;
//   4. the outliers are taken in channel order by contiguous per-thread
//      chunks and block scans (ties, then selected counts) into an LDS list
//      and a channel bitmap;
//   5. a8 is written once, coalesced, with the outlier slots zero.
// |a| is compared as its IEEE bit pattern, which orders non-negative floats.
#include "frq_internal.h"

namespace frq {

namespace {

constexpr int CAP = 1024;

__device__ __forceinline__ uint32_t absbits(float v) {
    return __float_as_uint(v) & 0x7FFFFFFFu;
}

// Exclusive scan of one uint per thread across the block; *total gets the sum.
template <int BLOCK>
__device__ uint32_t block_excl_scan(uint32_t v, uint32_t* lds /*BLOCK/64+1*/,
                                    uint32_t* total) {
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
        for (int w = 0; w < BLOCK / 64; ++w) {
            uint32_t c = lds[w];
            lds[w] = run;
            run += c;
        }
        lds[BLOCK / 64] = run;
    }
    __syncthreads();
    uint32_t r = lds[wave] + incl - v;
    *total = lds[BLOCK / 64];
    __syncthreads();
    return r;
}

// Value of descending rank `rank` (0 = largest) among n non-negative float
// bit patterns given by get(i).  Four 8-bit MSB-first digit passes.
template <int BLOCK, typename Get>
__device__ uint32_t radix_select_desc(Get get, int n, uint32_t rank,
                                      uint32_t* hist, uint32_t* bc) {
    uint32_t prefix = 0, mask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = threadIdx.x; i < 256; i += BLOCK) hist[i] = 0;
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += BLOCK) {
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

template <int BLOCK>
__global__ __launch_bounds__(BLOCK) void quant_rows(
    const float* __restrict__ A, int K, int Kp, int t, int8_t* __restrict__ a8,
    float* __restrict__ sa_out, uint32_t* __restrict__ oidx,
    float* __restrict__ oval, int* __restrict__ err) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t bc[2];
    __shared__ uint32_t vals[CAP > BLOCK ? CAP : BLOCK];
    __shared__ uint32_t scan_lds[BLOCK / 64 + 1];
    __shared__ uint32_t ncand;
    __shared__ int nan_flag;
    __shared__ uint32_t sel_i[FRQ_T];
    __shared__ float sel_v[FRQ_T];
    extern __shared__ uint32_t bitmap[];  // ceil(Kp/32) words

    const int row = blockIdx.x;
    const float* a = A + (size_t)row * K;
    int8_t* q = a8 + (size_t)row * Kp;
    const int tid = threadIdx.x;

    if (tid == 0) { ncand = 0; nan_flag = 0; }
    // 1. thread max and NaN check
    uint32_t mx = 0;
    int has_nan = 0;
    for (int k = tid; k < K; k += BLOCK) {
        float v = a[k];
        has_nan |= (v != v);
        uint32_t b = absbits(v);
        mx = b > mx ? b : mx;
    }
    __syncthreads();
    if (has_nan) nan_flag = 1;
    vals[tid] = mx;
    __syncthreads();

    uint32_t bulk = 0;
    if (t < K) {
        if (nan_flag) {
            // the reference panics here; the call reports FRQ_ERR_NAN.  Write
            // in-bounds placeholders (a8 = 0, sa = 1, outliers 0..t-1 with
            // value 0) so the kernels queued after this one read valid data.
            if (tid == 0) { atomicOr(err, 1); sa_out[row] = 1.0f; }
            for (int k = tid; k < Kp; k += BLOCK) q[k] = 0;
            for (int k = tid; k < FRQ_T; k += BLOCK) {
                oidx[(size_t)row * FRQ_T + k] = k < t ? (uint32_t)k : 0u;
                oval[(size_t)row * FRQ_T + k] = 0.0f;
            }
            return;  // uniform across the block
        }
        // 2. lower bound tau0 from the thread maxima
        uint32_t tau0 = radix_select_desc<BLOCK>([&](int i) { return vals[i]; },
                                                 BLOCK, (uint32_t)t, hist, bc);
        // 3. compact candidates >= tau0
        for (int k = tid; k < K; k += BLOCK) {
            uint32_t b = absbits(a[k]);
            if (b >= tau0) {
                uint32_t slot = atomicAdd(&ncand, 1u);
                if (slot < (uint32_t)CAP) vals[slot] = b;
            }
        }
        __syncthreads();
        const uint32_t nc = ncand;
        if (nc <= (uint32_t)CAP) {
            bulk = radix_select_desc<BLOCK>([&](int i) { return vals[i]; }, (int)nc,
                                            (uint32_t)t, hist, bc);
        } else {
            bulk = radix_select_desc<BLOCK>([&](int i) { return absbits(a[i]); }, K,
                                            (uint32_t)t, hist, bc);
        }
    }
    const float bulkf = __uint_as_float(bulk);
    const float sa = bulkf > 0.0f ? bulkf / 127.0f : 1.0f;

    // 4. outliers in ascending channel order -> LDS list + channel bitmap
    for (int w = tid; w < (Kp + 31) / 32; w += BLOCK) bitmap[w] = 0u;
    __syncthreads();
    if (t == K) {
        if (tid < K) { sel_i[tid] = (uint32_t)tid; sel_v[tid] = a[tid]; }
        __syncthreads();
        if (tid < K) atomicOr(&bitmap[tid >> 5], 1u << (tid & 31));
    } else {
        const int C = (K + BLOCK - 1) / BLOCK;
        const int lo = tid * C, hi = min(lo + C, K);
        uint32_t gt = 0, ties = 0;
        for (int k = lo; k < hi; ++k) {
            uint32_t b = absbits(a[k]);
            gt += b > bulk;
            ties += b == bulk;
        }
        uint32_t gt_total, ties_total;
        block_excl_scan<BLOCK>(gt, scan_lds, &gt_total);
        uint32_t tie_base = block_excl_scan<BLOCK>(ties, scan_lds, &ties_total);
        // ties to take (>= 1 when bulk is the exact (t+1)-th largest)
        const uint32_t need = gt_total < (uint32_t)t ? (uint32_t)t - gt_total : 0u;
        uint32_t take = need > tie_base ? min(need - tie_base, ties) : 0u;
        uint32_t sel_total;
        uint32_t base = block_excl_scan<BLOCK>(gt + take, scan_lds, &sel_total);
        if (gt + take) {
            uint32_t tie_seen = 0;
            for (int k = lo; k < hi; ++k) {
                float v = a[k];
                uint32_t b = absbits(v);
                bool s = b > bulk;
                if (b == bulk) { s = tie_seen < take; tie_seen++; }
                if (s && base < (uint32_t)FRQ_T) {
                    sel_i[base] = (uint32_t)k;
                    sel_v[base] = v;
                    atomicOr(&bitmap[k >> 5], 1u << (k & 31));
                    base++;
                }
            }
        }
    }
    __syncthreads();

    // 5. quantise (coalesced); outlier and padding channels are zero
    for (int k = tid; k < Kp; k += BLOCK) {
        int8_t r = 0;
        if (k < K && !((bitmap[k >> 5] >> (k & 31)) & 1u)) {
            float x = __builtin_roundf(a[k] / sa);
            // Rust `as i32` saturates and maps NaN to 0; then clamp(-127,127)
            r = (x != x) ? (int8_t)0
                         : (int8_t)(x < -127.0f ? -127 : (x > 127.0f ? 127 : (int)x));
        }
        q[k] = r;
    }
    uint32_t* oi = oidx + (size_t)row * FRQ_T;
    float* ov = oval + (size_t)row * FRQ_T;
    for (int k = tid; k < FRQ_T; k += BLOCK) {
        oi[k] = k < t ? sel_i[k] : 0u;
        ov[k] = k < t ? sel_v[k] : 0.0f;
    }
    if (tid == 0) sa_out[row] = sa;
}

}  // namespace

hipError_t launch_quant(const float* a, size_t m, size_t k, size_t kp,
                        int8_t* a8, float* sa, uint32_t* oidx, float* oval,
                        int* err, hipStream_t s) {
    if (m == 0) return hipSuccess;
    const int t = (int)(k < FRQ_T ? k : FRQ_T);
    const size_t lds = (kp + 31) / 32 * sizeof(uint32_t);
    if (lds > 96 * 1024) return hipErrorInvalidValue;
    if (m < 64)
        quant_rows<1024><<<dim3((unsigned)m), dim3(1024), lds, s>>>(
            a, (int)k, (int)kp, t, a8, sa, oidx, oval, err);
    else
        quant_rows<256><<<dim3((unsigned)m), dim3(256), lds, s>>>(
            a, (int)k, (int)kp, t, a8, sa, oidx, oval, err);
    return hipGetLastError();
}

}  // namespace frq
