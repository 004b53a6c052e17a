// quant.hip — outlier-aware per-token int8 activation quant (gfx950).
//
// Restates the I8 arm's activation quant of Bundle::mm
// (/root/reference/src/bundle.rs:691, 699-708 == 732-743; OUTLIER_T 309);
// the rule, tie order and outlier order are stated in quant_core.h.  A NaN
// in a row with t < K is the reference's partial_cmp().unwrap() panic: the
// kernel raises *err.
//
// One workgroup per row; HBM traffic is one read of the f32 row and one
// write of the i8 row.  The (t+1)-th largest is found without a full sort.
// quant_rows_fast (K % 4 == 0, 32 < K <= 20480, 16-byte aligned rows; every
// shape of the hot path): the row in registers, quant_core.h's row_select and
// row_quantize, the a8 row written once, coalesced.
// quant_rows (any other K or alignment): the same steps from global memory
// with LDS radix selects (four 8-bit MSB-first digit passes) and block scans,
// and an IEEE divide.
#include "quant_core.h"

namespace frq {

namespace {

using qc::absbits;
using qc::block_excl_scan;
using qc::radix_select_desc;

constexpr int CAP = 1024;

template <int BLOCK>
__global__ __launch_bounds__(BLOCK) void quant_rows(
    const float* __restrict__ A, int K, int Kp, int t, int8_t* __restrict__ a8,
    float* __restrict__ sa_out, uint32_t* __restrict__ oidx,
    float* __restrict__ oval, int* __restrict__ err, int mpb) {
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
    // a8 byte k of this row: row-major (pitch Kp) or blocked (R = mpb)
    auto qa = [&](int k) -> int8_t* {
        return mpb ? a8 + blk_off((size_t)row, (size_t)k, (size_t)mpb) : a8 + (size_t)row * Kp + k;
    };
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
            for (int k = tid; k < Kp; k += BLOCK) *qa(k) = 0;
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
        *qa(k) = r;
    }
    uint32_t* oi = oidx + (size_t)row * FRQ_T;
    float* ov = oval + (size_t)row * FRQ_T;
    for (int k = tid; k < FRQ_T; k += BLOCK) {
        oi[k] = k < t ? sel_i[k] : 0u;
        ov[k] = k < t ? sel_v[k] : 0.0f;
    }
    if (tid == 0) sa_out[row] = sa;
}

// ---------------------------------------------------------------------------
// Fast path: K % 4 == 0, 32 < K <= 1024 * NV4, 16-byte aligned rows.
template <int NV4>
__global__ __launch_bounds__(qc::BLOCK) void quant_rows_fast(
    const float* __restrict__ A, int K, int Kp, int8_t* __restrict__ a8,
    float* __restrict__ sa_out, uint32_t* __restrict__ oidx,
    float* __restrict__ oval, int* __restrict__ err, int mpb) {
    __shared__ qc::RowLds L;
    __shared__ unsigned long long cand[qc::FCAP];
    extern __shared__ uint32_t bitmap[];  // ceil(Kp/32) words

    const int row = blockIdx.x, tid = threadIdx.x;
    const float* a = A + (size_t)row * K;
    // a8 byte k of this row: row-major (pitch Kp) or blocked (R = mpb)
    auto qa = [&](int k) -> int8_t* {
        return mpb ? a8 + blk_off((size_t)row, (size_t)k, (size_t)mpb) : a8 + (size_t)row * Kp + k;
    };
    const int K4 = K >> 2;
    float4 v[NV4];
    qc::row_load<NV4>(a, K4, v);
    const qc::RowSel s = qc::row_select<NV4>(a, K, v, L, cand, bitmap, (Kp + 31) / 32);
    if (s.nan) {
        // the reference panics here; the call reports FRQ_ERR_NAN.  In-bounds
        // placeholders (a8 = 0, sa = 1, outliers 0..31 with value 0) keep the
        // kernels queued after this one on valid data.
        if (tid == 0) atomicOr(err, 1);
        for (int i4 = tid; i4 < K4; i4 += qc::BLOCK) *reinterpret_cast<uint32_t*>(qa(4 * i4)) = 0u;
    } else {
        qc::row_quantize<NV4>(v, K4, bitmap, s.sa, s.fast,
                              [&](int i4, uint32_t w) { *reinterpret_cast<uint32_t*>(qa(4 * i4)) = w; });
    }
    for (int i4 = K4 + tid; i4 < Kp / 4; i4 += qc::BLOCK) *reinterpret_cast<uint32_t*>(qa(4 * i4)) = 0u;
    if (tid < FRQ_T) {
        oidx[(size_t)row * FRQ_T + tid] = L.sel_i[tid];
        oval[(size_t)row * FRQ_T + tid] = L.sel_v[tid];
    }
    if (tid == 0) sa_out[row] = s.sa;
}

}  // namespace

template <int NV4>
static void launch_fast(const float* a, size_t m, size_t k, size_t kp, int8_t* a8, float* sa,
                        uint32_t* oidx, float* oval, int* err, size_t lds, hipStream_t s, int mpb) {
    quant_rows_fast<NV4><<<dim3((unsigned)m), dim3(256), lds, s>>>(
        a, (int)k, (int)kp, a8, sa, oidx, oval, err, mpb);
}

hipError_t launch_quant(const float* a, size_t m, size_t k, size_t kp,
                        int8_t* a8, float* sa, uint32_t* oidx, float* oval,
                        int* err, hipStream_t s, size_t mpb) {
    if (m == 0) return hipSuccess;
    if (mpb && (mpb < m || mpb % 16 || kp % 64)) return hipErrorInvalidValue;
    const int t = (int)(k < FRQ_T ? k : FRQ_T);
    const size_t lds = (kp + 31) / 32 * sizeof(uint32_t);
    if (lds > 32 * 1024) return hipErrorInvalidValue;
    if (k > FRQ_T && k % 4 == 0 && ((uintptr_t)a & 15) == 0 && k <= 256 * 20 * 4) {
        const size_t nv4 = (k / 4 + 255) / 256;
        if (nv4 <= 1) launch_fast<1>(a, m, k, kp, a8, sa, oidx, oval, err, lds, s, (int)mpb);
        else if (nv4 <= 2) launch_fast<2>(a, m, k, kp, a8, sa, oidx, oval, err, lds, s, (int)mpb);
        else if (nv4 <= 4) launch_fast<4>(a, m, k, kp, a8, sa, oidx, oval, err, lds, s, (int)mpb);
        else if (nv4 <= 8) launch_fast<8>(a, m, k, kp, a8, sa, oidx, oval, err, lds, s, (int)mpb);
        else if (nv4 <= 14) launch_fast<14>(a, m, k, kp, a8, sa, oidx, oval, err, lds, s, (int)mpb);
        else launch_fast<20>(a, m, k, kp, a8, sa, oidx, oval, err, lds, s, (int)mpb);
        return hipGetLastError();
    }
    if (m < 64)
        quant_rows<1024><<<dim3((unsigned)m), dim3(1024), lds, s>>>(
            a, (int)k, (int)kp, t, a8, sa, oidx, oval, err, (int)mpb);
    else
        quant_rows<256><<<dim3((unsigned)m), dim3(256), lds, s>>>(
            a, (int)k, (int)kp, t, a8, sa, oidx, oval, err, (int)mpb);
    return hipGetLastError();
}

}  // namespace frq
