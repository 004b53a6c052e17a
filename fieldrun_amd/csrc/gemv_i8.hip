// gemv_i8.hip — int8 W8A8 GEMV for decode shapes (1 <= M <= 4), gfx950.
//
// Restates the M==1 arm of Bundle::mm's I8 path and its M>1 twin
// (/root/reference/src/bundle.rs:744-752, 709-715):
//   acc  = i8dot(a8, wt[j])                    i32, exact (1036-1053)
//   corr = sum over outliers of av * (wt[j,ch] as f32), ascending channel,
//          folded from -0.0 (Rust f32 Sum)
//   out  = scale[j] * (sa * (acc as f32) + corr)   (separate mul / add: the
//          library is built with -ffp-contract=off)
//
// HBM-bound: one pass over the (Np, Kp) int8 weight.  A workgroup of 256
// threads owns R output rows per row group; the group's threads split K in
// 16-byte chunks (128-bit coalesced loads), take four v_dot4_i32_i8 per chunk
// per token row, and reduce across the wave with DPP/shuffles and across the
// group's waves through LDS.  The activations (M x Kp bytes) sit in LDS and
// each 16-byte activation chunk is reused for the R weight rows.
#include "frq_internal.h"

namespace frq {

namespace {

__device__ __forceinline__ int dot16(const int4 a, const int4 w, int acc) {
    acc = __builtin_amdgcn_sdot4(a.x, w.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a.y, w.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, w.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, w.w, acc, false);
    return acc;
}

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// TPG threads per row group (64, 128 or 256); each group owns R rows.
template <int M, int R, int TPG>
__global__ __launch_bounds__(256) void gemv_i8_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ scale, int N,
    int Kp, int t, const int8_t* __restrict__ a8, const float* __restrict__ sa,
    const uint32_t* __restrict__ oidx, const float* __restrict__ oval,
    float* __restrict__ out, int32_t* __restrict__ acc_dbg) {
    constexpr int G = 256 / TPG;        // row groups per workgroup
    constexpr int WPG = TPG / 64;       // waves per group
    extern __shared__ int4 lds_a[];     // M * Kp bytes
    __shared__ int red[4][R][M];
    __shared__ uint32_t s_oi[M][FRQ_T];
    __shared__ float s_ov[M][FRQ_T];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = tid / TPG, gtid = tid % TPG;
    const int nch = Kp >> 4;
    for (int c = tid; c < M * nch; c += 256)
        lds_a[c] = reinterpret_cast<const int4*>(a8)[c];
    for (int c = tid; c < M * FRQ_T; c += 256) {
        s_oi[c / FRQ_T][c % FRQ_T] = oidx[c];
        s_ov[c / FRQ_T][c % FRQ_T] = oval[c];
    }
    __syncthreads();

    const int j0 = (blockIdx.x * G + grp) * R;
    int acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0;

    const int4* Wv = reinterpret_cast<const int4*>(W);
    const size_t rstride = (size_t)nch;
    int c = gtid;
    // two chunks in flight per row
    for (; c + TPG < nch; c += 2 * TPG) {
        int4 w0[R], w1[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            w0[r] = ntload16(&Wv[(size_t)(j0 + r) * rstride + c]);
            w1[r] = ntload16(&Wv[(size_t)(j0 + r) * rstride + c + TPG]);
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const int4 x0 = lds_a[m * nch + c], x1 = lds_a[m * nch + c + TPG];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                acc[r][m] = dot16(x0, w0[r], acc[r][m]);
                acc[r][m] = dot16(x1, w1[r], acc[r][m]);
            }
        }
    }
    if (c < nch) {
        int4 w0[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            w0[r] = ntload16(&Wv[(size_t)(j0 + r) * rstride + c]);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const int4 x0 = lds_a[m * nch + c];
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r][m] = dot16(x0, w0[r], acc[r][m]);
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            int v = wave_sum(acc[r][m]);
            if (lane == 0) red[wave][r][m] = v;
        }
    __syncthreads();

    // epilogue: one thread per (group, r, m)
    if (tid < G * R * M) {
        const int g = tid / (R * M), r = (tid / M) % R, m = tid % M;
        const int j = (blockIdx.x * G + g) * R + r;
        if (j < N) {
            int total = 0;
#pragma unroll
            for (int w = 0; w < WPG; ++w) total += red[g * WPG + w][r][m];
            const int8_t* wrow = W + (size_t)j * Kp;
            float corr = -0.0f;
            for (int q = 0; q < t; ++q)
                corr = corr + s_ov[m][q] * (float)wrow[min(s_oi[m][q], (uint32_t)(Kp - 1))];
            const float sam = sa[m];
            out[(size_t)m * N + j] = scale[j] * (sam * (float)total + corr);
            if (acc_dbg) acc_dbg[(size_t)m * N + j] = total;
        }
    }
}

template <int M, int R, int TPG>
hipError_t launch_t(const Weight& w, const int8_t* a8, const float* sa,
                    const uint32_t* oidx, const float* oval, float* out,
                    int32_t* acc, hipStream_t s) {
    constexpr int G = 256 / TPG;
    const unsigned grid = (unsigned)((w.n + (size_t)G * R - 1) / ((size_t)G * R));
    const size_t lds = (size_t)M * w.kp;
    const int t = (int)(w.k < FRQ_T ? w.k : FRQ_T);
    gemv_i8_kernel<M, R, TPG><<<dim3(grid), dim3(256), lds, s>>>(
        w.wt, w.scale, (int)w.n, (int)w.kp, t, a8, sa, oidx, oval, out, acc);
    return hipGetLastError();
}

template <int M>
hipError_t launch_m(const Weight& w, const int8_t* a8, const float* sa,
                    const uint32_t* oidx, const float* oval, float* out,
                    int32_t* acc, hipStream_t s) {
    const size_t nch = w.kp / 16;
    if (nch <= 64) return launch_t<M, 4, 64>(w, a8, sa, oidx, oval, out, acc, s);
    if (nch <= 256) return launch_t<M, 4, 128>(w, a8, sa, oidx, oval, out, acc, s);
    return launch_t<M, 4, 256>(w, a8, sa, oidx, oval, out, acc, s);
}

}  // namespace

hipError_t launch_gemv_i8(const Weight& w, size_t m, const int8_t* a8,
                          const float* sa, const uint32_t* oidx,
                          const float* oval, float* out, int32_t* acc,
                          hipStream_t s) {
    // rows j >= N read zero padding of the (Np, Kp) weight and are not stored
    if ((size_t)m * w.kp > 64 * 1024) return hipErrorInvalidValue;
    switch (m) {
        case 1: return launch_m<1>(w, a8, sa, oidx, oval, out, acc, s);
        case 2: return launch_m<2>(w, a8, sa, oidx, oval, out, acc, s);
        case 3: return launch_m<3>(w, a8, sa, oidx, oval, out, acc, s);
        case 4: return launch_m<4>(w, a8, sa, oidx, oval, out, acc, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace frq
