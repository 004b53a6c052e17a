// i4.hip — group-wise int4 W4A32 linear (gfx950).
//
// Restates the I4 arm of Bundle::mm (/root/reference/src/bundle.rs:760-799):
//  M == 1 (767-776): out[j] = i4_dot(row j), which on x86 is i4_dot_avx2
//    (199-225): per group, 8 lane accumulators each an FMA chain over the
//    group's 8-nibble chunks, then hsum256 ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7))
//    (146-153), a scalar mul+add tail, then sum += scale[g] * gsum.
//  M > 1 (777-798): w[kk,j] = s4 * scale[j, kk/g] (f32) then a.dot(w); the
//    oracle's stand-in for matrixmultiply's sgemm is a sequential-k FMA chain
//    per output, which the batched kernel below reproduces.
//
// Decode (M == 1, g == 32, K % 32 == 0) uses the blocked layout built at
// upload: for each 64-row block and group, the 64 rows' 16-byte groups are
// contiguous, so a wave (one row per lane) reads 1 KB per group with one
// coalesced 128-bit load per lane, and the group's 32 activations are the
// same for every lane (scalar loads into SGPRs).  To fill the chip when N is
// small the groups are split into S contiguous segments, one wave each; the
// per-segment folds are combined in segment order by a second tiny kernel.
// Within a group the arithmetic is i4_dot_avx2's; the fold over groups is
// re-associated (the 4 waves of a block take interleaved groups, combined in
// wave order, and S > 1 segments), which stays within 1e-5 of sum |a*w|.
// Shapes outside the blocked layout run i4_gemv_generic, bit-identical to
// i4_dot_avx2.
#include "frq_internal.h"

namespace frq {

namespace {

__device__ __forceinline__ float s4f(uint32_t word, int nib) {
    return (float)((int)(word << (28 - 4 * nib)) >> 28);
}

// One group of 32 nibbles (4 words) against 32 activations, AVX2 order.
__device__ __forceinline__ float group_avx2(const uint4 w, const float* __restrict__ a) {
    float l[8];
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int q = 0; q < 8; ++q) l[q] = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int q = 0; q < 8; ++q)
            l[q] = __builtin_fmaf(s4f(ws[c], q), a[8 * c + q], l[q]);
    const float q0 = l[0] + l[4], q1 = l[1] + l[5], q2 = l[2] + l[6], q3 = l[3] + l[7];
    return (q0 + q2) + (q1 + q3);
}

// One workgroup = one 64-row block x one segment of its groups.  Wave w of
// the workgroup takes the segment's groups w, w+4, ...; lane = row.  The
// four wave sums are added in wave order; with S > 1 segments the partials
// go to the workspace and i4_fold adds them in segment order.
__global__ __launch_bounds__(256) void i4_gemv_blocked(
    const uint8_t* __restrict__ blk, const uint16_t* __restrict__ sblk,
    const float* __restrict__ a, int N, int ng, int S,
    float* __restrict__ part, float* __restrict__ out) {
    __shared__ float wsum[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = blockIdx.x / S, seg = blockIdx.x % S;
    const int g0 = (int)((long)ng * seg / S), g1 = (int)((long)ng * (seg + 1) / S);
    const uint4* wp = reinterpret_cast<const uint4*>(blk) + ((size_t)b * ng) * 64 + lane;
    const uint16_t* sp = sblk + ((size_t)b * ng) * 64 + lane;
    float sum = 0.0f;
    for (int gi = g0 + wave; gi < g1; gi += 4) {
        const uint4 w = ntload16u(wp + (size_t)gi * 64);
        const float sc = h2f(sp[(size_t)gi * 64]);
        sum = sum + sc * group_avx2(w, a + 32 * gi);
    }
    wsum[wave][lane] = sum;
    __syncthreads();
    const int row = b * 64 + threadIdx.x;
    if (threadIdx.x < 64 && row < N) {
        const float p = ((wsum[0][lane] + wsum[1][lane]) + wsum[2][lane]) + wsum[3][lane];
        if (S == 1) out[row] = p;
        else part[(size_t)seg * N + row] = p;
    }
}

__global__ void i4_fold(const float* __restrict__ part, int N, int S,
                        float* __restrict__ out) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= N) return;
    float s = part[j];
    for (int q = 1; q < S; ++q) s = s + part[(size_t)q * N + j];
    out[j] = s;
}

// Generic M == 1 (any K, g): one thread per output row, i4_dot_avx2 order.
__global__ void i4_gemv_generic(const uint8_t* __restrict__ packed,
                                const uint16_t* __restrict__ scale, int N,
                                int K, int g, const float* __restrict__ a,
                                float* __restrict__ out) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= N) return;
    const int rb = (K + 1) / 2, ng = (K + g - 1) / g;
    const uint8_t* prow = packed + (size_t)j * rb;
    auto nib = [&](int i) -> float {
        const uint8_t byte = prow[i >> 1];
        const int v = (i & 1) ? (byte >> 4) : (byte & 0x0F);
        return (float)((int)((uint32_t)v << 28) >> 28);
    };
    float sum = 0.0f;
    int kk = 0, gi = 0;
    while (kk < K) {
        const int hi = min(kk + g, K);
        float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        while (kk + 8 <= hi) {
            const int base = (kk / 2) * 2;
            for (int q = 0; q < 8; ++q) l[q] = __builtin_fmaf(nib(base + q), a[kk + q], l[q]);
            kk += 8;
        }
        const float q0 = l[0] + l[4], q1 = l[1] + l[5], q2 = l[2] + l[6], q3 = l[3] + l[7];
        float gs = (q0 + q2) + (q1 + q3);
        for (; kk < hi; ++kk) gs = gs + a[kk] * nib(kk);
        sum = sum + h2f(scale[(size_t)j * ng + gi]) * gs;
        ++gi;
    }
    out[j] = sum;
}

// M > 1: dequantise w = s4 * scale (f32, exact) and run a sequential-k FMA
// chain per output (the oracle's sgemm order).  One thread per column j and
// up to 16 token rows; the token rows' activations are uniform across the
// wave (scalar loads), the weight row is the thread's own packed row.
template <int MT>
__global__ __launch_bounds__(256) void i4_gemm_rows(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scale,
    int N, int K, int g, const float* __restrict__ a, int M,
    float* __restrict__ out) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    const int m0 = blockIdx.y * MT;
    if (j >= N) return;
    const int rb = (K + 1) / 2, ng = (K + g - 1) / g;
    const uint8_t* prow = packed + (size_t)j * rb;
    const uint16_t* srow = scale + (size_t)j * ng;
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    for (int kk = 0; kk < K; ++kk) {
        const uint8_t byte = prow[kk >> 1];
        const int v = (kk & 1) ? (byte >> 4) : (byte & 0x0F);
        const float w = (float)((int)((uint32_t)v << 28) >> 28) * h2f(srow[kk / g]);
#pragma unroll
        for (int m = 0; m < MT; ++m)
            if (m0 + m < M) acc[m] = __builtin_fmaf(a[(size_t)(m0 + m) * K + kk], w, acc[m]);
    }
#pragma unroll
    for (int m = 0; m < MT; ++m)
        if (m0 + m < M) out[(size_t)(m0 + m) * N + j] = acc[m];
}

// Re-layout (N, K/2) packed + (N, ng) scales into 64-row blocks.
__global__ void i4_block_kernel(const uint8_t* __restrict__ raw,
                                const uint16_t* __restrict__ sraw, int N,
                                int K, uint8_t* __restrict__ blk,
                                uint16_t* __restrict__ sblk) {
    const int ng = K / 32, nblk = (N + 63) / 64;
    const size_t total = (size_t)nblk * ng * 64;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i % 64);
        const size_t bg = i / 64;
        const int gi = (int)(bg % ng), b = (int)(bg / ng);
        const int row = b * 64 + r;
        uint4 v = make_uint4(0, 0, 0, 0);
        uint16_t s = 0;
        if (row < N) {
            v = *reinterpret_cast<const uint4*>(raw + (size_t)row * (K / 2) + gi * 16);
            s = sraw[(size_t)row * ng + gi];
        }
        reinterpret_cast<uint4*>(blk)[i] = v;
        sblk[i] = s;
    }
}

int pick_segments(size_t n, size_t ng) {
    const size_t nblk = (n + 63) / 64;
    size_t s = (512 + nblk - 1) / nblk;  // aim for >= 512 workgroups (2048 waves)
    if (s > 8) s = 8;                    // the fold reads S partials per row
    if (s > ng / 4) s = ng / 4;          // >= 4 groups (one per wave) per segment
    if (s < 1) s = 1;
    return (int)s;
}

}  // namespace

size_t i4_ws_floats(const Weight& w, size_t m) {
    if (m != 1 || !w.i4_blocked) return 0;
    return (size_t)pick_segments(w.n, w.k / 32) * w.n;
}

hipError_t launch_i4_block(const uint8_t* raw, const uint16_t* sraw, size_t n,
                           size_t k, uint8_t* blk, uint16_t* sblk,
                           hipStream_t s) {
    i4_block_kernel<<<dim3(1024), dim3(256), 0, s>>>(raw, sraw, (int)n, (int)k, blk, sblk);
    return hipGetLastError();
}

hipError_t launch_i4(const Weight& w, size_t m, const float* a, float* out,
                     float* wsf, unsigned* tickets, hipStream_t s) {
    (void)tickets;
    if (m == 0) return hipSuccess;
    if (m == 1 && w.i4_blocked) {
        const int ng = (int)(w.k / 32), nblk = (int)((w.n + 63) / 64);
        const int S = pick_segments(w.n, (size_t)ng);
        i4_gemv_blocked<<<dim3((unsigned)(nblk * S)), dim3(256), 0, s>>>(
            w.q4, w.s4, a, (int)w.n, ng, S, wsf, out);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess || S == 1) return e;
        i4_fold<<<dim3((unsigned)((w.n + 255) / 256)), dim3(256), 0, s>>>(wsf, (int)w.n, S, out);
        return hipGetLastError();
    }
    if (m == 1) {
        i4_gemv_generic<<<dim3((unsigned)((w.n + 255) / 256)), dim3(256), 0, s>>>(
            w.q4raw, w.s4raw, (int)w.n, (int)w.k, (int)w.g, a, out);
        return hipGetLastError();
    }
    dim3 grid((unsigned)((w.n + 255) / 256), (unsigned)((m + 15) / 16));
    i4_gemm_rows<16><<<grid, dim3(256), 0, s>>>(w.q4raw, w.s4raw, (int)w.n, (int)w.k,
                                                (int)w.g, a, (int)m, out);
    return hipGetLastError();
}

}  // namespace frq
