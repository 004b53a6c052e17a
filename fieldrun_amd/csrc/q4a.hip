// q4a.hip — group-wise affine int4 (q4a) linears, gfx950.
//
// Restates Bundle::mm's Q4A arm (/root/reference/src/bundle.rs:802-845):
// w[k, j] = scale[j, k/g] * q + min[j, k/g], q the unsigned nibble of the
// packed (N, ceil(K/2)) rows (even k in the low nibble).
//   M == 1: out[j] = q4a_dot_avx2(row j) (231-258), the x86 production
//           order: per group two sets of eight lane accumulators over the
//           8-nibble chunks from the group's start (q lanes FMA chains of
//           q * a, a lanes add chains of a), each folded by hsum256
//           ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)), a mul+add tail, then
//           sum += scale*qsum + min*asum across the groups in order.
//   M > 1:  the dequantised weight (scale*q + min, a mul then an add) and
//           a.dot's order per output (matrixmultiply's sgemm: MM_KC-long k
//           blocks, each an FMA chain from +0, added in order):
//           q4a_rows_chain, a thread per (row, token),
//           where K and g are multiples of 32, else q4a_gemm_rows.
// Both bit-exact to the oracle.
//
// M == 1 layout of the work: the groups of a row are independent until the
// final in-order sum, so a thread takes one (row, group) pair at a time —
// adjacent threads read adjacent groups, so the packed bytes and the scale /
// min words arrive coalesced — and leaves scale*qsum + min*asum in LDS; one
// lane per row then adds its row's groups in order.  Rows are stored with a
// 16-byte pitch and the f16 scale and min of a group side by side in one
// 32-bit word (scale low, min high).
#include "frq_internal.h"

namespace frq {

namespace {

constexpr int QT = 256;

__device__ __forceinline__ float q4a_group(const uint8_t* __restrict__ prow, const float* __restrict__ a, int kk,
                                           int hi, uint32_t sm) {
    float l[8] = {0, 0, 0, 0, 0, 0, 0, 0}, m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (; kk + 8 <= hi; kk += 8) {
        const int base = kk & ~1;  // unpack8_nibbles reads from byte kk / 2
        const uint8_t* pb = prow + (base >> 1);
        const uint32_t w = (uint32_t)pb[0] | ((uint32_t)pb[1] << 8) | ((uint32_t)pb[2] << 16) | ((uint32_t)pb[3] << 24);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float av = a[kk + q];
            l[q] = __builtin_fmaf((float)((w >> (4 * q)) & 15u), av, l[q]);
            m[q] = m[q] + av;
        }
    }
    float qsum = ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7]));
    float asum = ((m[0] + m[4]) + (m[2] + m[6])) + ((m[1] + m[5]) + (m[3] + m[7]));
    for (; kk < hi; ++kk) {
        const uint8_t byte = prow[kk >> 1];
        const float q = (float)((kk & 1) ? (byte >> 4) : (byte & 15));
        qsum = qsum + a[kk] * q;
        asum = asum + a[kk];
    }
    return h2f((uint16_t)(sm & 0xffffu)) * qsum + h2f((uint16_t)(sm >> 16)) * asum;
}

// The same for a group of 32 * G4 nibbles held in registers (G4 16-byte
// words, loaded by the caller), the activations from
// the workgroup's LDS copy (as, padded 4 floats per 32 so the lanes, which
// take adjacent groups, fall on different banks).
template <int G4>
__device__ __forceinline__ float q4a_group_vec(const uint4 (&wv)[G4], const float* __restrict__ as, int k0,
                                               uint32_t sm) {
    float l[8] = {0, 0, 0, 0, 0, 0, 0, 0}, m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int h = 0; h < G4; ++h) {
        const uint32_t ws[4] = {wv[h].x, wv[h].y, wv[h].z, wv[h].w};
        const float* ab = as + (k0 + 32 * h) / 32 * 36;  // 32 activations at a 36-float stride
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float4 a0 = *reinterpret_cast<const float4*>(ab + 8 * c);
            const float4 a1 = *reinterpret_cast<const float4*>(ab + 8 * c + 4);
            const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                l[q] = __builtin_fmaf((float)((ws[c] >> (4 * q)) & 15u), av[q], l[q]);
                m[q] = m[q] + av[q];
            }
        }
    }
    const float qsum = ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7]));
    const float asum = ((m[0] + m[4]) + (m[2] + m[6])) + ((m[1] + m[5]) + (m[3] + m[7]));
    return h2f((uint16_t)(sm & 0xffffu)) * qsum + h2f((uint16_t)(sm >> 16)) * asum;
}

// M == 1: a workgroup owns `rb` rows; cg (LDS) holds their rb * ng group
// terms.  G4 > 0: g == 32 * G4 and the rows' 16-byte pitch keep every group
// aligned, and the activation row is staged in LDS first; G4 == 0: any g,
// byte loads and activations from global memory.
template <int G4>
__global__ __launch_bounds__(QT) void q4a_gemv_kernel(const uint8_t* __restrict__ packed, size_t pitch,
                                                      const uint32_t* __restrict__ sm, int N, int K, int g, int rb,
                                                      const float* __restrict__ a, float* __restrict__ out) {
    extern __shared__ float4 lds4[];
    float* cg = reinterpret_cast<float*>(lds4);
    const int ng = (K + g - 1) / g;
    const int r0 = blockIdx.x * rb;
    const int nr = min(rb, N - r0);
    const int items = nr * ng;
    const int ngp = (ng + 3) & ~3;  // row stride of the terms: 16-byte aligned rows
    if constexpr (G4 > 0) {
        float* as = cg + rb * ngp;
        for (int i = threadIdx.x; i < K / 4; i += QT)
            *reinterpret_cast<float4*>(as + (4 * i) / 32 * 36 + (4 * i) % 32) = reinterpret_cast<const float4*>(a)[i];
        __syncthreads();
        // the next item's nibbles and scale / min load while this one
        // computes (the index clamped to the last item: unconditional loads)
        auto fetch = [&](int p, uint4 (&w)[G4], uint32_t& s) {
            const int r = p / ng, gi = p - r * ng;
            const uint8_t* pg = packed + (size_t)(r0 + r) * pitch + (size_t)gi * 16 * G4;
#pragma unroll
            for (int h = 0; h < G4; ++h) w[h] = *reinterpret_cast<const uint4*>(pg + 16 * h);
            s = sm[(size_t)(r0 + r) * ng + gi];
        };
        if ((int)threadIdx.x < items) {
            uint4 wn[G4];
            uint32_t sn;
            fetch(threadIdx.x, wn, sn);
            for (int p = threadIdx.x; p < items; p += QT) {
                uint4 wc[G4];
#pragma unroll
                for (int h = 0; h < G4; ++h) wc[h] = wn[h];
                const uint32_t sc = sn;
                fetch(min(p + QT, items - 1), wn, sn);
                const int rr = p / ng, gi = p - rr * ng;
                cg[rr * ngp + gi] = q4a_group_vec<G4>(wc, as, gi * g, sc);
            }
        }
    } else {
        for (int p = threadIdx.x; p < items; p += QT) {
            const int r = p / ng, gi = p - r * ng;
            const int j = r0 + r;
            const int kk = gi * g, hi = min(kk + g, K);
            cg[r * ngp + gi] = q4a_group(packed + (size_t)j * pitch, a, kk, hi, sm[(size_t)j * ng + gi]);
        }
    }
    __syncthreads();
    for (int r = threadIdx.x; r < nr; r += QT) out[r0 + r] = lds_seq_sum(cg + r * ngp, ng, 0.0f);
}

// M > 1: one thread per output column j and up to MT token rows.
template <int MT>
__global__ __launch_bounds__(QT) void q4a_gemm_rows(const uint8_t* __restrict__ packed, size_t pitch,
                                                    const uint32_t* __restrict__ sm, int N, int K, int g,
                                                    const float* __restrict__ a, int M, float* __restrict__ out) {
    const int j = blockIdx.x * QT + threadIdx.x;
    const int m0 = blockIdx.y * MT;
    if (j >= N) return;
    const int ng = (K + g - 1) / g;
    const uint8_t* prow = packed + (size_t)j * pitch;
    const uint32_t* srow = sm + (size_t)j * ng;
    float acc[MT], tot[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) tot[m] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += MM_KC) {
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
        for (int kk = k0; kk < min(K, k0 + MM_KC); ++kk) {
            const uint8_t byte = prow[kk >> 1];
            const uint32_t s = srow[kk / g];
            const float w = h2f((uint16_t)(s & 0xffffu)) * (float)((kk & 1) ? (byte >> 4) : (byte & 15)) +
                            h2f((uint16_t)(s >> 16));
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (m0 + m < M) acc[m] = __builtin_fmaf(a[(size_t)(m0 + m) * K + kk], w, acc[m]);
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) tot[m] = tot[m] + acc[m];
    }
#pragma unroll
    for (int m = 0; m < MT; ++m)
        if (m0 + m < M) out[(size_t)(m0 + m) * N + j] = tot[m];
}

// M > 1 with K % 32 == 0, g % 32 == 0 and 16-byte aligned activation rows:
// one thread per (column j, token row blockIdx.y), the packed row read 16
// bytes (32 nibbles) and the token's 32 activations (uniform across the
// workgroup) at a time, one chunk ahead of the chain.  The order per output
// is q4a_gemm_rows' (a.dot's blocks over kk, w = scale * q + min), bit for
// bit.
__global__ __launch_bounds__(QT) void q4a_rows_chain(const uint8_t* __restrict__ packed, size_t pitch,
                                                     const uint32_t* __restrict__ sm, int N, int K, int g,
                                                     const float* __restrict__ a, float* __restrict__ out) {
    const int j = blockIdx.x * QT + threadIdx.x, m = blockIdx.y;
    const int jj = min(j, N - 1);  // clamped: the loads stay unconditional, the store is guarded
    const int nc = K / 32, ng = K / g;
    const uint4* prow = reinterpret_cast<const uint4*>(packed + (size_t)jj * pitch);
    const uint32_t* srow = sm + (size_t)jj * ng;
    const float4* arow = reinterpret_cast<const float4*>(a + (size_t)m * K);
    struct Chunk {
        uint4 w;
        uint32_t s;
        float4 av[8];
    };
    auto ld = [&](Chunk& c, int i) {
        c.w = prow[i];
        c.s = srow[(32 * i) / g];
#pragma unroll
        for (int u = 0; u < 8; ++u) c.av[u] = arow[8 * i + u];
    };
    float acc = 0.0f;
    auto chain = [&](const Chunk& c) {
        const uint32_t ws[4] = {c.w.x, c.w.y, c.w.z, c.w.w};
        const float sc = h2f((uint16_t)(c.s & 0xffffu)), mn = h2f((uint16_t)(c.s >> 16));
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
            const float x[8] = {c.av[2 * c4].x, c.av[2 * c4].y, c.av[2 * c4].z, c.av[2 * c4].w,
                                c.av[2 * c4 + 1].x, c.av[2 * c4 + 1].y, c.av[2 * c4 + 1].z, c.av[2 * c4 + 1].w};
#pragma unroll
            for (int q = 0; q < 8; ++q)
                acc = __builtin_fmaf(x[q], sc * (float)((ws[c4] >> (4 * q)) & 15u) + mn, acc);
        }
    };
    // a.dot's blocks: MM_KC / 32 chunks (an even count) each, folded in
    // where a block starts (an even chunk)
    static_assert(MM_KC % 64 == 0, "blocks start on even chunks");
    float tot = 0.0f;
    auto fold = [&](int i) {
        if (i > 0 && i % (MM_KC / 32) == 0) {
            tot = tot + acc;
            acc = 0.0f;
        }
    };
    Chunk c0, c1;
    ld(c0, 0);
    ld(c1, min(1, nc - 1));
    __builtin_amdgcn_sched_barrier(0);
    int i = 0;
    for (; i + 2 <= nc; i += 2) {
        fold(i);
        chain(c0);
        ld(c0, min(i + 2, nc - 1));
        __builtin_amdgcn_sched_barrier(0);
        chain(c1);
        ld(c1, min(i + 3, nc - 1));
        __builtin_amdgcn_sched_barrier(0);
    }
    if (i < nc) {
        fold(i);
        chain(c0);
    }
    if (j < N) out[(size_t)m * N + j] = tot + acc;
}

}  // namespace

size_t q4a_pitch(size_t k) { return round_up((k + 1) / 2, 16); }

hipError_t launch_q4a(const Weight& w, size_t m, const float* a, float* out, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    if (w.n > (size_t)INT32_MAX || w.k > (size_t)INT32_MAX || m > (size_t)INT32_MAX) return hipErrorInvalidValue;
    const int ng = (int)((w.k + w.g - 1) / w.g);
    if (m == 1) {
        if (ng > 8192) return hipErrorInvalidValue;  // one row's group terms must fit in LDS
        // rows per workgroup: the group terms in <= 32 KB of LDS, and enough
        // workgroups to spread over the CUs
        int rb = (int)std::min<size_t>(64, std::max<size_t>(1, 8192 / (size_t)std::max(ng, 1)));
        while (rb > 8 && (w.n + rb - 1) / rb < 512) rb /= 2;
        const unsigned grid = (unsigned)((w.n + rb - 1) / rb);
        const size_t cgb = (size_t)rb * ((ng + 3) & ~3) * sizeof(float);
        const size_t asb = (w.k / 32) * 36 * sizeof(float);
        const bool vec = w.k % 32 == 0 && (w.g == 32 || w.g == 64) && cgb + asb <= 64 * 1024;
        if (vec && w.g == 32)
            q4a_gemv_kernel<1><<<dim3(grid), dim3(QT), cgb + asb, s>>>(w.q4raw, w.rpitch, w.q4a_sm, (int)w.n,
                                                                      (int)w.k, (int)w.g, rb, a, out);
        else if (vec)
            q4a_gemv_kernel<2><<<dim3(grid), dim3(QT), cgb + asb, s>>>(w.q4raw, w.rpitch, w.q4a_sm, (int)w.n,
                                                                      (int)w.k, (int)w.g, rb, a, out);
        else
            q4a_gemv_kernel<0><<<dim3(grid), dim3(QT), cgb, s>>>(w.q4raw, w.rpitch, w.q4a_sm, (int)w.n, (int)w.k,
                                                                (int)w.g, rb, a, out);
        return hipGetLastError();
    }
    if (w.k % 32 == 0 && w.g % 32 == 0 && ((uintptr_t)a & 15) == 0 && m <= 65535) {
        q4a_rows_chain<<<dim3((unsigned)((w.n + QT - 1) / QT), (unsigned)m), dim3(QT), 0, s>>>(
            w.q4raw, w.rpitch, w.q4a_sm, (int)w.n, (int)w.k, (int)w.g, a, out);
        return hipGetLastError();
    }
    dim3 grid((unsigned)((w.n + QT - 1) / QT), (unsigned)((m + 15) / 16));
    q4a_gemm_rows<16><<<grid, dim3(QT), 0, s>>>(w.q4raw, w.rpitch, w.q4a_sm, (int)w.n, (int)w.k, (int)w.g, a, (int)m,
                                                 out);
    return hipGetLastError();
}

}  // namespace frq
