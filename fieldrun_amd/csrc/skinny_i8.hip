// skinny_i8.hip — int8 W8A8 linear for decode batches (2 <= M <= 16), gfx950.
//
// Restates the M > 1 arm of Bundle::mm's I8 path on pre-quantised rows
// (/root/reference/src/bundle.rs:709-715): acc = i8dot(a8[i], wt[j]) in i32,
// corr = sum over row i's outliers of av * (wt[j, ch] as f32) in ascending
// channel order from -0.0, out = scale[j] * (sa[i] * acc + corr) (separate
// mul / add).  Every output is bit-exact to that order.
//
// HBM-bound: the weights stream once.  A workgroup owns CB blocks of 16
// output rows (16 CB weight rows) over all of K; its KS waves split the
// k-blocks.  Per k-block a wave issues one A operand (the M <= 16 token rows
// of a8, 64 bytes each, L2-resident and shared by every workgroup) and CB B
// operands from the blocked weight copy wblk (each a contiguous 1 KB wave
// load), and CB v_mfma_i32_16x16x64_i8: C[token][weight row].  The waves'
// int32 partials are added through LDS (exact in any order).  The outlier
// correction runs on VALU in the reference's order: the 16-byte runs
// W[j0 .. j0 + 16 CB), ch] of the (K, Np) copy for the rows' 32 outlier
// channels are loaded at the start (they do not depend on the dot) and wait
// in registers until the epilogue.
#include "frq_internal.h"

namespace frq {

namespace {

template <int CB, int KS>
__global__ __launch_bounds__(64 * KS) void skinny_i8_kernel(
    const int8_t* __restrict__ Wb, const int8_t* __restrict__ Wkn, const float* __restrict__ scale,
    int N, int Np, int Kp, const int8_t* __restrict__ a8, int M, const float* __restrict__ sa,
    const uint32_t* __restrict__ oidx, const float* __restrict__ oval, int t,
    float* __restrict__ out, int32_t* __restrict__ acc_dbg) {
    constexpr int NT = 64 * KS, TC = 16 * CB;  // threads, tile columns (weight rows)
    __shared__ v4i red[KS - 1][CB][64];
    __shared__ int tot[16][TC + 1];
    __shared__ __attribute__((aligned(16))) int8_t gat[16 * FRQ_T][TC];  // W[j0 + c, ch(i, q)]
    __shared__ float ovs[16][FRQ_T];

    const int tid = threadIdx.x, lane = tid & 63;
    const int ks = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int jb0 = blockIdx.x * CB, j0 = jb0 * 16;
    // outlier gathers first: pair p = (row i, outlier q), TC bytes each
    constexpr int PPT = (16 * FRQ_T + NT - 1) / NT;  // pairs per thread
    v4i gv[PPT][CB];
    float ovv[PPT];
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
        const int pr = tid + NT * u, i = pr / FRQ_T, q = pr % FRQ_T;
        const bool ok = pr < 16 * FRQ_T && i < M && q < t;
        const uint32_t ch = ok ? min(oidx[(size_t)i * FRQ_T + q], (uint32_t)(Kp - 1)) : 0u;
        ovv[u] = ok ? oval[(size_t)i * FRQ_T + q] : 0.0f;
#pragma unroll
        for (int c = 0; c < CB; ++c)
            gv[u][c] = ok ? *reinterpret_cast<const v4i*>(Wkn + (size_t)ch * Np + j0 + 16 * c)
                          : v4i{0, 0, 0, 0};
    }
    // main loop: lane 16g + r reads token row r (zero past M), k-bytes 16g..
    const int nkb = Kp / 64;
    const int kb0 = nkb * ks / KS, kb1 = nkb * (ks + 1) / KS;
    const int r = lane & 15, g = lane >> 4;
    const bool arow = r < M;
    const int8_t* ap = a8 + (size_t)(arow ? r : 0) * Kp + 16 * g;
    const int8_t* wp = Wb + (size_t)jb0 * 1024 + lane * 16;
    const size_t kstride = (size_t)(Np / 16) * 1024;
    v4i acc[CB];
#pragma unroll
    for (int c = 0; c < CB; ++c) acc[c] = v4i{0, 0, 0, 0};
    constexpr int U = 4;
    for (int kb = kb0; kb < kb1; kb += U) {
        v4i av[U], bv[U][CB];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool in = kb + u < kb1;
            av[u] = (in && arow) ? *reinterpret_cast<const v4i*>(ap + (size_t)(kb + u) * 64) : v4i{0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c < CB; ++c)
                bv[u][c] = in ? ntload_v4i(wp + (size_t)(kb + u) * kstride + (size_t)c * 1024) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < CB; ++c)
                acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[u], bv[u][c], acc[c], 0, 0, 0);
    }
    if (ks > 0) {
#pragma unroll
        for (int c = 0; c < CB; ++c) red[ks - 1][c][lane] = acc[c];
    }
    // the gathered bytes and outlier values to LDS
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
        const int pr = tid + NT * u;
        if (pr < 16 * FRQ_T) {
#pragma unroll
            for (int c = 0; c < CB; ++c) *reinterpret_cast<v4i*>(&gat[pr][16 * c]) = gv[u][c];
            ovs[pr / FRQ_T][pr % FRQ_T] = ovv[u];
        }
    }
    __syncthreads();
    if (ks == 0) {
#pragma unroll
        for (int w = 0; w < KS - 1; ++w)
#pragma unroll
            for (int c = 0; c < CB; ++c) acc[c] += red[w][c][lane];
        // C lane l: tokens 4 (l / 16) + e, weight row l % 16
#pragma unroll
        for (int c = 0; c < CB; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) tot[4 * (lane >> 4) + e][16 * c + (lane & 15)] = acc[c][e];
    }
    __syncthreads();
    // epilogue: one thread per (token, column), the reference's order
    for (int o = tid; o < M * TC; o += NT) {
        const int i = o / TC, cl = o % TC, j = j0 + cl;
        if (j >= N) continue;
        const int total = tot[i][cl];
        float corr = -0.0f;
        for (int q = 0; q < t; ++q) corr = corr + ovs[i][q] * (float)gat[i * FRQ_T + q][cl];
        out[(size_t)i * N + j] = scale[j] * (sa[i] * (float)total + corr);
        if (acc_dbg) acc_dbg[(size_t)i * N + j] = total;
    }
}

template <int CB, int KS>
hipError_t launch_s(const Weight& w, size_t m, const int8_t* a8, const float* sa,
                    const uint32_t* oidx, const float* oval, float* out, int32_t* acc, hipStream_t s) {
    const unsigned grid = (unsigned)(w.np / (16 * CB));
    const int t = (int)(w.k < FRQ_T ? w.k : FRQ_T);
    skinny_i8_kernel<CB, KS><<<dim3(grid), dim3(64 * KS), 0, s>>>(
        w.wblk, w.wkn, w.scale, (int)w.n, (int)w.np, (int)w.kp, a8, (int)m, sa, oidx, oval, t, out, acc);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_skinny_i8(const Weight& w, size_t m, const int8_t* a8, const float* sa,
                            const uint32_t* oidx, const float* oval, float* out, int32_t* acc,
                            hipStream_t s) {
    // a8: m rows of pitch Kp; wblk / wkn padded to Np (a multiple of 256)
    if (m < 1 || m > 16 || !w.wblk || w.kp % 64) return hipErrorInvalidValue;
    // enough workgroups to fill the chip: two column blocks per workgroup
    // when N is large, and the k-blocks split over more waves when K is long
    const size_t blocks = w.np / 16;
    if (w.kp > 8192) return launch_s<1, 8>(w, m, a8, sa, oidx, oval, out, acc, s);
    if (blocks >= 2048) return launch_s<2, 4>(w, m, a8, sa, oidx, oval, out, acc, s);
    return launch_s<1, 4>(w, m, a8, sa, oidx, oval, out, acc, s);
}

}  // namespace frq
