// gemv_i8.hip — int8 W8A8 GEMV for single-token decode (M == 1), gfx950.
//
// Restates the M==1 arm of Bundle::mm's I8 path
// (/root/reference/src/bundle.rs:744-752):
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
#include "quant_core.h"
// after the HIP runtime (quant_core.h): its memcpy is the device one
#include "libm_f32.h"

#include <algorithm>

namespace frq {

namespace {

__device__ __forceinline__ int dot16(const int4 a, const int4 w, int acc) {
    acc = __builtin_amdgcn_sdot4(a.x, w.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a.y, w.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, w.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, w.w, acc, false);
    return acc;
}

// Sum over aligned runs of LW lanes (LW a power of two <= 64), every lane
// of a run getting it: butterfly exchanges in DPP / permlane (xshfl), no
// LDS round trips.
template <int LW>
__device__ __forceinline__ int lane_sum(int v) {
    if constexpr (LW >= 64) v += (int)xshfl<32>((uint32_t)v);
    if constexpr (LW >= 32) v += (int)xshfl<16>((uint32_t)v);
    if constexpr (LW >= 16) v += (int)xshfl<8>((uint32_t)v);
    if constexpr (LW >= 8) v += (int)xshfl<4>((uint32_t)v);
    if constexpr (LW >= 4) v += (int)xshfl<2>((uint32_t)v);
    if constexpr (LW >= 2) v += (int)xshfl<1>((uint32_t)v);
    return v;
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

// ---------------------------------------------------------------------------
// GEMV v3 (M == 1): persistent grid-stride over groups of RPP = 256/L rows,
// the next group's weight chunks (and its outlier bytes) in flight while the
// current group is reduced.  Outlier correction: lane (q, r4) reads the four
// bytes W[row0+4r4 .. +3, ch_q] as one word of the (K, Np) copy, forms the
// products av_q * w in LDS, and one thread per row adds its t products in
// channel order (-0.0 start) — the oracle's order, so outputs stay bit-exact.
template <int L, int CPL, bool DB>
__global__ __launch_bounds__(256) void gemv3_i8_kernel(
    const int8_t* __restrict__ W, const int8_t* __restrict__ Wkn,
    const float* __restrict__ scale, int N, int Np, int Kp, int t,
    const int8_t* __restrict__ a8, const float* __restrict__ sa,
    const uint32_t* __restrict__ oidx, const float* __restrict__ oval,
    float* __restrict__ out, int32_t* __restrict__ acc_dbg, int n_rg) {
    constexpr int RPP = 256 / L;
    constexpr int NQW = FRQ_T * (RPP / 4);  // outlier words per group
    __shared__ int accs[2][RPP];
    __shared__ float prod[2][RPP][FRQ_T + 1];
    const int tid = threadIdx.x;
    const int sub = tid % L, rloc = tid / L;
    const int nch = Kp >> 4;
    const float sam = sa[0];
    int4 x[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = sub + L * i;
        x[i] = c < nch ? *reinterpret_cast<const int4*>(a8 + 16 * c) : make_int4(0, 0, 0, 0);
    }
    // outlier word this thread fetches each group: channel q, rows 4*r4..
    const int q = tid % FRQ_T, r4 = tid / FRQ_T;
    const bool qw = tid < NQW && q < t;
    const uint32_t chq = qw ? min(oidx[q], (uint32_t)(Kp - 1)) : 0u;
    const float ovq = qw ? oval[q] : 0.0f;

    int rg = blockIdx.x;
    int4 w[CPL], wn[DB ? CPL : 1];
    uint32_t ow = 0, own = 0;
    auto load_group = [&](int g, int4* dst, uint32_t& o) {
        const int8_t* wr = W + (size_t)(g * RPP + rloc) * Kp;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = sub + L * i;
            dst[i] = c < nch ? *reinterpret_cast<const int4*>(wr + 16 * c) : make_int4(0, 0, 0, 0);
        }
        if (qw) o = *reinterpret_cast<const uint32_t*>(Wkn + (size_t)chq * Np + g * RPP + 4 * r4);
    };
    if (rg < n_rg) load_group(rg, w, ow);
    int buf = 0;
    while (rg < n_rg) {
        const int rgn = rg + gridDim.x;
        if (DB && rgn < n_rg) load_group(rgn, wn, own);
        int acc = 0;
#pragma unroll
        for (int i = 0; i < CPL; ++i) acc = dot16(x[i], w[i], acc);
        acc = lane_sum<L>(acc);
        if (sub == 0) accs[buf][rloc] = acc;
        if (qw) {
#pragma unroll
            for (int b = 0; b < 4; ++b)
                prod[buf][4 * r4 + b][q] = ovq * (float)(int8_t)(ow >> (8 * b));
        }
        __syncthreads();
        if (tid < RPP) {
            const int j = rg * RPP + tid;
            if (j < N) {
                float corr = -0.0f;
                for (int qq = 0; qq < t; ++qq) corr = corr + prod[buf][tid][qq];
                const int total = accs[buf][tid];
                out[j] = scale[j] * (sam * (float)total + corr);
                if (acc_dbg) acc_dbg[j] = total;
            }
        }
        buf ^= 1;
        if (DB) {
#pragma unroll
            for (int i = 0; i < CPL; ++i) w[i] = wn[i];
            ow = own;
        } else if (rgn < n_rg) {
            load_group(rgn, w, ow);
        }
        rg = rgn;
    }
}

template <int L, int CPL, bool DB>
hipError_t launch_v3(const Weight& w, const int8_t* a8, const float* sa,
                     const uint32_t* oidx, const float* oval, float* out,
                     int32_t* acc, hipStream_t s) {
    constexpr int RPP = 256 / L;
    const int n_rg = (int)((w.n + RPP - 1) / RPP);  // rows < Np (RPP divides 256)
    const int grid = n_rg < 2048 ? n_rg : 2048;
    const int t = (int)(w.k < FRQ_T ? w.k : FRQ_T);
    gemv3_i8_kernel<L, CPL, DB><<<dim3((unsigned)grid), dim3(256), 0, s>>>(
        w.wt, w.wkn, w.scale, (int)w.n, (int)w.np, (int)w.kp, t, a8, sa, oidx, oval, out, acc, n_rg);
    return hipGetLastError();
}

hipError_t launch_v3_m1(const Weight& w, const int8_t* a8, const float* sa,
                        const uint32_t* oidx, const float* oval, float* out,
                        int32_t* acc, hipStream_t s) {
    const size_t nch = w.kp / 16;
    if (nch <= 64) return launch_v3<8, 8, true>(w, a8, sa, oidx, oval, out, acc, s);
    if (nch <= 128) return launch_v3<64, 2, true>(w, a8, sa, oidx, oval, out, acc, s);
    if (nch <= 256) return launch_v3<64, 4, true>(w, a8, sa, oidx, oval, out, acc, s);
    if (nch <= 512) return launch_v3<64, 8, true>(w, a8, sa, oidx, oval, out, acc, s);
    if (nch <= 1024) return launch_v3<64, 16, false>(w, a8, sa, oidx, oval, out, acc, s);
    if (nch <= 1280) return launch_v3<64, 20, false>(w, a8, sa, oidx, oval, out, acc, s);
    return launch_m<1>(w, a8, sa, oidx, oval, out, acc, s);
}

// ---------------------------------------------------------------------------
// Fused M == 1 linear: activation quant + GEMV v3 in one launch.  Every
// workgroup issues the loads of its first weight row group(s), reads the f32
// activation row (K*4 bytes: L2 hits after the first workgroups) and runs
// quant_core.h's selection and quantisation on it — the routine of the
// standalone quant kernel, so all workgroups hold the same a8 / sa /
// outliers bit for bit without communicating — then streams its row groups
// as gemv3 does.  Workgroup 0 also writes a8 / sa / outliers when asked.
// LDS: the bitmap, then one region that holds the candidate keys, then the
// quantised row, then (with DB) the correction products.  Without DB (long
// rows) the activation chunks are read from the quantised row in LDS at each
// group instead of being held in registers, and the products follow it.
// Group order of the fused linear's grid-stride loop.  Workgroup b runs on
// XCD b % 8 (round-robin dispatch) and visits virtual groups v = b + i*G
// (G % 8 == 0, or a single visit), so v % 8 names the XCD.  The outlier
// gather reads RPP bytes per channel per group from the (K, Np) copy; a
// 128-byte line spans S = 128 / RPP consecutive groups.  Within each chunk
// of 8 S groups, XCD x takes the S consecutive groups x S .. x S + S - 1, so
// every line of the gather is fetched by one XCD, once; the partial chunk
// at the end keeps the identity order.
template <int RPP>
__device__ __forceinline__ int xcd_group(int v, int n_rg) {
    constexpr int S = 128 / RPP, C = 8 * S;
    const int c = v / C, j = v % C;
    return (c + 1) * C <= n_rg ? c * C + (j % 8) * S + j / 8 : v;
}

// bytes of the fused linear's candidate-key / quantised-row region
__host__ __device__ inline size_t lm1_urow(size_t kp) {
    return kp > (size_t)qc::FCAP * 8 ? kp : (size_t)qc::FCAP * 8;
}

constexpr int LM1_ACT_IT = 16;  // groups a workgroup of the ACT form at most

// ACT: the weight is a gated pair whose rows are interleaved in runs of
// RPP/2 (gate columns RPP/2 g .., then the same up columns, in group g:
// gated_rows), and the output is act(gate) * up (N / 2 values); each
// group's row values stay in LDS and after the loop every thread takes some
// (gate, up) pairs (in the loop the activation would delay every group
// behind its barrier).  act: SiLU, x / (1 +
// exp(-x)) (rope.rs:39-41), or, silu == 0, gelu_tanh with constant gc
// (gemma.rs:31-34), the operations of the separate activation kernel.
// (etab: expf's 32-entry table, a copy in LDS: a global table read in the
// epilogue would stall every group behind its barrier)
__device__ __forceinline__ float gated_act(float x, int silu, float gc, const uint64_t* etab) {
    return silu ? x / (1.0f + libm::frq_expf_sel_t(-x, etab))
                : 0.5f * x * (1.0f + libm::frq_tanhf(gc * (x + 0.044715f * x * x * x)));
}

template <int L, int CPL, bool DB, int NV4, int NT, bool ACT = false, bool PB = false>
__global__ __launch_bounds__(NT) void linear_m1_kernel(
    const int8_t* __restrict__ W, const int8_t* __restrict__ Wkn,
    const float* __restrict__ scale, int N, int Np, int Kp, int K,
    const float* __restrict__ A, float* __restrict__ out, int32_t* __restrict__ acc_dbg,
    int8_t* __restrict__ a8o, float* __restrict__ sao, uint32_t* __restrict__ oio,
    float* __restrict__ ovo, int* __restrict__ err, int n_rg, int silu = 1, float gc_act = 0.0f) {
    constexpr int RPP = NT / L, HR = RPP / 2;
    constexpr int LW = L < 64 ? L : 64, WPR = L / LW;  // lanes per wave of a row, waves per row
    constexpr int NQW = FRQ_T * (RPP / 4);  // outlier words per group
    static_assert(NQW <= NT && RPP % 4 == 0, "one outlier word per thread");
    __shared__ qc::RowLdsT<NT> Q;
    __shared__ int accs[2][RPP * WPR];
    // ACT: each visited group's RPP row values (and the group), for the
    // activation after the loop (at most LM1_ACT_IT groups a workgroup)
    __shared__ float actv[ACT ? LM1_ACT_IT * RPP : 1];
    __shared__ int actg[ACT ? LM1_ACT_IT : 1];
    __shared__ uint64_t etab[ACT ? 32 : 1];
    if (ACT && threadIdx.x < 32) etab[threadIdx.x] = libm::kExp2Tab[threadIdx.x];
    int it = 0;
    extern __shared__ __align__(16) unsigned char dyn[];
    const int nbw = Kp >> 5;  // Kp % 128 == 0
    uint32_t* bitmap = reinterpret_cast<uint32_t*>(dyn);
    unsigned char* U = dyn + 4 * nbw;

    const int tid = threadIdx.x;
    const int sub = tid % L, rloc = tid / L;
    const int nch = Kp >> 4, K4 = K >> 2;
    const int G = (int)gridDim.x;
    int rg = blockIdx.x;
    int4 w[CPL], wn[(DB || PB) ? CPL : 1];
    // chunks past the row are clamped, not skipped (no branches between the
    // loads); the activation chunk they meet is zero
    auto load_w = [&](int g, int4* dst) {
        const int8_t* wr = W + (size_t)(g * RPP + rloc) * Kp;
#pragma unroll
        for (int i = 0; i < CPL; ++i) dst[i] = ntload16(wr + 16 * min(sub + L * i, nch - 1));
    };
    // the activation row first (loads retire in issue order), then the
    // weight stream, in flight during the quant
    // (rg < n_rg: the grid is at most n_rg; a workgroup without a second
    // group loads the last one, shared in L2, so that no branch separates
    // these loads from the row's and the quant waits for the row only)
    float4 v[NV4];
    qc::row_load<NV4, NT>(A, K4, v);
    load_w(xcd_group<RPP>(rg, n_rg), w);
    if (DB) load_w(xcd_group<RPP>(min(rg + G, n_rg - 1), n_rg), wn);
    const qc::RowSel s = qc::row_select<NV4, NT>(A, K, v, Q, reinterpret_cast<unsigned long long*>(U),
                                             bitmap, nbw);
    uint32_t* a8w = reinterpret_cast<uint32_t*>(U);  // the candidate keys are dead
    if (s.nan) {
        // the reference panics; the call reports FRQ_ERR_NAN and computes on
        // the standalone quant's placeholders (a8 = 0, sa = 1, zero outliers)
        for (int i4 = tid; i4 < K4; i4 += NT) a8w[i4] = 0u;
    } else {
        qc::row_quantize<NV4, NT>(v, K4, bitmap, s.sa, s.fast, [&](int i4, uint32_t x) { a8w[i4] = x; });
    }
    for (int i4 = K4 + tid; i4 < (Kp >> 2); i4 += NT) a8w[i4] = 0u;
    __syncthreads();
    const float sam = s.sa;
    if (blockIdx.x == 0) {
        if (s.nan && tid == 0) atomicOr(err, 1);
        if (a8o) {
            for (int c = tid; c < nch; c += NT)
                reinterpret_cast<int4*>(a8o)[c] = reinterpret_cast<const int4*>(U)[c];
            if (tid < FRQ_T) { oio[tid] = Q.sel_i[tid]; ovo[tid] = Q.sel_v[tid]; }
            if (tid == 0) sao[0] = sam;
        }
    }
    const int4* xs = reinterpret_cast<const int4*>(U);
    int4 x[DB ? CPL : 1];
    if (DB) {
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = sub + L * i;
            x[i] = c < nch ? xs[c] : make_int4(0, 0, 0, 0);
        }
    }
    // outlier word this thread fetches each group: channel q, rows 4*r4..
    const int q = tid % FRQ_T, r4 = tid / FRQ_T;
    const bool qw = tid < NQW;
    const uint32_t chq = qw ? min(Q.sel_i[q], (uint32_t)(Kp - 1)) : 0u;
    const float ovq = qw ? Q.sel_v[q] : 0.0f;
    if (DB) __syncthreads();  // U holds the correction products from here on
    float (*prod)[RPP][FRQ_T + 1] = reinterpret_cast<float (*)[RPP][FRQ_T + 1]>(
        DB ? U : U + lm1_urow(Kp));
    auto load_o = [&](int g) -> uint32_t {
        return qw ? *reinterpret_cast<const uint32_t*>(Wkn + (size_t)chq * Np + g * RPP + 4 * r4) : 0u;
    };
    // the epilogue thread's scale comes with its group's loads (a dependent
    // load in the epilogue would stall every group behind the barrier)
    auto load_s = [&](int g) -> float { return tid < RPP ? scale[g * RPP + tid] : 0.0f; };
    int gc = xcd_group<RPP>(rg, n_rg);  // rg < n_rg: the grid is at most n_rg
    uint32_t ow = load_o(gc), own = 0;
    float sc = load_s(gc), scn = 0.0f;
    if ((DB || PB) && rg + G < n_rg) {
        const int g1 = xcd_group<RPP>(rg + G, n_rg);
        // PB: the second group goes out once the selection has freed its
        // registers (both groups in flight through the stream)
        if (PB) load_w(g1, wn);
        own = load_o(g1);
        scn = load_s(g1);
    }
    int buf = 0;
    bool first = true;
    while (rg < n_rg) {
        const int rgn = rg + G;
        const int gn = rgn < n_rg ? xcd_group<RPP>(rgn, n_rg) : 0;
        if ((DB || PB) && !first && rgn < n_rg) {
            load_w(gn, wn);
            own = load_o(gn);
            scn = load_s(gn);
        }
        first = false;
        int acc = 0;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = sub + L * i;
            acc = dot16(DB ? x[i] : (c < nch ? xs[c] : make_int4(0, 0, 0, 0)), w[i], acc);
        }
        // single-buffered: the next group's weights go out as soon as the dot
        // has consumed these, overlapping the reduction and the epilogue
        if (!DB && !PB && rgn < n_rg) load_w(gn, w);
        acc = lane_sum<LW>(acc);
        if (sub % LW == 0) accs[buf][rloc * WPR + sub / LW] = acc;
        if (qw) {
#pragma unroll
            for (int b = 0; b < 4; ++b) prod[buf][4 * r4 + b][q] = ovq * (float)(int8_t)(ow >> (8 * b));
        }
        if (!DB && !PB && rgn < n_rg) {
            own = load_o(gn);
            scn = load_s(gn);
        }
        __syncthreads();
        if constexpr (ACT) {
            if (tid < RPP) {  // the group's RPP row values, kept for after the loop
                float corr = -0.0f;
#pragma unroll
                for (int qq = 0; qq < FRQ_T; ++qq) corr = corr + prod[buf][tid][qq];
                int total = accs[buf][tid * WPR];
#pragma unroll
                for (int h = 1; h < WPR; ++h) total += accs[buf][tid * WPR + h];
                actv[it * RPP + tid] = sc * (sam * (float)total + corr);
                if (tid == 0) actg[it] = gc;
            }
            ++it;
        } else if (tid < RPP) {
            const int j = gc * RPP + tid;
            if (j < N) {
                float corr = -0.0f;
#pragma unroll
                for (int qq = 0; qq < FRQ_T; ++qq) corr = corr + prod[buf][tid][qq];
                int total = accs[buf][tid * WPR];
#pragma unroll
                for (int h = 1; h < WPR; ++h) total += accs[buf][tid * WPR + h];
                out[j] = sc * (sam * (float)total + corr);
                if (acc_dbg) acc_dbg[j] = total;
            }
        }
        buf ^= 1;
        if (DB || PB) {
#pragma unroll
            for (int i = 0; i < CPL; ++i) w[i] = wn[i];
        }
        ow = own;
        sc = scn;
        gc = gn;
        rg = rgn;
    }
    if constexpr (ACT) {  // out = act(gate) * up for every kept group, all threads at once
        __syncthreads();
        for (int x = tid; x < it * HR; x += NT) {
            const int i = x / HR, r = x - i * HR;
            out[HR * actg[i] + r] = gated_act(actv[i * RPP + r], silu, gc_act, etab) * actv[i * RPP + HR + r];
        }
    }
}

template <int L, int CPL, bool DB, int NV4, int NT = 256, bool ACT = false, bool PB = false>
hipError_t launch_lm1(const Weight& w, const float* a, float* out, int32_t* acc, int8_t* a8o,
                      float* sao, uint32_t* oio, float* ovo, int* err, int gmax, hipStream_t s, int silu = 1,
                      float gc = 0.0f) {
    constexpr int RPP = NT / L;
    const int n_rg = (int)((w.n + RPP - 1) / RPP);  // rows < Np (RPP divides 256)
    int grid = n_rg < gmax ? n_rg : gmax;
    if (ACT && (n_rg + grid - 1) / grid > LM1_ACT_IT) grid = (n_rg + LM1_ACT_IT - 1) / LM1_ACT_IT;
    const size_t prod = (size_t)2 * RPP * (FRQ_T + 1) * 4;
    const size_t lds = w.kp / 8 + (DB ? std::max(lm1_urow(w.kp), prod) : lm1_urow(w.kp) + prod);
    linear_m1_kernel<L, CPL, DB, NV4, NT, ACT, PB><<<dim3((unsigned)grid), dim3(NT), lds, s>>>(
        w.wt, w.wkn, w.scale, (int)w.n, (int)w.np, (int)w.kp, (int)w.k, a, out, acc, a8o, sao, oio,
        ovo, err, n_rg, silu, gc);
    return hipGetLastError();
}

// The two launches lm1_dispatch makes: the plain fused linear and the one
// with the gated activation in its epilogue.
struct Lm1Call {
    const Weight& w; const float* a; float* out; int32_t* acc; int8_t* a8o; float* sao; uint32_t* oio;
    float* ovo; int* err; hipStream_t s;
    template <int L, int CPL, bool DB, int NV4, int NT>
    hipError_t operator()(int g) const {
        return launch_lm1<L, CPL, DB, NV4, NT, false, !DB>(w, a, out, acc, a8o, sao, oio, ovo, err, g, s);
    }
};
struct Lm1ActCall {
    const Weight& w; const float* a; float* out; int silu; float gc; int* err; hipStream_t s;
    template <int L, int CPL, bool DB, int NV4, int NT>
    hipError_t operator()(int g) const {
        return launch_lm1<L, CPL, DB, NV4, NT, true, !DB>(w, a, out, nullptr, nullptr, nullptr, nullptr, nullptr, err,
                                                          g, s, silu, gc);
    }
};

// The fused linear's configuration for a row of nch 16-byte chunks and N
// outputs, as a call of f<L, CPL, DB, NV4, NT>(gmax default).
template <typename F>
hipError_t lm1_dispatch(const Weight& w, int g, F f) {
    const size_t nch = w.kp / 16;
    // grid caps: about the workgroups resident at once (256 CUs times the
    // occupancy each variant's registers allow), measured best on MI355X
    // short rows: 8 lanes a row (32-row groups) when N is large, 16 lanes
    // (16-row groups: twice the groups, a shorter quant-bound tail) below
    if (nch <= 64 && w.n >= 65536) return f.template operator()<8, 8, true, 1, 256>(g ? g : 768);
    if (nch <= 64) return f.template operator()<16, 4, true, 1, 256>(g ? g : 768);
    if (nch <= 128) return f.template operator()<64, 2, true, 2, 256>(g ? g : 1024);
    // rows of 2049..4096 bytes: one 512-thread workgroup a CU (8-row groups,
    // two in flight during the quant; the quant once a CU, half the
    // elements a thread), two a CU for long outputs (N >= 12288: gate|up);
    // measured against two / four 256-thread workgroups a CU: o 9.64 ->
    // 8.3 us, q|k|v 9.78 -> 9.56, gate|up 27.3 -> 26.0 (configs[4] shapes);
    // the two-a-CU threshold: K 4096 N 14336 16.2 -> 15.2 us, K 3584 N
    // 12288 14.5 -> 14.2, but N 8192 11.5 -> 12.5
    if (nch <= 256) return f.template operator()<64, 4, true, 2, 512>(g ? g : (w.n >= 12288 ? 512 : 256));
    if (nch <= 512) return f.template operator()<64, 8, true, 8, 256>(g ? g : 512);
    // long rows: 1024 threads (a quarter of the quant per thread), every
    // workgroup's first group in flight during the quant
    // (256 lanes, four waves, per row: 4 rows per group, at most 5 chunks a
    // lane — 110 VGPRs with the second buffer issued after the quant; 128
    // lanes with 10 chunks spilled to scratch)
    if (nch <= 1024) return f.template operator()<256, 4, false, 4, 1024>(g ? g : 256);
    return f.template operator()<256, 5, false, 5, 1024>(g ? g : 256);
}

}  // namespace

hipError_t launch_gemv_i8(const Weight& w, size_t m, const int8_t* a8,
                          const float* sa, const uint32_t* oidx,
                          const float* oval, float* out, int32_t* acc,
                          hipStream_t s) {
    // rows j >= N read zero padding of the (Np, Kp) weight and are not stored
    if ((size_t)m * w.kp > 64 * 1024) return hipErrorInvalidValue;
    if (m != 1) return hipErrorInvalidValue;
    return launch_v3_m1(w, a8, sa, oidx, oval, out, acc, s);
}

bool linear_m1_ok(const Weight& w, const float* a) {
    return w.k > FRQ_T && w.k % 4 == 0 && ((uintptr_t)a & 15) == 0 && w.kp / 16 <= 1280;
}

hipError_t launch_linear_m1(const Weight& w, const float* a, float* out, int32_t* acc,
                            int8_t* a8o, float* sao, uint32_t* oio, float* ovo, int* err,
                            hipStream_t s, int gmax) {
    if (!linear_m1_ok(w, a)) return hipErrorInvalidValue;
    return lm1_dispatch(w, gmax, Lm1Call{w, a, out, acc, a8o, sao, oio, ovo, err, s});
}

int linear_m1_rpp(size_t kp, size_t n) {
    const size_t nch = kp / 16;  // as lm1_dispatch: NT / L
    return nch <= 64 ? (n >= 65536 ? 32 : 16) : nch <= 128 ? 4 : nch <= 256 ? 8 : 4;
}

bool linear_m1_act_ok(const Weight& w, const float* a, int hr) {
    // whole groups of hr gate and hr up rows, hr the dispatch's RPP / 2
    return linear_m1_ok(w, a) && hr > 0 && 2 * hr == linear_m1_rpp(w.kp, w.n) && w.n % (2 * (size_t)hr) == 0;
}

hipError_t launch_linear_m1_act(const Weight& w, const float* a, float* out, int hr, int silu, float gc, int* err,
                                hipStream_t s) {
    if (!linear_m1_act_ok(w, a, hr)) return hipErrorInvalidValue;
    return lm1_dispatch(w, 0, Lm1ActCall{w, a, out, silu, gc, err, s});
}

}  // namespace frq
