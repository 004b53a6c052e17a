// gemm_i8.hip — int8 W8A8 GEMM on CDNA4 MFMA for prefill / batched shapes
// (M > 4), gfx950.
//
// Same arithmetic as Bundle::mm's I8 arm (/root/reference/src/bundle.rs:
// 688-724):  out[i,j] = scale[j] * (sa[i] * (acc[i,j] as f32) + corr[i,j]),
// acc = i8dot(a8[i], wt[j]) in i32 (bit-exact), corr = sum over row i's
// outliers of av * wt[j,ch].
//
// acc: LDS-tiled v_mfma_i32_16x16x64_i8 over a8 (Mp,Kp) x wt (Np,Kp), both
// K-contiguous.  128x256 output tile per 256-thread workgroup, 2x2 waves of
// 64x128 (4x8 MFMA blocks), k-step 64; operands go HBM -> LDS directly
// (global_load_lds, no register staging) through a 3-stage ring with one
// barrier per k-step, and the tile order is XCD-aware (tile_of below).
//
// corr: 32 VALU multiply-adds per output would cost as much as the whole
// MFMA GEMM, so corr also runs on the int8 MFMA.  For each 128-row M tile
// the union U of its rows' outlier channels is formed (sorted) and each
// outlier value is written as X = round(av / so[i]), |X| <= 127*2^16, with
// so[i] = max|av| / (127*2^16), split into three signed int8 digits
// X = d2*2^16 + d1*2^8 + d0.  Then C_d = D_d (BM x |U|) . W[:, U]^T is an
// exact int32 MFMA GEMM per digit and corr = so * ((C2*256 + C1)*256 + C0).
// W[:, U] is staged from the (K, Np) row-major copy of the weight (wkn), one
// 128-byte row per channel, transposed into LDS.  The 24-bit split makes
// corr differ from the reference's f32 sum by ~1e-7 relative; acc stays
// bit-exact.  Rows with a non-finite outlier take the exact sequential
// corr in the epilogue instead.
#include "frq_internal.h"

namespace frq {

namespace {

constexpr int BM = 128, BK = 128;   // union tile rows; union padding unit
constexpr int UMAX = BM * FRQ_T;     // max union size per M tile
constexpr float XMAX = 8323072.0f;   // 127 * 2^16

struct UnionView {
    int32_t* nu;     // [tiles]
    uint32_t* u;     // [tiles][UMAX]
    float* so;       // [Mp]
    int32_t* fin;    // [Mp] 1 = non-finite outlier in row
    int8_t* d;       // [tiles][3][BM][UMAX]
};

__host__ __device__ inline UnionView union_view(void* base, size_t m) {
    const size_t tiles = (m + BM - 1) / BM, mp = tiles * BM;
    char* p = (char*)base;
    UnionView v;
    v.nu = (int32_t*)p; p += round_up(tiles * 4, 256);
    v.u = (uint32_t*)p; p += round_up(tiles * UMAX * 4, 256);
    v.so = (float*)p; p += round_up(mp * 4, 256);
    v.fin = (int32_t*)p; p += round_up(mp * 4, 256);
    v.d = (int8_t*)p;
    return v;
}

// ---- union of outlier channels + digit split, one workgroup per M tile --
__global__ __launch_bounds__(256) void union_kernel(
    const uint32_t* __restrict__ oidx, const float* __restrict__ oval, int M,
    int K, int t, UnionView uv) {
    extern __shared__ uint32_t sm[];
    const int nw = (K + 31) / 32;
    uint32_t* bitmap = sm;           // nw words
    uint32_t* wpre = sm + nw;        // nw words: popcount prefix
    __shared__ uint32_t scan_lds[5];

    const int tile = blockIdx.x, tid = threadIdx.x;
    const int r0 = tile * BM, nrows = min(BM, M - r0);
    for (int w = tid; w < nw; w += 256) bitmap[w] = 0u;
    __syncthreads();
    for (int i = tid; i < nrows * t; i += 256) {
        const uint32_t c = oidx[(size_t)(r0 + i / t) * FRQ_T + i % t];
        if (c < (uint32_t)K) atomicOr(&bitmap[c >> 5], 1u << (c & 31));
    }
    __syncthreads();
    // prefix popcount over words (contiguous chunk per thread)
    const int C = (nw + 255) / 256;
    const int lo = tid * C, hi = min(lo + C, nw);
    uint32_t cnt = 0;
    for (int w = lo; w < hi; ++w) cnt += __popc(bitmap[w]);
    const int lane = tid & 63, wave = tid >> 6;
    uint32_t incl = cnt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        uint32_t y = __shfl_up(incl, off, 64);
        if (lane >= off) incl += y;
    }
    if (lane == 63) scan_lds[wave] = incl;
    __syncthreads();
    if (tid == 0) {
        uint32_t run = 0;
        for (int w = 0; w < 4; ++w) { uint32_t c = scan_lds[w]; scan_lds[w] = run; run += c; }
        scan_lds[4] = run;
    }
    __syncthreads();
    uint32_t base = scan_lds[wave] + incl - cnt;
    const uint32_t nu = scan_lds[4];
    uint32_t* U = uv.u + (size_t)tile * UMAX;
    for (int w = lo; w < hi; ++w) {
        wpre[w] = base;
        uint32_t bits = bitmap[w];
        while (bits) {
            const int b = __ffs(bits) - 1;
            bits &= bits - 1;
            U[base++] = (uint32_t)(w * 32 + b);
        }
    }
    const uint32_t nup = (nu + BK - 1) / BK * BK;
    for (uint32_t u = nu + tid; u < nup; u += 256) U[u] = 0u;  // digits are 0 there
    if (tid == 0) uv.nu[tile] = (int32_t)nu;
    __syncthreads();
    // one thread per row: scale, flag and its three digit rows
    if (tid < BM) {
        const int row = r0 + tid;
        float mx = 0.0f;
        int fin = 0;
        if (tid < nrows)
            for (int q = 0; q < t; ++q) {
                const float v = oval[(size_t)row * FRQ_T + q];
                fin |= !(fabsf(v) <= 3.0e38f);
                mx = fmaxf(mx, fabsf(v));
            }
        float so = mx > 0.0f ? mx / XMAX : 1.0f;
        if (!(so >= 1.0e-30f) || !(so <= 1.0e30f)) fin = 1;  // keep digits exact
        if (fin) so = 1.0f;
        uv.so[row] = so;
        uv.fin[row] = fin;
        int q = 0;
        for (uint32_t ch = 0; ch < nup; ch += 16) {
            uint32_t v0[4] = {0, 0, 0, 0}, v1[4] = {0, 0, 0, 0}, v2[4] = {0, 0, 0, 0};
            while (!fin && tid < nrows && q < t) {
                const uint32_t c = min(oidx[(size_t)row * FRQ_T + q], (uint32_t)(K - 1));
                const uint32_t pos = wpre[c >> 5] + __popc(bitmap[c >> 5] & ((1u << (c & 31)) - 1u));
                if (pos >= ch + 16) break;
                float xf = rintf(oval[(size_t)row * FRQ_T + q] / so);
                xf = fminf(fmaxf(xf, -XMAX), XMAX);
                const int X = (int)xf;
                const int d0 = (int)(int8_t)(X & 0xFF);
                const int X1 = (X - d0) >> 8;
                const int d1 = (int)(int8_t)(X1 & 0xFF);
                const int d2 = (X1 - d1) >> 8;
                const int byte = (int)(pos - ch), wd = byte >> 2, sh = (byte & 3) * 8;
                v0[wd] |= (uint32_t)(d0 & 0xFF) << sh;
                v1[wd] |= (uint32_t)(d1 & 0xFF) << sh;
                v2[wd] |= (uint32_t)(d2 & 0xFF) << sh;
                ++q;
            }
            int8_t* drow = uv.d + ((size_t)tile * 3 * BM + tid) * UMAX + ch;
            *reinterpret_cast<uint4*>(drow) = make_uint4(v0[0], v0[1], v0[2], v0[3]);
            *reinterpret_cast<uint4*>(drow + (size_t)BM * UMAX) = make_uint4(v1[0], v1[1], v1[2], v1[3]);
            *reinterpret_cast<uint4*>(drow + (size_t)2 * BM * UMAX) = make_uint4(v2[0], v2[1], v2[2], v2[3]);
        }
    }
}

// ---- the GEMM -------------------------------------------------------------
// 128 x 256 output tile per 256-thread workgroup; waves 2 (M) x 2 (N), each
// 64 x 128 = 4 x 8 blocks of v_mfma_i32_16x16x64_i8.  k-step 64; a ring of
// NST stages in LDS filled by global_load_lds_dwordx4, each 1 KB LDS block
// holding one 16-row x 64-byte MFMA operand in lane order (lane l = 16*g + r
// -> row r, bytes 16g..16g+15), so every operand fetch is one conflict-free
// ds_read_b128 at block*1024 + lane*16.
constexpr int GBM = 128, GBN = 256, GBK = 64, NST = 3;
constexpr int ABLK = GBM / 16, BBLK = GBN / 16, SBLK = ABLK + BBLK;  // 8 + 16 blocks
constexpr int STAGE = SBLK * 1024;                                   // 24 KB

typedef __attribute__((address_space(1))) void gvoid_t;
typedef __attribute__((address_space(3))) void lvoid_t;

__device__ __forceinline__ void dma16(const void* g, void* lds_base) {
    __builtin_amdgcn_global_load_lds((gvoid_t*)g, (lvoid_t*)lds_base, 16, 0, 0);
}

// s_waitcnt vmcnt(n) (gfx9 encoding; expcnt / lgkmcnt not waited on)
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

__device__ __forceinline__ v4i mfma(const v4i a, const v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Issue this wave's 6 block loads of k-step ks into LDS stage buffer `st`.
__device__ __forceinline__ void issue_stage(const int8_t* __restrict__ A, const int8_t* __restrict__ W,
                                            int Kp, int m0, int n0, int ks, int8_t* st) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const size_t k0 = (size_t)ks * GBK + g * 16;
#pragma unroll
    for (int i = 0; i < SBLK / 4; ++i) {
        const int t = wave + 4 * i;
        const int8_t* src = t < ABLK ? A + (size_t)(m0 + 16 * t + r) * Kp + k0
                                     : W + (size_t)(n0 + 16 * (t - ABLK) + r) * Kp + k0;
        dma16(src, st + t * 1024);
    }
}

// Bijective XCD-aware tile order: workgroups on the same XCD (id % 8) take a
// contiguous run of tiles ordered N-tile major, M-tile minor, so the A
// panel is shared in that XCD's L2 and each weight panel is read once.
__device__ __forceinline__ void tile_of(int b, int G, int MT, int& mt, int& nt) {
    const int x = b & 7, j = b >> 3;
    const int q = G >> 3, rem = G & 7;
    const int start = x * q + min(x, rem);
    const int tau = start + j;
    nt = tau / MT;
    mt = tau % MT;
}

__global__ __launch_bounds__(256) void gemm_i8_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ W,
    const int8_t* __restrict__ Wkn, const float* __restrict__ scale,
    const float* __restrict__ sa, int M, int N, int Np, int Kp, int t,
    UnionView uv, const uint32_t* __restrict__ oidx,
    const float* __restrict__ oval, float* __restrict__ out,
    int32_t* __restrict__ acc_dbg, int MT) {
    __shared__ __attribute__((aligned(1024))) int8_t lds[NST * STAGE];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    int mt, nt;
    tile_of(blockIdx.x, gridDim.x, MT, mt, nt);
    const int m0 = mt * GBM, n0 = nt * GBN;
    const int S = Kp / GBK;

    v4i acc[4][8];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 8; ++b) acc[a][b] = v4i{0, 0, 0, 0};

    issue_stage(A, W, Kp, m0, n0, 0, lds);
    if (S > 1) issue_stage(A, W, Kp, m0, n0, 1, lds + STAGE);
    for (int s = 0; s < S; ++s) {
        if (s + 1 < S) wait_vm<SBLK / 4>(); else wait_vm<0>();
        __syncthreads();
        if (s + 2 < S) issue_stage(A, W, Kp, m0, n0, s + 2, lds + ((s + 2) % NST) * STAGE);
        const int8_t* st = lds + (s % NST) * STAGE;
        v4i af[4], bf[8];
#pragma unroll
        for (int bm = 0; bm < 4; ++bm)
            af[bm] = *reinterpret_cast<const v4i*>(st + (wm * 4 + bm) * 1024 + lane * 16);
#pragma unroll
        for (int bn = 0; bn < 8; ++bn)
            bf[bn] = *reinterpret_cast<const v4i*>(st + (ABLK + wn * 8 + bn) * 1024 + lane * 16);
#pragma unroll
        for (int bm = 0; bm < 4; ++bm)
#pragma unroll
            for (int bn = 0; bn < 8; ++bn) acc[bm][bn] = mfma(af[bm], bf[bn], acc[bm][bn]);
    }

    // ---- epilogue, one 32-column sub-tile (2 MFMA blocks) at a time:
    // t = sa * acc, plus the outlier correction so * C from three int8 digit
    // MFMAs over the tile's channel union, then out = scale * t.  Lane holds
    // rows 4*(lane/16)+c and column lane%16 of each 16x16 block.
    // per-row sa, so and the non-finite flag of the tile, in the last stage
    // buffer (free in the epilogue)
    float* meta = reinterpret_cast<float*>(lds + 2 * STAGE + 16 * 1024);
    __syncthreads();
    if (threadIdx.x < GBM) {
        const int i = min(m0 + (int)threadIdx.x, M - 1);
        meta[threadIdx.x] = sa[i];
        meta[GBM + threadIdx.x] = uv.fin[i] ? 0.0f : uv.so[i];
        meta[2 * GBM + threadIdx.x] = uv.fin[i] ? 1.0f : 0.0f;
    }
    const int nu = uv.nu[mt];
    const uint32_t* U = uv.u + (size_t)mt * UMAX;
    const int r = lane & 15, g = lane >> 4;
    int8_t* bt = lds + 24 * 1024;
    // stage digit chunk u0 (3 x 8 DMA blocks) and W[:, U[u0..u0+63]]^T (16 blocks)
    __syncthreads();
    auto stage_chunk = [&](int u0) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 6; ++i) {
            const int tb = wave + 4 * i;  // digit tb/8, row block tb%8
            const int8_t* src = uv.d + (((size_t)mt * 3 + tb / 8) * BM + 16 * (tb % 8) + r) * UMAX + u0 + g * 16;
            dma16(src, lds + tb * 1024);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = threadIdx.x + 256 * i;  // 64 channels x 16 chunks of 16 columns
            const int uu = idx >> 4, cch = idx & 15;
            const v4i w = *reinterpret_cast<const v4i*>(Wkn + (size_t)U[u0 + uu] * Np + n0 + cch * 16);
#pragma unroll
            for (int b = 0; b < 16; ++b)
                bt[cch * 1024 + ((uu >> 4) * 16 + b) * 16 + (uu & 15)] = (int8_t)((uint32_t)w[b >> 2] >> ((b & 3) * 8));
        }
        wait_vm<0>();
        __syncthreads();
    };
    const bool one_chunk = nu <= GBK;
    if (nu > 0 && one_chunk) stage_chunk(0);
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
        float tv[4][2][4];
#pragma unroll
        for (int bm = 0; bm < 4; ++bm)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int rl = wm * 64 + bm * 16 + (lane >> 4) * 4 + c;
                const float sai = meta[rl];
#pragma unroll
                for (int x = 0; x < 2; ++x) {
                    const int av = acc[bm][sub * 2 + x][c];
                    if (acc_dbg) {
                        const int i = m0 + rl;
                        const int j = n0 + wn * 128 + (sub * 2 + x) * 16 + (lane & 15);
                        if (i < M && j < N) acc_dbg[(size_t)i * N + j] = av;
                    }
                    tv[bm][x][c] = sai * (float)av;
                }
            }
        for (int u0 = 0; u0 < nu; u0 += GBK) {
            if (!one_chunk) stage_chunk(u0);
            v4i bf2[2];
#pragma unroll
            for (int x = 0; x < 2; ++x)
                bf2[x] = *reinterpret_cast<const v4i*>(bt + (wn * 8 + sub * 2 + x) * 1024 + lane * 16);
            // tv += so * (C2 * 2^16 + C1 * 2^8 + C0); so is 0 on non-finite rows
#pragma unroll
            for (int d = 2; d >= 0; --d) {
                const float wd = d == 2 ? 65536.0f : (d == 1 ? 256.0f : 1.0f);
#pragma unroll
                for (int bm = 0; bm < 4; ++bm) {
                    const v4i af = *reinterpret_cast<const v4i*>(lds + (d * 8 + wm * 4 + bm) * 1024 + lane * 16);
#pragma unroll
                    for (int x = 0; x < 2; ++x) {
                        const v4i cd = mfma(af, bf2[x], v4i{0, 0, 0, 0});
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            const float so = meta[GBM + wm * 64 + bm * 16 + (lane >> 4) * 4 + c];
                            tv[bm][x][c] = tv[bm][x][c] + (so * wd) * (float)cd[c];
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int bm = 0; bm < 4; ++bm)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int i = m0 + wm * 64 + bm * 16 + (lane >> 4) * 4 + c;
                if (i >= M) continue;
#pragma unroll
                for (int x = 0; x < 2; ++x) {
                    const int j = n0 + wn * 128 + (sub * 2 + x) * 16 + (lane & 15);
                    if (j >= N) continue;
                    float v = tv[bm][x][c];
                    if (meta[2 * GBM + wm * 64 + bm * 16 + (lane >> 4) * 4 + c] != 0.0f) {
                        // non-finite outlier: exact sequential corr
                        float corr = -0.0f;
                        const int8_t* wrow = W + (size_t)j * Kp;
                        for (int q = 0; q < t; ++q)
                            corr = corr + oval[(size_t)i * FRQ_T + q] *
                                              (float)wrow[min(oidx[(size_t)i * FRQ_T + q], (uint32_t)(Kp - 1))];
                        v = v + corr;
                    }
                    out[(size_t)i * N + j] = scale[j] * v;
                }
            }
    }
}

}  // namespace

size_t gemm_union_bytes(size_t m, size_t k) {
    (void)k;
    const size_t tiles = (m + BM - 1) / BM, mp = tiles * BM;
    return round_up(tiles * 4, 256) + round_up(tiles * UMAX * 4, 256) +
           2 * round_up(mp * 4, 256) + tiles * 3 * BM * UMAX;
}

hipError_t launch_union(size_t m, size_t k, const uint32_t* oidx,
                        const float* oval, void* ubuf, hipStream_t s) {
    const size_t tiles = (m + BM - 1) / BM;
    const size_t nw = (k + 31) / 32;
    const size_t lds = 2 * nw * sizeof(uint32_t);
    if (lds > 60 * 1024) return hipErrorInvalidValue;
    const int t = (int)(k < FRQ_T ? k : FRQ_T);
    union_kernel<<<dim3((unsigned)tiles), dim3(256), lds, s>>>(
        oidx, oval, (int)m, (int)k, t, union_view(ubuf, m));
    return hipGetLastError();
}

hipError_t launch_gemm_i8(const Weight& w, size_t m, const int8_t* a8,
                          const float* sa, const uint32_t* oidx,
                          const float* oval, const void* ubuf, float* out,
                          int32_t* acc, hipStream_t s) {
    // a8 holds round_up(m, 128) rows; wt / wkn are padded to (Np, Kp) / (Kp, Np)
    const int MT = (int)((m + GBM - 1) / GBM), NT = (int)(w.np / GBN);
    const int t = (int)(w.k < FRQ_T ? w.k : FRQ_T);
    gemm_i8_kernel<<<dim3((unsigned)(MT * NT)), dim3(256), 0, s>>>(
        a8, w.wt, w.wkn, w.scale, sa, (int)m, (int)w.n, (int)w.np, (int)w.kp, t,
        union_view(const_cast<void*>(ubuf), m), oidx, oval, out, acc, MT);
    return hipGetLastError();
}

}  // namespace frq
