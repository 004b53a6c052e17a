// gemm_i8.hip — int8 W8A8 GEMM on CDNA4 MFMA for prefill / batched shapes
// (M > 4), gfx950.
//
// Same arithmetic as Bundle::mm's I8 arm (/root/reference/src/bundle.rs:
// 688-724):  out[i,j] = scale[j] * (sa[i] * (acc[i,j] as f32) + corr[i,j]),
// acc = i8dot(a8[i], wt[j]) in i32 (bit-exact), corr = sum over row i's
// outliers of av * wt[j,ch].
//
// acc: LDS-tiled v_mfma_i32_16x16x64_i8 over a8 (Mp,Kp) x wt (Np,Kp), both
// K-contiguous.  128x128 output tile per 256-thread workgroup, 2x2 waves of
// 64x64 (4x4 MFMA blocks), k-step 128 (one 128-byte line per row), register
// prefetch of the next k-step while the current one is multiplied.
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

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int LP = BK + 16;          // LDS row pitch (bytes): conflict-free
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
__device__ __forceinline__ v4i mfma(const int4 a, const int4 b, v4i c) {
    v4i av = {a.x, a.y, a.z, a.w}, bv = {b.x, b.y, b.z, b.w};
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, c, 0, 0, 0);
}

// 16 x int4 of a 128x128-byte tile per thread-quad: thread tid owns rows
// tid/8 + 32*i (i < 4), 16-byte column chunk tid%8.
__device__ __forceinline__ void load_tile(const int8_t* __restrict__ g, size_t pitch,
                                          int4 (&r)[4]) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        r[i] = *reinterpret_cast<const int4*>(g + (size_t)(tid / 8 + 32 * i) * pitch + (tid % 8) * 16);
}
__device__ __forceinline__ void store_tile(int8_t* s, const int4 (&r)[4]) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        *reinterpret_cast<int4*>(s + (tid / 8 + 32 * i) * LP + (tid % 8) * 16) = r[i];
}

__device__ __forceinline__ void mma_tile(const int8_t* As, const int8_t* Bs,
                                         v4i (&acc)[4][4]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        int4 af[4], bf[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            af[b] = *reinterpret_cast<const int4*>(As + (wm * 64 + b * 16 + (lane & 15)) * LP + kb * 64 + (lane >> 4) * 16);
            bf[b] = *reinterpret_cast<const int4*>(Bs + (wn * 64 + b * 16 + (lane & 15)) * LP + kb * 64 + (lane >> 4) * 16);
        }
#pragma unroll
        for (int bm = 0; bm < 4; ++bm)
#pragma unroll
            for (int bn = 0; bn < 4; ++bn) acc[bm][bn] = mfma(af[bm], bf[bn], acc[bm][bn]);
    }
}

__global__ __launch_bounds__(256) void gemm_i8_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ W,
    const int8_t* __restrict__ Wkn, const float* __restrict__ scale,
    const float* __restrict__ sa, int M, int N, int Np, int Kp, int t,
    UnionView uv, const uint32_t* __restrict__ oidx,
    const float* __restrict__ oval, float* __restrict__ out,
    int32_t* __restrict__ acc_dbg) {
    __shared__ __attribute__((aligned(16))) int8_t As[BM * LP];
    __shared__ __attribute__((aligned(16))) int8_t Bs[BN * LP];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int n0 = blockIdx.x * BN, tile = blockIdx.y, m0 = tile * BM;

    // ---- corr = so * C, C via three int8 digit GEMMs over the union ----
    float accf[4][4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int c = 0; c < 4; ++c) accf[a][b][c] = 0.0f;
    const int nu = uv.nu[tile];
    const int nup = (nu + BK - 1) / BK * BK;
    const uint32_t* U = uv.u + (size_t)tile * UMAX;
    for (int d = 2; d >= 0 && nu > 0; --d) {
        v4i acc[4][4];
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b) acc[a][b] = v4i{0, 0, 0, 0};
        const int8_t* Dd = uv.d + ((size_t)tile * 3 + d) * BM * UMAX;
        for (int u0 = 0; u0 < nup; u0 += BK) {
            int4 ra[4];
            load_tile(Dd + u0, UMAX, ra);
            // B^T chunk: channel U[u0+uu], columns n0..n0+127 from wkn
            int4 rb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int uu = tid / 8 + 32 * i;
                rb[i] = *reinterpret_cast<const int4*>(Wkn + (size_t)U[u0 + uu] * Np + n0 + (tid % 8) * 16);
            }
            __syncthreads();
            store_tile(As, ra);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int uu = tid / 8 + 32 * i, jb = (tid % 8) * 16;
                const uint32_t w4[4] = {(uint32_t)rb[i].x, (uint32_t)rb[i].y, (uint32_t)rb[i].z, (uint32_t)rb[i].w};
#pragma unroll
                for (int b = 0; b < 16; ++b) Bs[(jb + b) * LP + uu] = (int8_t)(w4[b >> 2] >> ((b & 3) * 8));
            }
            __syncthreads();
            mma_tile(As, Bs, acc);
        }
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    accf[a][b][c] = accf[a][b][c] * 256.0f + (float)acc[a][b][c];
    }

    // ---- acc = a8 . wt^T ----
    v4i acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = v4i{0, 0, 0, 0};
    const int8_t* Ag = A + (size_t)m0 * Kp;
    const int8_t* Bg = W + (size_t)n0 * Kp;
    int4 ra[4], rb[4];
    load_tile(Ag, Kp, ra);
    load_tile(Bg, Kp, rb);
    for (int k0 = 0; k0 < Kp; k0 += BK) {
        __syncthreads();
        store_tile(As, ra);
        store_tile(Bs, rb);
        __syncthreads();
        if (k0 + BK < Kp) {
            load_tile(Ag + k0 + BK, Kp, ra);
            load_tile(Bg + k0 + BK, Kp, rb);
        }
        mma_tile(As, Bs, acc);
    }

    // ---- epilogue: lane holds rows 4*(lane/16)+c, column lane%16 of each
    // 16x16 block ----
#pragma unroll
    for (int bm = 0; bm < 4; ++bm)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int i = m0 + wm * 64 + bm * 16 + (lane >> 4) * 4 + c;
            if (i >= M) continue;
            const float sai = sa[i], soi = uv.so[i];
            const int fin = uv.fin[i];
#pragma unroll
            for (int bn = 0; bn < 4; ++bn) {
                const int j = n0 + wn * 64 + bn * 16 + (lane & 15);
                if (j >= N) continue;
                const int av = acc[bm][bn][c];
                float corr;
                if (!fin) {
                    corr = soi * accf[bm][bn][c];
                } else {
                    corr = -0.0f;
                    const int8_t* wrow = W + (size_t)j * Kp;
                    for (int q = 0; q < t; ++q)
                        corr = corr + oval[(size_t)i * FRQ_T + q] *
                                          (float)wrow[min(oidx[(size_t)i * FRQ_T + q], (uint32_t)(Kp - 1))];
                }
                out[(size_t)i * N + j] = scale[j] * (sai * (float)av + corr);
                if (acc_dbg) acc_dbg[(size_t)i * N + j] = av;
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
    const size_t tiles = (m + BM - 1) / BM;
    const int t = (int)(w.k < FRQ_T ? w.k : FRQ_T);
    dim3 grid((unsigned)(w.np / BN), (unsigned)tiles);
    gemm_i8_kernel<<<grid, dim3(256), 0, s>>>(
        a8, w.wt, w.wkn, w.scale, sa, (int)m, (int)w.n, (int)w.np, (int)w.kp, t,
        union_view(const_cast<void*>(ubuf), m), oidx, oval, out, acc);
    return hipGetLastError();
}

}  // namespace frq
