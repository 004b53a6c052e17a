// gemm_i8.hip — int8 W8A8 GEMM on CDNA4 MFMA for prefill / batched shapes
// (M > 4), gfx950.
//
// Same arithmetic as Bundle::mm's I8 arm (/root/reference/src/bundle.rs:
// 688-724):  out[i,j] = scale[j] * (sa[i] * (acc[i,j] as f32) + corr[i,j]),
// acc = i8dot(a8[i], wt[j]) in i32 (bit-exact), corr = sum over row i's
// outliers of av * wt[j,ch].
//
// Operand layout ("blocked", both a8 and the weight copy wblk): the MFMA
// operand of 16 rows x 64 k-bytes is one contiguous 1 KB block in lane order
// (lane 16g + r holds row r, k-bytes 16g..16g+15), blocks ordered k-block
// major: block (kb, rb) at (kb * R/16 + rb) * 1 KB.  Every global_load_lds
// of the main loop therefore reads 1 KB of contiguous memory, and a k-step's
// 8 (A) or 16 (B) blocks are consecutive.  (Loading the same operands from
// row-major (R, Kp) arrays, 16 rows x 64 bytes per instruction, runs the
// L2 -> LDS path at a third of the contiguous rate.)
//
// acc: 128 x BN output tile per 256-thread workgroup (BN = 256 or 128),
// 2x2 waves of 64 x BN/2, v_mfma_i32_16x16x64_i8, k-step 64; operands go
// HBM -> LDS directly (global_load_lds_dwordx4) through an NST-stage ring.
// The ring's waits are explicit vmcnt counts before a raw s_barrier:
// __syncthreads() would also drain every LDS-DMA load still in flight and
// serialise the ring.  The tile order is XCD-aware (tile_of).
//
// corr: 32 VALU multiply-adds per output would cost as much as the MFMA GEMM
// itself, so corr also runs on the int8 MFMA.  Per workgroup, after the main
// loop, the union U of its 128 rows' outlier channels is built in LDS (a
// channel bitmap and its prefix popcounts); each outlier value becomes
// X = round(av / so[i]), |X| <= 127*2^16, so[i] = max|av| / (127*2^16),
// split into three signed int8 digits X = d2*2^16 + d1*2^8 + d0.  Then
// C_d = D_d (128 x |U|) . W[:, U]^T is an exact int32 MFMA product per digit
// and corr = so * ((C2*256 + C1)*256 + C0).  W[:, U] is read from the (K, Np)
// row-major weight copy (wkn): for a channel, the tile's columns are
// contiguous bytes.  The 24-bit split makes corr differ from the reference's
// f32 sum by ~1e-7 relative; acc stays bit-exact.  Rows with a non-finite
// outlier take the exact sequential corr instead.
#include "frq_internal.h"

namespace frq {

namespace {

constexpr int GBM = 128, GBK = 64;
constexpr int CH = 64;              // union channels per correction chunk
constexpr float XMAX = 8323072.0f;  // 127 * 2^16

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

// Bijective XCD-aware tile order: workgroup b runs on XCD b % 8; the
// workgroups of one XCD take a contiguous run of tiles ordered N-tile
// major, M-tile minor, so an XCD's concurrent tiles share A k-slices and
// each weight panel in its L2.
__device__ __forceinline__ void tile_of(int b, int G, int MT, int& mt, int& nt) {
    const int x = b & 7, j = b >> 3;
    const int q = G >> 3, rem = G & 7;
    const int start = x * q + min(x, rem);
    const int tau = start + j;
    nt = tau / MT;
    mt = tau % MT;
}

// Block-exclusive prefix sum of one value per thread (256 threads).
__device__ uint32_t excl_scan256(uint32_t v, uint32_t* sc /*5 words*/, uint32_t* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(incl, off, 64);
        if (lane >= off) incl += y;
    }
    if (lane == 63) sc[wave] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t run = 0;
        for (int w = 0; w < 4; ++w) { const uint32_t c = sc[w]; sc[w] = run; run += c; }
        sc[4] = run;
    }
    __syncthreads();
    const uint32_t r = sc[wave] + incl - v;
    *total = sc[4];
    return r;
}

template <int BN, int NST>
__global__ __launch_bounds__(256, 2) void gemm_i8_kernel(
    const int8_t* __restrict__ Ab, const int8_t* __restrict__ Wb,
    const int8_t* __restrict__ Wkn, const int8_t* __restrict__ Wrow,
    const float* __restrict__ scale, const float* __restrict__ sa, int M, int Mp,
    int N, int Np, int K, int Kp, int t, const uint32_t* __restrict__ oidx,
    const float* __restrict__ oval, float* __restrict__ out,
    int32_t* __restrict__ acc_dbg, int MT) {
    constexpr int ABLK = GBM / 16, BBLK = BN / 16, SBLK = ABLK + BBLK;
    constexpr int STAGE = SBLK * 1024;
    constexpr int TM = 4, TN = BN / 32;  // 16x16 blocks per wave (64 x BN/2)
    constexpr int PW = SBLK / 4;         // DMA blocks per wave per stage
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    int mt, nt;
    tile_of(blockIdx.x, gridDim.x, MT, mt, nt);
    const int m0 = mt * GBM, n0 = nt * BN;
    const int S = Kp / GBK;
    const size_t arb = (size_t)Mp / 16, wrb = (size_t)Np / 16;

    auto issue = [&](int ks, int8_t* st) {
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            const int tb = wave + 4 * i;  // wave-uniform
            const int8_t* src = tb < ABLK
                ? Ab + ((size_t)ks * arb + m0 / 16 + tb) * 1024 + lane * 16
                : Wb + ((size_t)ks * wrb + n0 / 16 + (tb - ABLK)) * 1024 + lane * 16;
            dma16(src, st + tb * 1024);
        }
    };

    v4i acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = v4i{0, 0, 0, 0};

#pragma unroll
    for (int p = 0; p < NST - 1; ++p)
        if (p < S) issue(p, lds + p * STAGE);
    for (int s = 0; s < S; ++s) {
        // stage s has landed once at most (stages issued after s) x PW loads
        // of this wave are outstanding; then every wave's part is in LDS
        const int ahead = min(S - 1 - s, NST - 2);
        if (ahead >= 2) wait_vm<2 * PW>();
        else if (ahead == 1) wait_vm<PW>();
        else wait_vm<0>();
        __builtin_amdgcn_s_barrier();
        // the buffer refilled here held stage s-1, which every wave finished
        // reading (its fragments feed MFMAs issued before this barrier)
        if (s + NST - 1 < S) issue(s + NST - 1, lds + ((s + NST - 1) % NST) * STAGE);
        const int8_t* st = lds + (s % NST) * STAGE;
        v4i af[TM], bf[TN];
#pragma unroll
        for (int bm = 0; bm < TM; ++bm)
            af[bm] = *reinterpret_cast<const v4i*>(st + (wm * TM + bm) * 1024 + lane * 16);
#pragma unroll
        for (int bn = 0; bn < TN; ++bn)
            bf[bn] = *reinterpret_cast<const v4i*>(st + (ABLK + wn * TN + bn) * 1024 + lane * 16);
#pragma unroll
        for (int bm = 0; bm < TM; ++bm)
#pragma unroll
            for (int bn = 0; bn < TN; ++bn) acc[bm][bn] = mfma(af[bm], bf[bn], acc[bm][bn]);
    }
    __syncthreads();  // every fragment read; the ring is free for the epilogue

    // ---- epilogue ------------------------------------------------------------
    // LDS carve (the ring is free): header 8 KB (bitmap, prefix, row meta,
    // scan, chunk channels, column scales), digits 16 KB, union positions 8 KB, digit
    // blocks D 24 KB (first used as per-channel flags), W[:, U] blocks BN KB/16.
    const int nwk = Kp >> 5;                                   // <= 640 bitmap words
    uint32_t* bitmap = reinterpret_cast<uint32_t*>(lds);       // [640]
    uint32_t* wpre = bitmap + 640;                             // [640]
    float* meta = reinterpret_cast<float*>(lds + 5120);        // sa, so, fin: [3][128]
    uint32_t* scan = reinterpret_cast<uint32_t*>(lds + 6656);  // [8]
    uint32_t* uch = reinterpret_cast<uint32_t*>(lds + 6688);   // chunk channels [CH]
    float* scl = reinterpret_cast<float*>(lds + 7168);         // tile column scales [BN]
    uint32_t* dig = reinterpret_cast<uint32_t*>(lds + 8192);   // [128][32] digits d2|d1|d0
    uint16_t* dpos = reinterpret_cast<uint16_t*>(lds + 24576); // [128][32] union position
    int8_t* D = lds + 32768;                                   // 3 x 8 blocks (CH = 64)
    uint8_t* flag = reinterpret_cast<uint8_t*>(D);             // [Kp] before D is built
    int8_t* WU = lds + 32768 + 24 * 1024;                      // BN/16 blocks

    const int tid = threadIdx.x;
    const int nrows = min(GBM, M - m0);
    // every global operand of the epilogue in one batch of independent loads:
    // thread (er, eh) takes outliers 16eh..16eh+15 of tile row er; the tile's
    // column scales go to LDS
    const int er = tid >> 1, eh = tid & 1;
    const bool rv = er < nrows;
    uint32_t oi_r[16];
    float ov_r[16];
    {
        const size_t base = (size_t)(m0 + (rv ? er : 0)) * FRQ_T + eh * 16;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 x = *reinterpret_cast<const uint4*>(oidx + base + 4 * v);
            const float4 y = *reinterpret_cast<const float4*>(oval + base + 4 * v);
            oi_r[4 * v] = x.x; oi_r[4 * v + 1] = x.y; oi_r[4 * v + 2] = x.z; oi_r[4 * v + 3] = x.w;
            ov_r[4 * v] = y.x; ov_r[4 * v + 1] = y.y; ov_r[4 * v + 2] = y.z; ov_r[4 * v + 3] = y.w;
        }
    }
    const float sa_r = sa[min(m0 + er, M - 1)];
    if (tid < BN) scl[tid] = scale[n0 + tid];  // Np-padded: in bounds
    // valid outliers of this thread: q = 16eh + v < t
    auto qv = [&](int v) { return rv && 16 * eh + v < t; };

    // union of the tile's outlier channels: byte flags, then bitmap words
    for (int i = tid; i < Kp / 16; i += 256) reinterpret_cast<uint4*>(flag)[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();
#pragma unroll
    for (int v = 0; v < 16; ++v)
        if (qv(v) && oi_r[v] < (uint32_t)K) flag[oi_r[v]] = 1;
    __syncthreads();
    for (int w = tid; w < nwk; w += 256) {
        const uint4 f0 = reinterpret_cast<const uint4*>(flag)[2 * w];
        const uint4 f1 = reinterpret_cast<const uint4*>(flag)[2 * w + 1];
        const uint32_t fw[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
        uint32_t bits = 0;
#pragma unroll
        for (int b = 0; b < 32; ++b) bits |= ((fw[b >> 2] >> (8 * (b & 3))) & 1u) << b;
        bitmap[w] = bits;
    }
    __syncthreads();
    {
        const int C = (nwk + 255) / 256, lo = tid * C, hi = min(lo + C, nwk);
        uint32_t cnt = 0;
        for (int w = lo; w < hi; ++w) cnt += __popc(bitmap[w]);
        uint32_t nu_total;
        uint32_t base = excl_scan256(cnt, scan, &nu_total);
        for (int w = lo; w < hi; ++w) { wpre[w] = base; base += __popc(bitmap[w]); }
        if (tid == 0) scan[5] = nu_total;
    }
    // per row: sa, the digit scale so and the non-finite flag (the row's two
    // threads are adjacent lanes)
    float mx = 0.0f;
    int fin = 0;
#pragma unroll
    for (int v = 0; v < 16; ++v)
        if (qv(v)) {
            fin |= !(fabsf(ov_r[v]) <= 3.0e38f);
            mx = fmaxf(mx, fabsf(ov_r[v]));
        }
    mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    fin |= __shfl_xor(fin, 1, 64);
    float so = mx > 0.0f ? mx / XMAX : 1.0f;
    if (!(so >= 1.0e-30f) || !(so <= 1.0e30f)) fin = 1;  // keep digits exact
    if (eh == 0) {
        meta[er] = sa_r;
        meta[GBM + er] = fin ? 0.0f : so;
        meta[2 * GBM + er] = fin ? 1.0f : 0.0f;
    }
    __syncthreads();
    const int nu = (int)scan[5];
    // union position and three int8 digits of each outlier
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        uint32_t dv = 0;
        uint16_t p = 0xFFFF;
        if (qv(v) && !fin) {
            const uint32_t c = min(oi_r[v], (uint32_t)(K - 1));
            p = (uint16_t)(wpre[c >> 5] + __popc(bitmap[c >> 5] & ((1u << (c & 31)) - 1u)));
            float xf = rintf(ov_r[v] / so);
            xf = fminf(fmaxf(xf, -XMAX), XMAX);
            const int X = (int)xf;
            const int d0 = (int)(int8_t)(X & 0xFF);
            const int X1 = (X - d0) >> 8;
            const int d1 = (int)(int8_t)(X1 & 0xFF);
            const int d2 = (X1 - d1) >> 8;
            dv = (uint32_t)(d0 & 0xFF) | ((uint32_t)(d1 & 0xFF) << 8) | ((uint32_t)(d2 & 0xFF) << 16);
        }
        dig[er * FRQ_T + 16 * eh + v] = dv;
        dpos[er * FRQ_T + 16 * eh + v] = p;
    }

    if (acc_dbg) {
#pragma unroll
        for (int bm = 0; bm < TM; ++bm)
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int bn = 0; bn < TN; ++bn) {
                    const int i = m0 + wm * 64 + bm * 16 + (lane >> 4) * 4 + c;
                    const int j = n0 + wn * (BN / 2) + bn * 16 + (lane & 15);
                    if (i < M && j < N) acc_dbg[(size_t)i * N + j] = acc[bm][bn][c];
                }
    }
    // t = sa * acc for the whole wave tile, in place of acc
    float tv[TM][TN][4];
#pragma unroll
    for (int bm = 0; bm < TM; ++bm)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float sai = meta[wm * 64 + bm * 16 + (lane >> 4) * 4 + c];
#pragma unroll
            for (int bn = 0; bn < TN; ++bn) tv[bm][bn][c] = sai * (float)acc[bm][bn][c];
        }

    // corr, one union chunk of CH channels at a time: D_d blocks (d, rb) hold
    // rows 16rb.., chunk entries in lane order; WU block cb holds tile
    // columns 16cb.., the chunk's channels in lane order
    for (int u0 = 0; u0 < nu; u0 += CH) {
        __syncthreads();  // dig/dpos written; the previous chunk's blocks consumed
        for (int i = tid; i < 24 * 64; i += 256) reinterpret_cast<uint4*>(D)[i] = make_uint4(0, 0, 0, 0);
        if (tid < CH) {
            // the (u0 + tid)-th set bit of the bitmap: last word with wpre <= target
            const uint32_t target = (uint32_t)(u0 + tid);
            uint32_t ch = 0;
            if (target < (uint32_t)nu) {
                int lo = 0, hi = nwk - 1;
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (wpre[mid] <= target) lo = mid; else hi = mid - 1;
                }
                uint32_t bits = bitmap[lo];
                for (uint32_t k = target - wpre[lo]; k > 0; --k) bits &= bits - 1;
                ch = bits ? (uint32_t)lo * 32 + (uint32_t)(__ffs(bits) - 1) : 0u;
                ch = min(ch, (uint32_t)(K - 1));
            }
            uch[tid] = ch;
        }
        __syncthreads();
        for (int i = tid; i < GBM * FRQ_T; i += 256) {
            const int e = (int)dpos[i] - u0;
            if (e < 0 || e >= CH) continue;
            const int r = i / FRQ_T;
            const uint32_t dv = dig[i];
            const int off = ((16 * (e >> 4) + (r & 15)) * 16) + (e & 15);
#pragma unroll
            for (int d = 0; d < 3; ++d)
                D[(d * 8 + (r >> 4)) * 1024 + off] = (int8_t)((dv >> (8 * d)) & 0xFF);
        }
        {
            constexpr int NL = CH * (BN / 16) / 256;  // 16-byte loads per thread
            v4i wv[NL];
#pragma unroll
            for (int l = 0; l < NL; ++l) {
                const int idx = tid + 256 * l, e = idx % CH, cb = idx / CH;
                wv[l] = *reinterpret_cast<const v4i*>(Wkn + (size_t)uch[e] * Np + n0 + cb * 16);
            }
#pragma unroll
            for (int l = 0; l < NL; ++l) {
                const int idx = tid + 256 * l, e = idx % CH, cb = idx / CH;
#pragma unroll
                for (int b = 0; b < 16; ++b)
                    WU[cb * 1024 + ((16 * (e >> 4) + b) * 16) + (e & 15)] =
                        (int8_t)((uint32_t)wv[l][b >> 2] >> ((b & 3) * 8));
            }
        }
        __syncthreads();
        // tv += so * (C2 * 2^16 + C1 * 2^8 + C0); so is 0 on non-finite rows
#pragma unroll
        for (int bm = 0; bm < TM; ++bm) {
            float sow[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) sow[c] = meta[GBM + wm * 64 + bm * 16 + (lane >> 4) * 4 + c];
            v4i af[3];
#pragma unroll
            for (int d = 0; d < 3; ++d)
                af[d] = *reinterpret_cast<const v4i*>(D + (d * 8 + wm * 4 + bm) * 1024 + lane * 16);
#pragma unroll
            for (int bn = 0; bn < TN; ++bn) {
                const v4i bf = *reinterpret_cast<const v4i*>(WU + (wn * TN + bn) * 1024 + lane * 16);
                const v4i c2 = mfma(af[2], bf, v4i{0, 0, 0, 0});
                const v4i c1 = mfma(af[1], bf, v4i{0, 0, 0, 0});
                const v4i c0 = mfma(af[0], bf, v4i{0, 0, 0, 0});
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    tv[bm][bn][c] = tv[bm][bn][c] + (sow[c] * 65536.0f) * (float)c2[c];
                    tv[bm][bn][c] = tv[bm][bn][c] + (sow[c] * 256.0f) * (float)c1[c];
                    tv[bm][bn][c] = tv[bm][bn][c] + sow[c] * (float)c0[c];
                }
            }
        }
    }

    // out = scale * t; rows with a non-finite outlier add the exact sequential corr
#pragma unroll
    for (int bm = 0; bm < TM; ++bm)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int rl = wm * 64 + bm * 16 + (lane >> 4) * 4 + c;
            const int i = m0 + rl;
            if (i >= M) continue;
            const bool exact = meta[2 * GBM + rl] != 0.0f;
#pragma unroll
            for (int bn = 0; bn < TN; ++bn) {
                const int j = n0 + wn * (BN / 2) + bn * 16 + (lane & 15);
                if (j >= N) continue;
                float v = tv[bm][bn][c];
                if (exact) {
                    float corr = -0.0f;
                    const int8_t* wr = Wrow + (size_t)j * Kp;
                    for (int q = 0; q < t; ++q)
                        corr = corr + oval[(size_t)i * FRQ_T + q] *
                                          (float)wr[min(oidx[(size_t)i * FRQ_T + q], (uint32_t)(Kp - 1))];
                    v = v + corr;
                }
                out[(size_t)i * N + j] = scl[wn * (BN / 2) + bn * 16 + (lane & 15)] * v;
            }
        }
}

// (R, Kp) row-major (pitch) -> blocked, R a multiple of 16; rows >= valid are zero.
__global__ void blockify_kernel(const int8_t* __restrict__ src, size_t valid, size_t R,
                                size_t Kp, size_t pitch, int8_t* __restrict__ dst) {
    const size_t cpr = Kp / 16, total = R * cpr;
    for (size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const size_t row = idx / cpr, c = idx % cpr;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (row < valid) v = *reinterpret_cast<const uint4*>(src + row * pitch + c * 16);
        *reinterpret_cast<uint4*>(dst + blk_off(row, c * 16, R)) = v;
    }
}

template <int BN, int NST>
hipError_t launch_t(const Weight& w, size_t m, const int8_t* a8b, const float* sa,
                    const uint32_t* oidx, const float* oval, float* out, int32_t* acc,
                    hipStream_t s) {
    const int MT = (int)((m + GBM - 1) / GBM), NT = (int)(w.np / BN);
    const size_t lds = (size_t)NST * (GBM + BN) / 16 * 1024;
    const int t = (int)(w.k < FRQ_T ? w.k : FRQ_T);
    auto kern = gemm_i8_kernel<BN, NST>;
    static bool attr_set = false;  // per process; the attribute is per function
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    kern<<<dim3((unsigned)(MT * NT)), dim3(256), lds, s>>>(
        a8b, w.wblk, w.wkn, w.wt, w.scale, sa, (int)m, (int)round_up(m, GBM), (int)w.n,
        (int)w.np, (int)w.k, (int)w.kp, t, oidx, oval, out, acc, MT);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_blockify(const int8_t* src, size_t valid, size_t R, size_t kp,
                           size_t pitch, int8_t* dst, hipStream_t s) {
    if (!R || !kp) return hipSuccess;
    const size_t total = R * kp / 16;
    const size_t g = (total + 255) / 256;
    const unsigned grid = (unsigned)(g < 8192 ? g : 8192);
    blockify_kernel<<<dim3(grid), dim3(256), 0, s>>>(src, valid, R, kp, pitch, dst);
    return hipGetLastError();
}

hipError_t launch_gemm_i8(const Weight& w, size_t m, const int8_t* a8b,
                          const float* sa, const uint32_t* oidx,
                          const float* oval, float* out, int32_t* acc,
                          hipStream_t s) {
    // a8b holds round_up(m, 128) blocked rows; wblk / wkn are padded to Np
    // (a multiple of 256) and Kp (a multiple of 128); Kp <= 20480 keeps the
    // channel bitmap within its 640 LDS words
    if (w.kp > 20480 || !w.wblk) return hipErrorInvalidValue;
    const size_t tiles256 = ((m + GBM - 1) / GBM) * (w.np / 256);
    if (tiles256 >= 512) return launch_t<256, 3>(w, m, a8b, sa, oidx, oval, out, acc, s);
    return launch_t<128, 4>(w, m, a8b, sa, oidx, oval, out, acc, s);
}

}  // namespace frq
