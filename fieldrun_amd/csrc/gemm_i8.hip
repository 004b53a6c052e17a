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
// itself, so corr runs on the f16 MFMA.  A pre-pass (gemm_prep_kernel) works
// once per 128-row tile, for every column tile at once: the union U of the
// tile's outlier channels (ascending, padded to a multiple of 64 with
// channel 0), each row's power-of-two scale so[i] = 2^(E-15) (max|av| =
// m * 2^E), and each outlier value x = av / so[i] (exact, |x| < 2^15) as an
// f16 pair hi = f16(x), lo = f16(x - hi), laid out as MFMA A blocks (128 x
// |U|, 64 union channels per chunk).  In the GEMM's epilogue a column tile
// gathers W[:, U] from the (Kp, Np) row-major copy (wkn: for a channel the
// tile's columns are contiguous bytes), turns the bytes into f16 B blocks in
// LDS with byte permutes (every int8 is exact in f16), and
// v_mfma_f32_16x16x32_f16 adds (hi + lo) . W[:, U]^T straight into the f32
// tile, which holds sa * acc / so (a power-of-two scaling, exact); the tile
// is scaled back by so at the end.  hi + lo is within 2^-22 |x|, so corr
// differs from the reference's f32 sum by ~1e-7 relative; acc stays
// bit-exact.  Rows with a non-finite or vanishing outlier take the exact
// sequential corr instead.  The f32 tile leaves through LDS, one wave slab
// of 16 rows at a time, as whole-row 16-byte stores.
//
// i8_exact_epilogue (for the decode engines, whose greedy tokens need the
// reference's bits) takes the GEMM's exact int32 sums instead and adds the
// outlier correction as the reference's sequential f32 sum.
#include "frq_internal.h"

#include <algorithm>

namespace frq {

namespace {

constexpr int GBM = 128, GBK = 64;
constexpr int CH = 64;              // union channels per correction chunk
// correction A blocks of one chunk: (hi, lo) x two 32-entry halves x 8 row blocks
constexpr int DCH = 2 * 2 * (GBM / 16) * 1024;

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

// The tile's union capacity: at most 128 rows x 32 outliers, at most Kp.
__host__ __device__ inline int union_cap(int kp) {
    const int u = kp < GBM * FRQ_T ? kp : GBM * FRQ_T;
    return (u + CH - 1) / CH * CH;
}

// Per 128-row tile (blockIdx.x): the union of its rows' outlier channels,
// per-row power-of-two scales, and the f16 (hi, lo) A blocks of chunks
// blockIdx.y, blockIdx.y + gridDim.y, ...  Outputs: nu[mt]; uch[mt][cap]
// (union channels ascending, then channel 0 up to the next multiple of 64);
// so[Mp] (0 on rows that take the exact corr), fin[Mp] (1 on those rows);
// D[mt][cap / 64][DCH bytes]: for chunk c the (hi, lo) x two 32-entry
// halves x 8 row-block f16 A blocks of rows 16rb.. against union entries
// 64c.., in MFMA A order.
__global__ __launch_bounds__(256) void gemm_prep_kernel(
    int M, int K, int Kp, int t, const uint32_t* __restrict__ oidx,
    const float* __restrict__ oval, int cap, int* __restrict__ nu_out,
    uint32_t* __restrict__ uch, float* __restrict__ so_out, float* __restrict__ fin_out,
    int8_t* __restrict__ D) {
    __shared__ uint32_t bitmap[640], wpre[640], scan[8];
    __shared__ __attribute__((aligned(16))) int8_t Dl[DCH];
    const int tid = threadIdx.x, mt = blockIdx.x, m0 = mt * GBM;
    const int nrows = min(GBM, M - m0);
    // thread (er, eh) takes outliers 16eh..16eh+15 of tile row er
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
    // valid outliers of this thread: q = 16eh + v < t, channel inside the row
    auto qv = [&](int v) { return rv && 16 * eh + v < t && oi_r[v] < (uint32_t)K; };

    // the row's digit scale and non-finite flag first, while the bitmap is
    // built below (its two threads are adjacent lanes)
    float mx = 0.0f;
    int fin = 0;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const bool in = rv && 16 * eh + v < t;
        const float av = fabsf(ov_r[v]);
        fin |= in && !(av <= 3.0e38f);
        mx = in ? fmaxf(mx, av) : mx;
    }
    mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    fin |= __shfl_xor(fin, 1, 64);
    // so = 2^(E - 15) with mx = m * 2^E, m in [0.5, 1): av / so is exact and
    // below 2^15 in magnitude; rows whose values are not finite, or so tiny
    // that 1/so leaves the f32 range, take the exact corr
    int E = 0;
    (void)frexpf(mx, &E);
    if (mx > 0.0f && E < -100) fin = 1;
    const bool sc = mx > 0.0f && !fin;
    const float so = sc ? ldexpf(1.0f, E - 15) : 1.0f, rso = sc ? ldexpf(1.0f, 15 - E) : 1.0f;

    // the union as byte flags (plain stores: the rows share channels, and
    // atomics on a few hot words would serialise), then bitmap words
    const int nwk = Kp >> 5;  // <= 640 bitmap words
    uint8_t* flag = reinterpret_cast<uint8_t*>(Dl);  // Kp bytes, before Dl holds digits
    for (int i = tid; i < Kp / 16; i += 256) reinterpret_cast<uint4*>(flag)[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();
#pragma unroll
    for (int v = 0; v < 16; ++v)
        if (qv(v)) flag[oi_r[v]] = 1;
    __syncthreads();
    {
        const int C = (nwk + 255) / 256, lo = tid * C, hi = min(lo + C, nwk);
        uint32_t cnt = 0;
        for (int w = lo; w < hi; ++w) {
            const uint4 f0 = reinterpret_cast<const uint4*>(flag)[2 * w];
            const uint4 f1 = reinterpret_cast<const uint4*>(flag)[2 * w + 1];
            const uint32_t fw[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
            uint32_t bits = 0;
#pragma unroll
            for (int d = 0; d < 8; ++d)
                bits |= ((fw[d] & 1u) | ((fw[d] >> 7) & 2u) | ((fw[d] >> 14) & 4u) | ((fw[d] >> 21) & 8u)) << (4 * d);
            bitmap[w] = bits;
            cnt += __popc(bits);
        }
        uint32_t nu_total;
        uint32_t base = excl_scan256(cnt, scan, &nu_total);
        for (int w = lo; w < hi; ++w) { wpre[w] = base; base += __popc(bitmap[w]); }
        if (tid == 0) scan[5] = nu_total;
    }
    __syncthreads();
    const int nu = (int)scan[5];
    // union position of each valid outlier (upos), and for rows that take
    // the MFMA corr (pos) the f16 pair (hi, lo) of av / so, hi + lo within
    // 2^-22 of it; branch-free, so the 32 LDS reads are in flight together
    int upos[16], pos[16];
    uint32_t dig[16];
    {
        uint32_t wp[16], bw[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint32_t w = qv(v) ? oi_r[v] >> 5 : 0u;
            wp[v] = wpre[w];
            bw[v] = bitmap[w];
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint32_t c = oi_r[v];
            upos[v] = qv(v) ? (int)(wp[v] + __popc(bw[v] & ((1u << (c & 31)) - 1u))) : -1;
            pos[v] = fin ? -1 : upos[v];
            const float x = ov_r[v] * rso;  // exact: rso = 1 / so, a power of two
            const _Float16 hi = (_Float16)x;
            const _Float16 lo = (_Float16)(x - (float)hi);
            dig[v] = (uint32_t)__builtin_bit_cast(uint16_t, hi) |
                     ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
        }
    }
    if (blockIdx.y == 0) {
        uint32_t* ut = uch + (size_t)mt * cap;
        if (tid == 0) nu_out[mt] = nu;
        if (eh == 0) {
            so_out[m0 + er] = rv ? so : 1.0f;
            fin_out[m0 + er] = (rv && fin) ? 1.0f : 0.0f;
        }
        // every union channel is some outlier's: equal values where shared
#pragma unroll
        for (int v = 0; v < 16; ++v)
            if (upos[v] >= 0) ut[upos[v]] = oi_r[v];
        for (int p = nu + tid; p < (nu + CH - 1) / CH * CH; p += 256) ut[p] = 0u;
    }
    const int nch = (nu + CH - 1) / CH;
    for (int c = blockIdx.y; c < nch; c += gridDim.y) {
        for (int i = tid; i < DCH / 16; i += 256) reinterpret_cast<uint4*>(Dl)[i] = make_uint4(0, 0, 0, 0);
        __syncthreads();
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int e = pos[v] - CH * c;
            if (e >= 0 && e < CH) {
                // entry e: half e / 32, lane group (e / 8) % 4, element e % 8
                const int off = (16 * ((e >> 3) & 3) + (er & 15)) * 8 + (e & 7);
                uint16_t* dl = reinterpret_cast<uint16_t*>(Dl);
#pragma unroll
                for (int p = 0; p < 2; ++p)
                    dl[((p * 2 + (e >> 5)) * 8 + (er >> 4)) * 512 + off] = (uint16_t)(dig[v] >> (16 * p));
            }
        }
        __syncthreads();
        int8_t* dst = D + ((size_t)mt * (cap / CH) + c) * DCH;
        for (int i = tid; i < DCH / 16; i += 256)
            reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(Dl)[i];
        __syncthreads();
    }
}

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// Two signed bytes of w (sel 0x04010400: bytes 0, 1; 0x04030402: bytes 2, 3)
// as an exact f16 pair: 0x6400 | (b ^ 0x80) is 1024 + b + 128.
__device__ __forceinline__ uint32_t i8x2_to_f16x2(uint32_t w, uint32_t sel) {
    const uint32_t m = __builtin_amdgcn_perm(0x64646464u, w ^ 0x80808080u, sel);
    const v2h h = __builtin_bit_cast(v2h, m) - (v2h){(_Float16)1152.0f, (_Float16)1152.0f};
    return __builtin_bit_cast(uint32_t, h);
}

// 4x4 byte transpose: out[y] byte x = in[x] byte y.
__device__ __forceinline__ void tr4(const uint32_t* in, uint32_t* out) {
    const uint32_t t0 = __builtin_amdgcn_perm(in[1], in[0], 0x05010400u);
    const uint32_t t1 = __builtin_amdgcn_perm(in[1], in[0], 0x07030602u);
    const uint32_t t2 = __builtin_amdgcn_perm(in[3], in[2], 0x05010400u);
    const uint32_t t3 = __builtin_amdgcn_perm(in[3], in[2], 0x07030602u);
    out[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
    out[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    out[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
    out[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

// MODE 0: the whole K range, then the epilogue.  MODE 1 (split K): workgroup
// b runs k-split b % nsplit of tile b / nsplit and stores its int32 tile to
// part.  MODE 2: one workgroup per tile adds the tile's nsplit partial tiles
// in split order (exact) and runs the epilogue.  AO: the epilogue only
// stores the exact int32 sums to acc (i8_exact_epilogue then forms out).
template <int BN, int NST, int MODE, bool AO>
__global__ __launch_bounds__(256, 2) void gemm_i8_kernel(
    const int8_t* __restrict__ Ab, const int8_t* __restrict__ Wb,
    const int8_t* __restrict__ Wkn, const int8_t* __restrict__ Wrow,
    const float* __restrict__ scale, const float* __restrict__ sa, int M, int Mp,
    int N, int Np, int Kp, int t, const uint32_t* __restrict__ oidx,
    const float* __restrict__ oval, float* __restrict__ out,
    int32_t* __restrict__ acc_dbg, int MT, int cap, const int* __restrict__ nu_g,
    const uint32_t* __restrict__ uch, const float* __restrict__ so_g,
    const float* __restrict__ fin_g, const int8_t* __restrict__ D, int32_t* __restrict__ part,
    int nsplit) {
    constexpr int ABLK = GBM / 16, BBLK = BN / 16, SBLK = ABLK + BBLK;
    constexpr int STAGE = SBLK * 1024;
    constexpr int TM = 4, TN = BN / 32;  // 16x16 blocks per wave (64 x BN/2)
    // DMA blocks per wave per stage: waves below SBLK % 4 take one more; the
    // ring's waits count the smaller number (waiting longer is safe)
    constexpr int PW = SBLK / 4, PWX = (SBLK + 3) / 4;
    extern __shared__ __attribute__((aligned(1024))) int8_t lds[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    int mt, nt;
    const int tb = MODE == 1 ? (int)blockIdx.x / nsplit : (int)blockIdx.x;
    const int sp = MODE == 1 ? (int)blockIdx.x % nsplit : 0;
    tile_of(tb, MODE == 1 ? (int)gridDim.x / nsplit : (int)gridDim.x, MT, mt, nt);
    const int m0 = mt * GBM, n0 = nt * BN;
    const int SK = Kp / GBK;  // k-steps of the whole row
    // this workgroup's k-steps: [k0, k0 + S)
    const int k0 = MODE == 1 ? SK * sp / nsplit : 0;
    const int S = MODE == 0 ? SK : MODE == 1 ? SK * (sp + 1) / nsplit - k0 : 0;
    const size_t arb = (size_t)Mp / 16, wrb = (size_t)Np / 16;

    auto issue = [&](int ks, int8_t* st) {
#pragma unroll
        for (int i = 0; i < PWX; ++i) {
            const int bl = wave + 4 * i;  // wave-uniform
            if (PWX == PW || bl < SBLK) {
                const int8_t* src = bl < ABLK
                    ? Ab + ((size_t)(k0 + ks) * arb + m0 / 16 + bl) * 1024 + lane * 16
                    : Wb + ((size_t)(k0 + ks) * wrb + n0 / 16 + (bl - ABLK)) * 1024 + lane * 16;
                dma16(src, st + bl * 1024);
            }
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
    // a k-split's int32 tile, 16 bytes per lane per block, 4 KB per block
    // over the workgroup
    int32_t* pt = part + ((size_t)(MODE == 1 ? blockIdx.x : tb * nsplit) * (TM * TN) * 256 + threadIdx.x) * 4;
    if constexpr (MODE == 1) {
#pragma unroll
        for (int bm = 0; bm < TM; ++bm)
#pragma unroll
            for (int bn = 0; bn < TN; ++bn)
                *reinterpret_cast<v4i*>(pt + (size_t)(bm * TN + bn) * 1024) = acc[bm][bn];
        return;
    }
    if constexpr (MODE == 2) {
        for (int q = 0; q < nsplit; ++q)
#pragma unroll
            for (int bm = 0; bm < TM; ++bm)
#pragma unroll
                for (int bn = 0; bn < TN; ++bn)
                    acc[bm][bn] += *reinterpret_cast<const v4i*>(pt + ((size_t)q * TM * TN + bm * TN + bn) * 1024);
    }
    if constexpr (AO) {
        // 16 lanes cover 64 contiguous bytes of a row per store
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
        return;
    }
    __syncthreads();  // every fragment read; the ring is free for the epilogue

    // ---- epilogue ------------------------------------------------------------
    // LDS carve (the ring is free): W[:, U] as f16 B blocks (2 x BN/16 x
    // 1 KB), row meta (sa, so, exact flag), column scales, and one 16-row
    // f32 slab per wave.
    constexpr int SP = BN / 2 + 4;  // slab pitch (floats)
    constexpr int WUB = BN * CH * 2;
    static_assert(WUB + 4 * (3 * GBM + BN + 4 * 16 * SP) <= NST * STAGE, "epilogue LDS exceeds the ring");
    int8_t* WU = lds;
    float* meta = reinterpret_cast<float*>(lds + WUB);  // [3][128]
    float* scl = meta + 3 * GBM;                            // [BN]
    float* slab = scl + BN + 16 * SP * wave;                // [16][SP]

    const int tid = threadIdx.x;
    const int nu = __builtin_amdgcn_readfirstlane(nu_g[mt]);
    const int nch = (nu + CH - 1) / CH;
    // the W[:, U] gather: unit (eg, cq) = union entries 8eg..8eg+7 of chunk c
    // at tile columns 4cq..4cq+3 (one dword of a wkn row each); UPT units
    // per thread
    constexpr int NQ = BN / 4, UPT = (8 * NQ + 255) / 256;
    const uint32_t* ut = uch + (size_t)mt * cap;
    uint32_t gw[8 * UPT];
    auto gather = [&](int c) {
#pragma unroll
        for (int u = 0; u < UPT; ++u) {
            int un = tid + 256 * u;
            if ((8 * NQ) % 256) un = min(un, 8 * NQ - 1);  // spare units repeat the last
            const int cq = un % NQ, eg = un / NQ;
            const uint4 q0 = *reinterpret_cast<const uint4*>(ut + c * CH + 8 * eg);
            const uint4 q1 = *reinterpret_cast<const uint4*>(ut + c * CH + 8 * eg + 4);
            const uint32_t chs[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
            for (int x = 0; x < 8; ++x)
                gw[8 * u + x] = *reinterpret_cast<const uint32_t*>(Wkn + (size_t)chs[x] * Np + n0 + 4 * cq);
        }
    };
    if (nch > 0) gather(0);
    if (tid < GBM) {
        meta[tid] = sa[min(m0 + tid, M - 1)];
        meta[GBM + tid] = so_g[m0 + tid];
        meta[2 * GBM + tid] = fin_g[m0 + tid];
    }
    if (tid < BN) scl[tid] = scale[n0 + tid];  // Np-padded: in bounds

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
    __syncthreads();  // meta, scl
    // t = (sa * acc) / so for the whole wave tile, in place of acc (so is a
    // power of two: exact both ways)
    v4f tv[TM][TN];
#pragma unroll
    for (int bm = 0; bm < TM; ++bm)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int rl = wm * 64 + bm * 16 + (lane >> 4) * 4 + c;
            const float sai = meta[rl], rso = 1.0f / meta[GBM + rl];
#pragma unroll
            for (int bn = 0; bn < TN; ++bn) tv[bm][bn][c] = (sai * (float)acc[bm][bn][c]) * rso;
        }

    // corr, one union chunk of 64 channels at a time: t += (hi + lo) . W[:, U]
    // on the f16 MFMA (32 entries per instruction), straight into t
    const int8_t* Dt = D + (size_t)mt * (cap / CH) * DCH + (wm * TM) * 1024 + lane * 16;
    for (int c = 0; c < nch; ++c) {
        // A fragments of one 16-row block at a time, the next one in flight:
        // [part (hi, lo)][half]
        const int8_t* Dc = Dt + (size_t)c * DCH;
        v4i af[2][4];
#pragma unroll
        for (int x = 0; x < 4; ++x) af[0][x] = *reinterpret_cast<const v4i*>(Dc + (x * 8) * 1024);
        // the gathered bytes -> f16 B blocks: half h, column block cb, lane
        // 16g + r = column 16cb + r, entries 32h + 8g .. +7
#pragma unroll
        for (int u = 0; u < UPT; ++u) {
            const int un = tid + 256 * u, cq = un % NQ, eg = un / NQ;  // entries 8eg..8eg+7
            if ((8 * NQ) % 256 && un >= 8 * NQ) continue;
            uint32_t o[4][2];
#pragma unroll
            for (int z = 0; z < 2; ++z) {
                uint32_t tmp[4];
                tr4(gw + 8 * u + 4 * z, tmp);
#pragma unroll
                for (int y = 0; y < 4; ++y) o[y][z] = tmp[y];
            }
#pragma unroll
            for (int y = 0; y < 4; ++y) {
                const int j = 4 * cq + y;
                uint4 hv;
                hv.x = i8x2_to_f16x2(o[y][0], 0x04010400u);
                hv.y = i8x2_to_f16x2(o[y][0], 0x04030402u);
                hv.z = i8x2_to_f16x2(o[y][1], 0x04010400u);
                hv.w = i8x2_to_f16x2(o[y][1], 0x04030402u);
                *reinterpret_cast<uint4*>(WU + ((eg >> 2) * (BN / 16) + (j >> 4)) * 1024 +
                                          (16 * (eg & 3) + (j & 15)) * 16) = hv;
            }
        }
        __syncthreads();
        if (c + 1 < nch) gather(c + 1);  // in flight during this chunk's MFMAs
#pragma unroll
        for (int bm = 0; bm < TM; ++bm) {
            if (bm + 1 < TM) {
#pragma unroll
                for (int x = 0; x < 4; ++x)
                    af[(bm + 1) & 1][x] = *reinterpret_cast<const v4i*>(Dc + (x * 8 + bm + 1) * 1024);
            }
#pragma unroll
            for (int bn = 0; bn < TN; ++bn) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const v4i bf = *reinterpret_cast<const v4i*>(WU + (h * (BN / 16) + wn * TN + bn) * 1024 + lane * 16);
#pragma unroll
                    for (int pp = 0; pp < 2; ++pp)
                        tv[bm][bn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(v8h, af[bm & 1][pp * 2 + h]), __builtin_bit_cast(v8h, bf), tv[bm][bn], 0, 0, 0);
                }
            }
        }
        __syncthreads();  // WU read by every wave before the next chunk's writes
    }

    // out = scale * t * so (rows with a non-finite outlier add the exact
    // sequential corr first), through the wave's LDS slab: 16 rows at a time,
    // written back as 16-byte runs of whole rows
    const bool vec = (N & 3) == 0;
    bool wexact = false;  // any exact-corr row among the wave's 64
#pragma unroll
    for (int bm = 0; bm < TM; ++bm)
#pragma unroll
        for (int q = 0; q < 4; ++q) wexact |= meta[2 * GBM + wm * 64 + bm * 16 + (lane >> 4) * 4 + q] != 0.0f;
    wexact = __builtin_amdgcn_ballot_w64(wexact) != 0;
    const int cbase = n0 + wn * (BN / 2);
    constexpr int Q4 = BN / 8, NIT = 16 * Q4 / 64;  // float4 runs per slab row, per lane
#pragma unroll
    for (int bm = 0; bm < TM; ++bm) {
        const int rbase = m0 + wm * 64 + bm * 16;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int rs = (lane >> 4) * 4 + q;  // slab row
            const int rl = wm * 64 + bm * 16 + rs;
            const float so = meta[GBM + rl];
#pragma unroll
            for (int bn = 0; bn < TN; ++bn) {
                const int cl = bn * 16 + (lane & 15);  // slab column
                float v = tv[bm][bn][q] * so;
                if (wexact && meta[2 * GBM + rl] != 0.0f && rbase + rs < M) {
                    const int i = rbase + rs, j = min(cbase + cl, N - 1);
                    float corr = -0.0f;
                    const int8_t* wr = Wrow + (size_t)j * Kp;
                    for (int qq = 0; qq < t; ++qq)
                        corr = corr + oval[(size_t)i * FRQ_T + qq] *
                                          (float)wr[min(oidx[(size_t)i * FRQ_T + qq], (uint32_t)(Kp - 1))];
                    v = v + corr;
                }
                slab[rs * SP + cl] = scl[wn * (BN / 2) + cl] * v;
            }
        }
        wave_sync();
        float4 vv[NIT];
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int idx = it * 64 + lane;
            vv[it] = *reinterpret_cast<const float4*>(slab + (idx / Q4) * SP + 4 * (idx % Q4));
        }
        if (vec && rbase + 16 <= M && cbase + BN / 2 <= N) {  // wave-uniform
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const int idx = it * 64 + lane;
                *reinterpret_cast<float4*>(out + (size_t)(rbase + idx / Q4) * N + cbase + 4 * (idx % Q4)) = vv[it];
            }
        } else {
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const int idx = it * 64 + lane, i = rbase + idx / Q4, j = cbase + 4 * (idx % Q4);
                if (i >= M) continue;
                float* o = out + (size_t)i * N + j;
                if (j < N) o[0] = vv[it].x;
                if (j + 1 < N) o[1] = vv[it].y;
                if (j + 2 < N) o[2] = vv[it].z;
                if (j + 3 < N) o[3] = vv[it].w;
            }
        }
        wave_sync();  // the slab is read before the next 16 rows overwrite it
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

// The pre-pass outputs, carved from the caller's workspace.
// The launch shape: tile width and the number of k-splits.
struct Plan {
    int bn = 128;
    int split = 1;
};

Plan plan_of(size_t m, size_t kp, size_t np) {
    Plan pl;
    const long MT = (long)((m + GBM - 1) / GBM);
    // tile width: two workgroups per CU run at once (512 slots); a launch
    // takes ceil(tiles / 512) rounds of a tile's time, about BN + 150 column
    // units (main loop plus a fixed share: the epilogue, whose correction
    // chunks cost much the same at either width)
    long best = -1;
    for (int cand : {256, 224, 128}) {
        if (np % cand) continue;
        const long tiles = MT * (long)(np / cand);
        const long cost = (tiles + 511) / 512 * (cand + 150);
        if (best < 0 || cost < best) { best = cost; pl.bn = cand; }
    }
    // fewer tiles than CUs: split K over more workgroups, at least four
    // k-steps each, up to the 512 slots
    const long tiles = MT * (long)(np / pl.bn), ks = (long)(kp / GBK);
    if (tiles < 256 && ks >= 8)
        pl.split = (int)std::max(1L, std::min(512 / tiles, ks / 4));
    return pl;
}

struct Prep {
    int cap = 0;
    int* nu = nullptr;
    uint32_t* uch = nullptr;
    float* so = nullptr;
    float* fin = nullptr;
    int8_t* D = nullptr;
    int32_t* part = nullptr;  // split-K partial tiles
};

size_t al256(size_t x) { return (x + 255) / 256 * 256; }

Prep carve_prep(void* ws, size_t mp, size_t kp) {
    Prep p;
    const size_t mt = mp / GBM;
    p.cap = union_cap((int)kp);
    char* c = static_cast<char*>(ws);
    p.nu = reinterpret_cast<int*>(c); c += al256(mt * 4);
    p.uch = reinterpret_cast<uint32_t*>(c); c += al256(mt * p.cap * 4);
    p.so = reinterpret_cast<float*>(c); c += al256(mp * 4);
    p.fin = reinterpret_cast<float*>(c); c += al256(mp * 4);
    p.D = reinterpret_cast<int8_t*>(c); c += al256(mt * (p.cap / CH) * DCH);
    p.part = reinterpret_cast<int32_t*>(c);
    return p;
}

template <int BN, int NST, int MODE, bool AO>
hipError_t launch_k(const Weight& w, size_t m, const int8_t* a8b, const float* sa,
                    const uint32_t* oidx, const float* oval, float* out, int32_t* acc,
                    const Prep& p, int split, hipStream_t s) {
    const int MT = (int)((m + GBM - 1) / GBM), NT = (int)(w.np / BN);
    const size_t lds = (size_t)NST * (GBM + BN) / 16 * 1024;
    const int t = (int)(w.k < FRQ_T ? w.k : FRQ_T);
    auto kern = gemm_i8_kernel<BN, NST, MODE, AO>;
    static bool attr_set = false;  // per process; the attribute is per function
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const unsigned grid = (unsigned)(MT * NT * (MODE == 1 ? split : 1));
    kern<<<dim3(grid), dim3(256), lds, s>>>(
        a8b, w.wblk, w.wkn, w.wt, w.scale, sa, (int)m, MT * GBM, (int)w.n, (int)w.np, (int)w.kp, t,
        oidx, oval, out, acc, MT, p.cap, p.nu, p.uch, p.so, p.fin, p.D, p.part, split);
    return hipGetLastError();
}

template <int BN, int NST, bool AO>
hipError_t launch_t(const Weight& w, size_t m, const int8_t* a8b, const float* sa,
                    const uint32_t* oidx, const float* oval, float* out, int32_t* acc,
                    const Prep& p, int split, hipStream_t s) {
    if (split <= 1) return launch_k<BN, NST, 0, AO>(w, m, a8b, sa, oidx, oval, out, acc, p, 1, s);
    if (hipError_t e = launch_k<BN, NST, 1, AO>(w, m, a8b, sa, oidx, oval, out, acc, p, split, s); e != hipSuccess)
        return e;
    return launch_k<BN, NST, 2, AO>(w, m, a8b, sa, oidx, oval, out, acc, p, split, s);
}

// The engines' exact epilogue for M > 16 rows: out[i, j] = scale[j] *
// (sa[i] * (acc[i, j] as f32) + corr), corr the reference's M > 1 sum over
// row i's outliers (ascending channel, from -0.0, each product rounded
// before its add: bundle.rs:732-743), from the GEMM's exact i32 sums: the
// skinny kernel's arithmetic, bit for bit.  A workgroup owns JB adjacent
// columns for a share of the rows.  Their weights, Kp x JB bytes from the
// (Np, Kp) rows, sit in LDS channel-major, SW words a channel (an odd
// number, so the random channels of 64 rows spread over the banks): each
// outlier's JB weights are JB / 4 word reads, and the weights of a column
// block come from HBM once however dense the rows' outlier channels are.
// A thread takes one row at a time with its 32 (channel, value) pairs in
// registers.  Workgroup b: row chunk b / nblk, column block b % nblk, which
// within whole runs of 64 blocks puts 8 adjacent blocks on one XCD (16- and
// 32-byte row segments of acc and out share their lines there).
constexpr size_t EPI_LDS = 80 * 1024;
__host__ __device__ constexpr int epi_sw(int jb) { return (jb / 4) % 2 ? jb / 4 : jb / 4 + 1; }
inline size_t epi_lds(int jb, size_t kp) { return kp * (size_t)epi_sw(jb) * 4; }

template <int JB, int NT>
__global__ __launch_bounds__(NT) void i8_exact_epilogue(const int8_t* __restrict__ wt, int Kp,
                                                        const float* __restrict__ scale, int N, int M, int t,
                                                        const float* __restrict__ sa,
                                                        const uint32_t* __restrict__ oidx,
                                                        const float* __restrict__ oval,
                                                        const int32_t* __restrict__ acc, float* __restrict__ out,
                                                        int nblk, int rch) {
    constexpr int SW = epi_sw(JB), JQ = JB / 4;
    extern __shared__ uint32_t wl[];
    const int tid = threadIdx.x;
    const int b = (int)blockIdx.x, rc = b / nblk, xb = b % nblk;
    const int cb = (nblk % 8 == 0 && (xb / 64 + 1) * 64 <= nblk) ? (xb / 64) * 64 + (xb % 8) * 8 + (xb % 64) / 8 : xb;
    const int n0 = JB * cb;
    // the block's weights: 4 rows x 4 channels a thread, transposed to 4
    // channel words (byte x of word y: column 4jq + x of channel 4cq + y)
    const int nq = Kp >> 2;
    for (int x = tid; x < JQ * nq; x += NT) {
        const int jq = x / nq, cq = x - jq * nq;
        const int8_t* src = wt + (size_t)(n0 + 4 * jq) * Kp + 4 * cq;
        uint32_t r[4], o[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) r[u] = *reinterpret_cast<const uint32_t*>(src + (size_t)u * Kp);
        tr4(r, o);
#pragma unroll
        for (int u = 0; u < 4; ++u) wl[(4 * cq + u) * SW + jq] = o[u];
    }
    float scl[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) scl[j] = scale[n0 + j];  // Np entries
    __syncthreads();
    const bool vec = (N & 3) == 0 && n0 + JB <= N;
    for (int i = rc * NT + tid; i < M; i += rch * NT) {
        uint32_t ch[FRQ_T];
        float ov[FRQ_T];
#pragma unroll
        for (int v = 0; v < FRQ_T / 4; ++v) {
            const uint4 c4 = reinterpret_cast<const uint4*>(oidx + (size_t)i * FRQ_T)[v];
            const float4 o4 = reinterpret_cast<const float4*>(oval + (size_t)i * FRQ_T)[v];
            ch[4 * v] = c4.x; ch[4 * v + 1] = c4.y; ch[4 * v + 2] = c4.z; ch[4 * v + 3] = c4.w;
            ov[4 * v] = o4.x; ov[4 * v + 1] = o4.y; ov[4 * v + 2] = o4.z; ov[4 * v + 3] = o4.w;
        }
        int32_t a[JB];
        const int32_t* ar = acc + (size_t)i * N + n0;
        if (vec) {
#pragma unroll
            for (int q = 0; q < JQ; ++q) {
                const int4 v = reinterpret_cast<const int4*>(ar)[q];
                a[4 * q] = v.x; a[4 * q + 1] = v.y; a[4 * q + 2] = v.z; a[4 * q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < JB; ++j) a[j] = n0 + j < N ? ar[j] : 0;
        }
        float corr[JB];
#pragma unroll
        for (int j = 0; j < JB; ++j) corr[j] = -0.0f;
#pragma unroll
        for (int q = 0; q < FRQ_T; ++q) {
            if (q < t) {  // uniform: t = min(K, 32)
                const uint32_t* wq = wl + min(ch[q], (uint32_t)(Kp - 1)) * SW;
#pragma unroll
                for (int m = 0; m < JQ; ++m) {
                    const uint32_t wv = wq[m];
#pragma unroll
                    for (int x = 0; x < 4; ++x)
                        corr[4 * m + x] = corr[4 * m + x] + ov[q] * (float)(int8_t)(wv >> (8 * x));
                }
            }
        }
        const float s = sa[i];
        float r[JB];
#pragma unroll
        for (int j = 0; j < JB; ++j) r[j] = scl[j] * (s * (float)a[j] + corr[j]);
        float* orow = out + (size_t)i * N + n0;
        if (vec) {
#pragma unroll
            for (int q = 0; q < JQ; ++q)
                reinterpret_cast<float4*>(orow)[q] = make_float4(r[4 * q], r[4 * q + 1], r[4 * q + 2], r[4 * q + 3]);
        } else {
#pragma unroll
            for (int j = 0; j < JB; ++j)
                if (n0 + j < N) orow[j] = r[j];
        }
    }
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

size_t gemm_ws_bytes(size_t m, size_t kp, size_t np) {
    const size_t mp = round_up(m, GBM), mt = mp / GBM, cap = (size_t)union_cap((int)kp);
    const Plan pl = plan_of(m, kp, np);
    const size_t part = pl.split > 1 ? (size_t)pl.split * mp * np * 4 : 0;
    return al256(mt * 4) + al256(mt * cap * 4) + 2 * al256(mp * 4) + al256(mt * (cap / CH) * DCH) + part;
}

hipError_t launch_gemm_i8(const Weight& w, size_t m, const int8_t* a8b,
                          const float* sa, const uint32_t* oidx,
                          const float* oval, float* out, int32_t* acc, void* ws,
                          hipStream_t s, bool acc_only) {
    // a8b holds round_up(m, 128) blocked rows; wblk / wkn are padded to Np
    // (a multiple of 256) and Kp (a multiple of 128); Kp <= 20480 keeps the
    // channel bitmap within its 640 LDS words; ws holds
    // gemm_ws_bytes(m, Kp, Np)
    if (w.kp > 20480 || !w.wblk || !ws || (acc_only && !acc)) return hipErrorInvalidValue;
    const size_t mp = round_up(m, GBM);
    const Prep p = carve_prep(ws, mp, w.kp);
    const Plan pl = plan_of(m, w.kp, w.np);
    if (acc_only) {  // no correction operands: the exact epilogue follows
        if (pl.bn == 256) return launch_t<256, 3, true>(w, m, a8b, sa, oidx, oval, out, acc, p, pl.split, s);
        if (pl.bn == 224) return launch_t<224, 3, true>(w, m, a8b, sa, oidx, oval, out, acc, p, pl.split, s);
        return launch_t<128, 4, true>(w, m, a8b, sa, oidx, oval, out, acc, p, pl.split, s);
    }
    const int MT = (int)(mp / GBM), nchmax = p.cap / CH;
    const int t = (int)(w.k < FRQ_T ? w.k : FRQ_T);
    // chunk groups: enough workgroups to build a dense union's chunks in
    // parallel; each one builds the (cheap) union itself
    const int ncg = std::max(1, std::min(nchmax, 256 / MT));
    gemm_prep_kernel<<<dim3((unsigned)MT, (unsigned)ncg), dim3(256), 0, s>>>(
        (int)m, (int)w.k, (int)w.kp, t, oidx, oval, p.cap, p.nu, p.uch, p.so, p.fin, p.D);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    if (pl.bn == 256) return launch_t<256, 3, false>(w, m, a8b, sa, oidx, oval, out, acc, p, pl.split, s);
    if (pl.bn == 224) return launch_t<224, 3, false>(w, m, a8b, sa, oidx, oval, out, acc, p, pl.split, s);
    return launch_t<128, 4, false>(w, m, a8b, sa, oidx, oval, out, acc, p, pl.split, s);
}

template <int JB>
hipError_t launch_epi(const Weight& w, size_t m, const float* sa, const uint32_t* oidx, const float* oval,
                      const int32_t* acc, float* out, hipStream_t s) {
    constexpr int NT = 512;
    const int t = (int)(w.k < FRQ_T ? w.k : FRQ_T);
    const int nblk = (int)((w.n + JB - 1) / JB);
    // row chunks so that about two rounds of workgroups fill the chip
    const int rch = (int)std::max<size_t>(1, std::min<size_t>((m + NT - 1) / NT, (size_t)(1024 + nblk - 1) / nblk));
    const size_t lds = epi_lds(JB, w.kp);
    auto kern = i8_exact_epilogue<JB, NT>;
    static bool attr_set = false;  // per process; the attribute is per function
    if (!attr_set) {
        if (hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)EPI_LDS);
            e != hipSuccess)
            return e;
        attr_set = true;
    }
    kern<<<dim3((unsigned)(nblk * rch)), dim3(NT), lds, s>>>(w.wt, (int)w.kp, w.scale, (int)w.n, (int)m, t, sa,
                                                            oidx, oval, acc, out, nblk, rch);
    return hipGetLastError();
}

hipError_t launch_i8_exact_epilogue(const Weight& w, size_t m, const float* sa, const uint32_t* oidx,
                                    const float* oval, const int32_t* acc, float* out, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    // the weight block comes from the (Np, Kp) rows (Np a multiple of 256,
    // Kp of 128: whole blocks, whole channel quads, in bounds)
    if (!w.wt || m > 65535 || w.np % 256 || w.np < w.n || w.kp == 0 || w.kp % 128 || w.kp > 20480)
        return hipErrorInvalidValue;
    if (epi_lds(16, w.kp) <= EPI_LDS) return launch_epi<16>(w, m, sa, oidx, oval, acc, out, s);
    if (epi_lds(8, w.kp) <= EPI_LDS) return launch_epi<8>(w, m, sa, oidx, oval, acc, out, s);
    return launch_epi<4>(w, m, sa, oidx, oval, acc, out, s);
}

}  // namespace frq
