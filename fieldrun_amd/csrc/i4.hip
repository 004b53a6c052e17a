// i4.hip — group-wise int4 W4A32 linear (gfx950).
//
// Restates the I4 arm of Bundle::mm (/root/reference/src/bundle.rs:760-799):
//  M == 1 (767-776): out[j] = i4_dot(row j), which on x86 is i4_dot_avx2
//    (199-225): per group, 8 lane accumulators each an FMA chain over the
//    group's 8-nibble chunks, then hsum256 ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7))
//    (146-153), a scalar mul+add tail, then sum += scale[g] * gsum.
//  M > 1 (777-798): w[kk,j] = s4 * scale[j, kk/g] (f32) then a.dot(w),
//    matrixmultiply's sgemm: per output, k in blocks of MM_KC, each an FMA
//    chain from +0, the blocks added in order; the exact M > 1 kernels below
//    reproduce that order.
//
// Blocked shapes (g == 32, K % 32 == 0, 1 <= M <= 16) run on the int8
// MFMA.  At upload the nibbles are re-laid out so that the B operand of
// v_mfma_i32_16x16x32_i8 (16 weight rows x 32 k = one group) for four
// consecutive groups is one 16-byte load per lane and a wave load is 1 KB of
// contiguous memory; in registers each packed dword (8 nibbles) becomes two
// dwords of sign-extended int8 with 8 VALU operations.  The f32 activations
// of each (token, group) are written as X = round(a / s), s = max|a| /
// (127 * 2^16), |X| <= 127 * 2^16, split into three int8 digits
// X = d2*2^16 + d1*2^8 + d0; token m's digits are A rows 4m, 4m+1, 4m+2, so
// one MFMA gives the exact integer group dots of 4 tokens, and
//   gsum = s * (C2 * 2^16 + C1 * 2^8 + C0),   out += scale[j,g] * gsum.
// The 24-bit fixed point per group keeps the result within ~1e-7 of
// max|a| * sum|w| of the group (the reference's own sums differ between its
// M == 1 and M > 1 arms by more); a (token, group) with a non-finite or
// extreme activation takes the group sum in the reference arm's own order
// instead (i4_dot_avx2 for M == 1, the dequantised a * (s4 * scale) chain
// for M > 1).  The digits are written once per call by a small kernel
// (L2-resident, read by every row block); K is split across the waves of
// one workgroup and the parts are added in order through LDS: a split across
// workgroups would need device-scope fences, which on this part write back
// and invalidate the whole L2.
// Other shapes run i4_gemv_generic (M == 1, bit-identical to i4_dot_avx2)
// or, M > 1 in the exact order, i4_mm_dpp (K % 32 == 0, g % 16 == 0),
// i4_rows_chain (K and g multiples of 32) or i4_gemm_rows.  Up to 16
// independent M == 1 rows (a batched decode) run i4_rows_dpp.
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

// M == 1 in i4_dot_avx2's order, fast: a group's term scale * gsum is
// independent of the others until the in-order sum, so a thread takes one
// (row, group) at a time (adjacent threads adjacent groups: the G4 16-byte
// nibble loads and the f16 scales arrive coalesced), the activations come
// from the workgroup's LDS copy (padded 4 floats per 32 against bank
// conflicts), and one lane per row adds its row's terms in order.  Needs
// K % 32 == 0 (16-byte aligned rows) and g == 32 G4.
template <int G4>
__global__ __launch_bounds__(256) void i4_gemv_terms(const uint8_t* __restrict__ packed,
                                                     const uint16_t* __restrict__ scale, int N, int K, int rb,
                                                     const float* __restrict__ a, float* __restrict__ out) {
    extern __shared__ float4 lds4[];
    float* cg = reinterpret_cast<float*>(lds4);
    constexpr int g = 32 * G4;
    const int ng = K / g, pitch = K / 2;
    const int r0 = blockIdx.x * rb;
    const int nr = min(rb, N - r0);
    const int items = nr * ng;
    const int ngp = (ng + 3) & ~3;  // row stride of the terms: 16-byte aligned rows
    float* as = cg + rb * ngp;
    for (int i = threadIdx.x; i < K / 4; i += 256)
        *reinterpret_cast<float4*>(as + (4 * i) / 32 * 36 + (4 * i) % 32) = reinterpret_cast<const float4*>(a)[i];
    __syncthreads();
    // the next item's nibbles and scale load while this one computes (the
    // index clamped to the last item, so every load is unconditional)
    auto fetch = [&](int p, uint4 (&w)[G4], float& sc) {
        const int r = p / ng, gi = p - r * ng;
        const uint8_t* pg = packed + (size_t)(r0 + r) * pitch + (size_t)gi * 16 * G4;
#pragma unroll
        for (int h = 0; h < G4; ++h) w[h] = *reinterpret_cast<const uint4*>(pg + 16 * h);
        sc = h2f(scale[(size_t)(r0 + r) * ng + gi]);
    };
    if (threadIdx.x < items) {
        uint4 wn[G4];
        float sn;
        fetch(threadIdx.x, wn, sn);
        for (int p = threadIdx.x; p < items; p += 256) {
            uint4 wc[G4];
#pragma unroll
            for (int h = 0; h < G4; ++h) wc[h] = wn[h];
            const float sc = sn;
            fetch(min(p + 256, items - 1), wn, sn);
            const int rr = p / ng, gi = p - rr * ng;
            float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
            for (int h = 0; h < G4; ++h) {
                const uint32_t ws[4] = {wc[h].x, wc[h].y, wc[h].z, wc[h].w};
                const float* ab = as + (gi * g + 32 * h) / 32 * 36;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float4 a0 = *reinterpret_cast<const float4*>(ab + 8 * c);
                    const float4 a1 = *reinterpret_cast<const float4*>(ab + 8 * c + 4);
                    const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
                    for (int q = 0; q < 8; ++q) l[q] = __builtin_fmaf(s4f(ws[c], q), av[q], l[q]);
                }
            }
            const float q0 = l[0] + l[4], q1 = l[1] + l[5], q2 = l[2] + l[6], q3 = l[3] + l[7];
            cg[rr * ngp + gi] = sc * ((q0 + q2) + (q1 + q3));
        }
    }
    __syncthreads();
    for (int r = threadIdx.x; r < nr; r += 256) out[r0 + r] = lds_seq_sum(cg + r * ngp, ng, 0.0f);
}

// M == 1 in i4_dot_avx2's order, streamed: a persistent grid of about one
// workgroup per CU, each owning a contiguous range of R rows, so its
// R * ng items (row, group) are one contiguous run of the packed weights
// and of the scales.  A thread takes items tid + NT i; every one of its
// nibble and scale loads is issued up front, right after the direct-to-LDS
// loads of the activation row (32-float units padded to 36 against bank
// conflicts), and items are consumed in issue order as the loads land.  A
// group's term scale * gsum goes to LDS; after one barrier a lane per row
// adds its row's terms in order.
//   Nibbles to f32: (x & 0x000F000F) ^ 0x64086408 puts (q ^ 8) of nibbles
// 0 and 4 of a word under the f16 exponent of 1024 (one bit operation),
// a packed f16 add of -1032 leaves the exact signed values q - 16 [q >= 8]
// in both halves, and v_fma_mix_f32 takes either half as an exactly
// widened f32 operand of the FMA: the products and their rounding are
// those of fma(float(s4), a, acc).
__device__ __forceinline__ void nib_f16x2(uint32_t x, uint32_t (&d)[4]) {
    d[0] = (x & 0x000F000Fu) ^ 0x64086408u;
    d[1] = ((x >> 4) & 0x000F000Fu) ^ 0x64086408u;
    d[2] = ((x >> 8) & 0x000F000Fu) ^ 0x64086408u;
    d[3] = ((x >> 12) & 0x000F000Fu) ^ 0x64086408u;
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// One 32-nibble unit (4 words) against 32 activations into the eight AVX2
// lane chains l[q] (element 8c + q is nibble q of word c).
__device__ __forceinline__ void unit_fma(const uint4 w, const float* __restrict__ ab, float (&l)[8]) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    const f16x2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        uint32_t d[4];
        nib_f16x2(ws[c], d);
        f16x2 h[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) h[j] = __builtin_bit_cast(f16x2, d[j]) + off;
        const float4 a0 = *reinterpret_cast<const float4*>(ab + 8 * c);
        const float4 a1 = *reinterpret_cast<const float4*>(ab + 8 * c + 4);
        const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
        for (int q = 0; q < 8; ++q) l[q] = __builtin_fmaf((float)(q < 4 ? h[q].x : h[q - 4].y), av[q], l[q]);
    }
}

// LDS bytes of the staged activation row: 16-byte slots of 9 a unit (8 of
// data, 1 of padding), whole 1 KB loads of 64 slots.
__host__ __device__ inline size_t i4_stream_as_bytes(int K) { return (size_t)(K / 32 * 9 + 63) / 64 * 1024; }

template <int G4, int IPT, int NT>
__global__ __launch_bounds__(NT) void i4_m1_stream(const uint8_t* __restrict__ packed,
                                                    const uint16_t* __restrict__ scale, int N, int K, int R,
                                                    const float* __restrict__ a, float* __restrict__ out) {
    extern __shared__ float4 lds4[];
    constexpr int g = 32 * G4;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, ng = K / g, nu = K / 32;
    constexpr int NW = NT / 64;
    const int r0 = blockIdx.x * R;
    if (r0 >= N) return;  // workgroup-uniform, before any barrier
    const int nr = min(R, N - r0), items = nr * ng;
    const int ngp = (ng + 3) & ~3;  // terms row stride: 16-byte aligned rows
    char* lds = reinterpret_cast<char*>(lds4);
    const float* as = reinterpret_cast<const float*>(lds);                // unit u at 36 u floats
    float* terms = reinterpret_cast<float*>(lds + i4_stream_as_bytes(K));  // nr rows of ngp floats, 1 dummy
    const float4* a4 = reinterpret_cast<const float4*>(a);
    // 1. the activation row straight into LDS (L2-resident, shared by every
    //    workgroup): load q of the workgroup fills slots 64 q .. 64 q + 63,
    //    slot k = 9 u + j holding float4 8 u + j (j == 8: padding, a dummy)
    const int nslot = nu * 9, nld = (nslot + 63) / 64;
    for (int q = wave; q < nld; q += NW) {
        const int k = q * 64 + lane, u = k / 9, j = k - 9 * u;
        dma16_lds(u < nu && j < 8 ? a4 + 8 * u + j : a4, lds + (size_t)q * 1024);
    }
    __builtin_amdgcn_sched_barrier(0);
    // 2. every item's nibbles and scale (indices clamped: unconditional)
    const uint4* wp = reinterpret_cast<const uint4*>(packed + (size_t)r0 * ng * 16 * G4);
    const uint16_t* sp = scale + (size_t)r0 * ng;
    uint4 w[IPT][G4];
    uint16_t sc[IPT];
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
        const int p = min(tid + NT * i, items - 1);
#pragma unroll
        for (int h = 0; h < G4; ++h) w[i][h] = wp[(size_t)p * G4 + h];
        sc[i] = sp[p];
    }
    asm volatile("" ::: "memory");  // no load sinks below this point
    __builtin_amdgcn_sched_barrier(0);
    // 3. the row's loads were issued before these IPT (G4 + 1): once at most
    //    that many are outstanding, this wave's share of the row is in LDS,
    //    and after the barrier every wave's is
    wait_vmcnt<IPT * (G4 + 1)>();
    __builtin_amdgcn_s_barrier();
    // item p = tid + NT i: row r = p / ng and group gi = p % ng, kept
    // incrementally; every item is computed (past the end: a copy of the
    // last, stored to a dummy slot)
    const int q256 = NT / ng, m256 = NT % ng;
    int r = tid / ng, gi = tid % ng;
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
        const int p = tid + NT * i;
        const int gc = p < items ? gi : ng - 1;
        float l[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int h = 0; h < G4; ++h) unit_fma(w[i][h], as + (gc * G4 + h) * 36, l);
        const float q0 = l[0] + l[4], q1 = l[1] + l[5], q2 = l[2] + l[6], q3 = l[3] + l[7];
        const float t = h2f(sc[i]) * ((q0 + q2) + (q1 + q3));
        terms[p < items ? r * ngp + gi : nr * ngp] = t;  // past the end: a dummy slot (the compute
                                                         // stays live, so its loads stay hoisted)
        r += q256;
        gi += m256;
        if (gi >= ng) {
            gi -= ng;
            ++r;
        }
    }
    __syncthreads();
    for (int rr = tid; rr < nr; rr += NT) out[r0 + rr] = lds_seq_sum(terms + rr * ngp, ng, 0.0f);
}

// 16 FMAs of one weight register v of a 32-unit into lane chains
// l[4 v .. 4 v + 3]: v_fmac_f32_dpp with row_newbcast:n gives each token
// lane of a 16-lane DPP row the weight held by lane n of that row.  Lane n
// holds element e = 8 (n & 3) + (n >> 2) + 4 v, which is nibble
// (n >> 2) + 4 v of word n & 3 (chain q = e & 7, chunk c = e >> 3), and its
// product takes av[e]; the FMAs go c-major so each chain advances in chunk
// order.  START begins the chains: chunk 0 is a v_mul_f32_dpp, which
// differs from fma(w, a, +0) only in giving -0 for a -0 product; a chain
// is exact otherwise, the lane sums of i4_dot_avx2 then differ at most in
// the sign of a zero, and so does a group term, which the running sum from
// +0 absorbs (+0 + -0 == +0): the row sums are bit-identical.  The s_nop
// gives the two wait states a DPP read needs after the VALU write of w,
// which the compiler does not see inside the asm.
#define FRQ_DPPF(op, acc, n, src) #op "_f32_dpp %" #acc ", %4, %" #src " row_newbcast:" #n " row_mask:0xf bank_mask:0xf\n\t"
#define FRQ_DPP_C0(op) FRQ_DPPF(op, 0, 0, 5) FRQ_DPPF(op, 1, 4, 9) FRQ_DPPF(op, 2, 8, 13) FRQ_DPPF(op, 3, 12, 17)
#define FRQ_DPP_C123                                                                                          \
    FRQ_DPPF(v_fmac, 0, 1, 6) FRQ_DPPF(v_fmac, 1, 5, 10) FRQ_DPPF(v_fmac, 2, 9, 14) FRQ_DPPF(v_fmac, 3, 13, 18) \
    FRQ_DPPF(v_fmac, 0, 2, 7) FRQ_DPPF(v_fmac, 1, 6, 11) FRQ_DPPF(v_fmac, 2, 10, 15)                            \
    FRQ_DPPF(v_fmac, 3, 14, 19) FRQ_DPPF(v_fmac, 0, 3, 8) FRQ_DPPF(v_fmac, 1, 7, 12)                            \
    FRQ_DPPF(v_fmac, 2, 11, 16) FRQ_DPPF(v_fmac, 3, 15, 20)
#define FRQ_DPP_OPS(V)                                                                              \
    : "+v"(l[4 * V]), "+v"(l[4 * V + 1]), "+v"(l[4 * V + 2]), "+v"(l[4 * V + 3])                    \
    : "v"(w), "v"(av[4 * V]), "v"(av[8 + 4 * V]), "v"(av[16 + 4 * V]), "v"(av[24 + 4 * V]),         \
      "v"(av[1 + 4 * V]), "v"(av[9 + 4 * V]), "v"(av[17 + 4 * V]), "v"(av[25 + 4 * V]),             \
      "v"(av[2 + 4 * V]), "v"(av[10 + 4 * V]), "v"(av[18 + 4 * V]), "v"(av[26 + 4 * V]),            \
      "v"(av[3 + 4 * V]), "v"(av[11 + 4 * V]), "v"(av[19 + 4 * V]), "v"(av[27 + 4 * V])
template <int V, bool START>
__device__ __forceinline__ void dpp_fma16(float (&l)[8], float w, const float (&av)[32]) {
    if constexpr (START)
        asm("s_nop 1\n\t" FRQ_DPP_C0(v_mul) FRQ_DPP_C123 FRQ_DPP_OPS(V));
    else
        asm("s_nop 1\n\t" FRQ_DPP_C0(v_fmac) FRQ_DPP_C123 FRQ_DPP_OPS(V));
}
#undef FRQ_DPP_OPS
#undef FRQ_DPP_C123
#undef FRQ_DPP_C0
#undef FRQ_DPPF

// One k of R FMA chains: c[r] = fma(w_r(lane n), a, c[r]) for r < R, where
// v_fmac_f32_dpp row_newbcast:n gives every token lane of a 16-lane DPP row
// the weight held by lane n of that row (lane n: k0 + n).  The s_nop gives
// the two wait states a DPP read needs after the VALU write of the weights.
#define FRQ_CHF(acc, w, a, n) "v_fmac_f32_dpp %" #acc ", %" #w ", %" #a " row_newbcast:" #n " row_mask:0xf bank_mask:0xf\n\t"
#define FRQ_CH8(n)                                                                                       \
    FRQ_CHF(0, 8, 16, n) FRQ_CHF(1, 9, 16, n) FRQ_CHF(2, 10, 16, n) FRQ_CHF(3, 11, 16, n) FRQ_CHF(4, 12, 16, n) \
    FRQ_CHF(5, 13, 16, n) FRQ_CHF(6, 14, 16, n) FRQ_CHF(7, 15, 16, n)
#define FRQ_CH8_OPS                                                                                          \
    : "+v"(c[0]), "+v"(c[1]), "+v"(c[2]), "+v"(c[3]), "+v"(c[4]), "+v"(c[5]), "+v"(c[6]), "+v"(c[7])         \
    : "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(a)
#define FRQ_CH8_CASE(n) \
    if constexpr (N == n) asm("s_nop 1\n\t" FRQ_CH8(n) FRQ_CH8_OPS);
template <int N>
__device__ __forceinline__ void dpp_chain8(float (&c)[8], const float (&w)[8], float a) {
    FRQ_CH8_CASE(0) FRQ_CH8_CASE(1) FRQ_CH8_CASE(2) FRQ_CH8_CASE(3) FRQ_CH8_CASE(4) FRQ_CH8_CASE(5)
    FRQ_CH8_CASE(6) FRQ_CH8_CASE(7) FRQ_CH8_CASE(8) FRQ_CH8_CASE(9) FRQ_CH8_CASE(10) FRQ_CH8_CASE(11)
    FRQ_CH8_CASE(12) FRQ_CH8_CASE(13) FRQ_CH8_CASE(14) FRQ_CH8_CASE(15)
}
#undef FRQ_CH8_CASE
#undef FRQ_CH8_OPS
#undef FRQ_CH8
#undef FRQ_CHF

// M > 1 rows in a.dot's order (each output: MM_KC-long k blocks, each an
// FMA chain from +0 over k with w = s4 * scale, the blocks added in order)
// with the weights broadcast across tokens: lane 16 d + t of a wave is
// token t of the workgroup's 16-row tile (blockIdx.y) in DPP row d.  The
// ND = 4 NW DPP rows D = BP rs + ph form ND / BP row sets of BP block
// phases: row set rs owns the R weight rows r0 + R rs .. + R - 1, phase ph
// takes blocks ph, ph + BP, ... .  For each 16-k chunk a lane dequantises
// its rows' 16 weights into one register a row (lane n: k0 + n, exact
// s4 * scale) and dpp_chain8 advances the R chains one k at a time; the
// chunk's activations are the lane's own 16 (row-major), one chunk ahead.
// A block's chain values go to LDS; after a slice of BP blocks, one barrier,
// and the lane of each (row, token) adds them to its running sum in block
// order (blocks past the end add +0, which a sum from +0 absorbs: no chain
// from +0 ends at -0).  Needs K % 32 == 0, g % 16 == 0, M rows of K floats
// 16-byte aligned.
template <int NW>
__global__ __launch_bounds__(64 * NW) void i4_mm_dpp(const uint8_t* __restrict__ packed,
                                                     const uint16_t* __restrict__ scale, int N, int K, int g,
                                                     const float* __restrict__ a, int M, float* __restrict__ out,
                                                     int BP) {
    constexpr int R = 8, ND = 4 * NW;
    constexpr int TB = ND * R * 16 * 2;  // term floats a buffer (RS R 16 pairs, BP + 1 apart)
    __shared__ float tb[2][TB];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t = lane & 15, D = 4 * wave + (lane >> 4);
    const int RS = ND / BP, rs = D / BP, ph = D - rs * BP, TS = BP + 1;
    const int nb = (K + MM_KC - 1) / MM_KC, nsl = (nb + BP - 1) / BP;
    const int rows = RS * R, r0 = blockIdx.x * rows + rs * R, m0 = blockIdx.y * 16;
    const int ng = (K + g - 1) / g;
    const size_t pitch = (size_t)K / 2;
    const uint8_t* wrow[R];
    const uint16_t* srow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const size_t row = (size_t)min(r0 + r, N - 1);  // clamped: loads stay unconditional
        wrow[r] = packed + row * pitch + 4 * (t >> 3);
        srow[r] = scale + row * ng;
    }
    const float* ar = a + (size_t)min(m0 + t, M - 1) * K;
    const int sh = 4 * (t & 7);
    // this lane's chunk sequence: slice s, chunk q of block s BP + ph
    // (clamped to the last chunk of the row past the end: its values go
    // unused)
    const int nck = (K / 16);
    auto chunk_k = [&](int s, int q) { return min((s * BP + ph) * MM_KC + 16 * q, 16 * (nck - 1)); };
    struct Ld {
        uint32_t w[R];
        uint32_t sc[R];
        float4 a[4];
    };
    auto load = [&](int k0, Ld& b) {
#pragma unroll
        for (int r = 0; r < R; ++r) b.w[r] = *reinterpret_cast<const uint32_t*>(wrow[r] + (uint32_t)k0 / 2);
        const uint32_t so = 2 * (uint32_t)(k0 / g);
#pragma unroll
        for (int r = 0; r < R; ++r)
            b.sc[r] = *reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint8_t*>(srow[r]) + so);
        const float4* ap = reinterpret_cast<const float4*>(ar + k0);
#pragma unroll
        for (int i = 0; i < 4; ++i) b.a[i] = ap[i];
    };
    auto issued = [] {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };
    float c[R];
    auto chunk = [&](const Ld& b) {
        float wv[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            wv[r] = (float)(int)__builtin_amdgcn_sbfe((int)b.w[r], sh, 4) * h2f((uint16_t)b.sc[r]);
        const float av[16] = {b.a[0].x, b.a[0].y, b.a[0].z, b.a[0].w, b.a[1].x, b.a[1].y, b.a[1].z, b.a[1].w,
                              b.a[2].x, b.a[2].y, b.a[2].z, b.a[2].w, b.a[3].x, b.a[3].y, b.a[3].z, b.a[3].w};
        dpp_chain8<0>(c, wv, av[0]); dpp_chain8<1>(c, wv, av[1]); dpp_chain8<2>(c, wv, av[2]);
        dpp_chain8<3>(c, wv, av[3]); dpp_chain8<4>(c, wv, av[4]); dpp_chain8<5>(c, wv, av[5]);
        dpp_chain8<6>(c, wv, av[6]); dpp_chain8<7>(c, wv, av[7]); dpp_chain8<8>(c, wv, av[8]);
        dpp_chain8<9>(c, wv, av[9]); dpp_chain8<10>(c, wv, av[10]); dpp_chain8<11>(c, wv, av[11]);
        dpp_chain8<12>(c, wv, av[12]); dpp_chain8<13>(c, wv, av[13]); dpp_chain8<14>(c, wv, av[14]);
        dpp_chain8<15>(c, wv, av[15]);
    };
    const int P = rows * 16;  // (row, token) pairs: pair p = (row p / 16, token p % 16)
    float sum[(ND * R * 16 + 64 * NW - 1) / (64 * NW)];
    constexpr int PPT = (ND * R * 16 + 64 * NW - 1) / (64 * NW);  // pairs a thread at most
#pragma unroll
    for (int i = 0; i < PPT; ++i) sum[i] = 0.0f;
    Ld b0, b1;
    load(chunk_k(0, 0), b0);
    for (int s = 0; s < nsl; ++s) {
        const int blk = s * BP + ph;
        const int nq = blk < nb ? min(16, (K - blk * MM_KC) / 16) : 16;  // past the end: any 16, unused
#pragma unroll
        for (int r = 0; r < R; ++r) c[r] = 0.0f;
        // chunks in pairs (K % 32 == 0: every block has an even count); the
        // last pair's second load is the next slice's first chunk
        for (int q = 0; q < nq; q += 2) {
            load(chunk_k(s, q + 1), b1);
            issued();
            chunk(b0);
            load(q + 2 < nq ? chunk_k(s, q + 2) : chunk_k(s + 1, 0), b0);
            issued();
            chunk(b1);
        }
        float* tbs = tb[s & 1];
#pragma unroll
        for (int r = 0; r < R; ++r) tbs[((rs * R + r) * 16 + t) * TS + ph] = blk < nb ? c[r] : 0.0f;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int p = tid + 64 * NW * i;
            if (p < P)
                for (int j = 0; j < BP; ++j) sum[i] = sum[i] + tbs[p * TS + j];
        }
    }
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
        const int p = tid + 64 * NW * i;
        const int row = blockIdx.x * rows + p / 16, tok = m0 + p % 16;
        if (p < P && row < N && tok < M) out[(size_t)tok * N + row] = sum[i];
    }
}

// The activation layout of i4_rows_dpp: the 16 token rows interleaved by
// k-quads, a4[64 (k / 4) + 4 t + k % 4] = a[t][k] (rows t >= M zero), so
// that the 16 token lanes of a DPP row read 256 contiguous bytes a load.
__global__ void rows_to_a4_kernel(const float* __restrict__ a, int M, int K, float* __restrict__ a4) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;  // float4 i of a4: k-quad i / 16, token i % 16
    const int kq = i >> 4, t = i & 15;
    if (kq >= K / 4) return;
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (t < M) v = *reinterpret_cast<const float4*>(a + (size_t)t * K + 4 * kq);
    reinterpret_cast<float4*>(a4)[i] = v;
}

// M independent rows (M <= 16), each in the M == 1 order (i4_dot_avx2),
// with the weights broadcast across tokens: lane 16 d + t of a wave is token
// t in DPP row d, and the workgroup's ND = 4 NW DPP rows D = 4 wave + d take
// a slice of 2 ND groups in two rounds (groups 2 ND s + ND i + D, i = 0, 1).
// A lane holds its token's 32 activations of the current 32-unit (read from
// the a4 layout) and, for each of the workgroup's R weight rows, the packed
// word t & 3 of the unit, whose nibbles t >> 2 and 4 + (t >> 2) become its
// two f32 weight registers (dpp_fma16): each activation register serves R
// rows and each weight register 16 tokens.  A group's term scale * gsum goes
// to LDS (+0 for the groups past the end, which the running sum absorbs
// exactly: it is never -0); after the slice's one barrier the lane of (row,
// token) adds the slice's 2 ND terms to its running sum in group order (two
// term buffers, so the next slice's writes never meet this slice's reads).
// Activations and scales are loaded one step ahead, weights two.  Needs
// K % (32 G4) == 0 and a matrix under 4 GB (32-bit offsets from each row's
// base).
template <int G4, int R, int NW>
__global__ __launch_bounds__(64 * NW) void i4_rows_dpp(const uint8_t* __restrict__ packed,
                                                       const uint16_t* __restrict__ scale, int N, int K,
                                                       const float* __restrict__ a4, int M, float* __restrict__ out) {
    static_assert(G4 == 1 || G4 == 2, "a group is one or two 32-units");
    constexpr int ND = 4 * NW;                 // DPP rows
    constexpr int GPS = 3 - G4;                // groups a DPP row takes a slice (two steps a slice)
    constexpr int SG = ND * GPS;               // groups a slice
    constexpr int TS = SG + 1;                 // term row stride (floats), odd: conflict-free reads
    constexpr int L = (16 * R + NW - 1) / NW;  // serial lanes a wave
    static_assert(L <= 64, "one (row, token) pair a lane");
    __shared__ float tb[2][16 * R][TS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t = lane & 15, D = 4 * wave + (lane >> 4);
    const int ng = K / (32 * G4), r0 = blockIdx.x * R;
    const int nst = (ng + SG - 1) / SG * 2;  // unit steps: two a slice
    const int sh = 4 * (t >> 2);
    const size_t pitch = (size_t)K / 2;
    const uint8_t* wrow[R];
    const uint16_t* srow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const size_t row = (size_t)min(r0 + r, N - 1);  // clamped: loads stay unconditional
        wrow[r] = packed + row * pitch;
        srow[r] = scale + row * ng;
    }
    const float* at = a4 + 4 * t;
    // serial lane: pair p = wave L + lane -> (row p >> 4, token p & 15)
    const int p = wave * L + lane;
    const bool ser = lane < L && p < 16 * R;
    float sum = 0.0f;
    struct WB {
        uint32_t w[R];
    };
    struct AB {
        float4 a[8];
        uint32_t sc[R];
    };
    // step j: slice j / 2; with G4 == 1 round j % 2 of the slice, with G4 == 2
    // unit j % 2 of the DPP row's one group
    auto group_of = [&](int j) { return (j >> 1) * SG + (G4 == 1 ? (j & 1) * ND : 0) + D; };
    auto unit_of = [&](int j, int gi) { return min(gi, ng - 1) * G4 + (G4 == 2 ? (j & 1) : 0); };
    auto load_w = [&](int j, WB& b) {
        const uint32_t wo = (uint32_t)unit_of(j, group_of(j)) * 16 + 4 * (t & 3);
#pragma unroll
        for (int r = 0; r < R; ++r) b.w[r] = *reinterpret_cast<const uint32_t*>(wrow[r] + wo);
    };
    auto load_a = [&](int j, AB& b) {
        const int gi = group_of(j);
        const float* ap = at + (size_t)unit_of(j, gi) * 512;
#pragma unroll
        for (int i = 0; i < 8; ++i) b.a[i] = *reinterpret_cast<const float4*>(ap + 64 * i);
        const uint32_t so = 2 * (uint32_t)min(gi, ng - 1);
#pragma unroll
        for (int r = 0; r < R; ++r)
            b.sc[r] = *reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint8_t*>(srow[r]) + so);
    };
    float l[R][8];  // each group's chains start with a product (dpp_fma16<., true>)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int q = 0; q < 8; ++q) l[r][q] = 0.0f;  // defined inputs for the first asm
    // ODD: the slice's second step, which ends every chain and the slice
    auto step = [&](auto odd, int j, const WB& wb, const AB& ab) {
        constexpr bool O = decltype(odd)::value;
        constexpr bool START = G4 == 1 || !O;
        float av[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            av[4 * i] = ab.a[i].x;
            av[4 * i + 1] = ab.a[i].y;
            av[4 * i + 2] = ab.a[i].z;
            av[4 * i + 3] = ab.a[i].w;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float w0 = (float)(int)__builtin_amdgcn_sbfe((int)wb.w[r], sh, 4);
            const float w1 = (float)(int)__builtin_amdgcn_sbfe((int)wb.w[r], sh + 16, 4);
            dpp_fma16<0, START>(l[r], w0, av);
            dpp_fma16<1, START>(l[r], w1, av);
        }
        if constexpr (G4 == 2 && !O) return;  // the group goes on in the odd step
        float(&tbs)[16 * R][TS] = tb[(j >> 1) & 1];
        const int gi = group_of(j);
        const int col = gi - (j >> 1) * SG;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float q0 = l[r][0] + l[r][4], q1 = l[r][1] + l[r][5], q2 = l[r][2] + l[r][6],
                        q3 = l[r][3] + l[r][7];
            const float term = h2f((uint16_t)ab.sc[r]) * ((q0 + q2) + (q1 + q3));
            tbs[r * 16 + t][col] = gi < ng ? term : 0.0f;
        }
        if constexpr (!O) return;
        __syncthreads();
        if (ser) {
            float v[SG];
#pragma unroll
            for (int i = 0; i < SG; ++i) v[i] = tbs[p][i];
#pragma unroll
            for (int i = 0; i < SG; ++i) sum = sum + v[i];
        }
    };
    using T = std::true_type;
    using F = std::false_type;
    // The loads are unconditional (past the end: the last step again), so
    // the wait for a step's data never covers a later one's, and fenced so
    // that they issue before the step they run ahead of.
    auto issued = [] {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };
    WB wc, wn, w2;
    AB a0, a1;
    load_w(0, wc);
    load_a(0, a0);
    load_w(1, wn);
    for (int j = 0; j < nst; j += 2) {
        load_w(min(j + 2, nst - 1), w2);
        load_a(j + 1, a1);
        issued();
        step(F{}, j, wc, a0);
        load_w(min(j + 3, nst - 1), wc);
        load_a(min(j + 2, nst - 1), a0);
        issued();
        step(T{}, j + 1, wn, a1);
        wn = wc;
        wc = w2;
    }
    if (ser) {
        const int pr = p >> 4, pt = p & 15;
        if (pt < M && r0 + pr < N) out[(size_t)pt * N + r0 + pr] = sum;
    }
}

// M > 1: dequantise w = s4 * scale (f32, exact) and sum in a.dot's order
// (MM_KC-long k blocks, each an FMA chain from +0, added in order).  One
// thread per column j and
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
    float acc[MT], tot[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) tot[m] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += MM_KC) {
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
        for (int kk = k0; kk < min(K, k0 + MM_KC); ++kk) {
            const uint8_t byte = prow[kk >> 1];
            const int v = (kk & 1) ? (byte >> 4) : (byte & 0x0F);
            const float w = (float)((int)((uint32_t)v << 28) >> 28) * h2f(srow[kk / g]);
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

// The same chain with one thread per (column j, token row blockIdx.y), for
// K % 32 == 0, g % 32 == 0 and 16-byte aligned activation rows: the thread
// reads its packed row 32 nibbles (16 bytes) at a time and the token's 32
// activations (uniform across the workgroup) with them, one chunk ahead of
// the chain, so the FMA chain is the only serial part.  The order per output
// is i4_gemm_rows' (a.dot's blocks over kk, w = s4 * scale), bit for bit.
__global__ __launch_bounds__(256) void i4_rows_chain(const uint8_t* __restrict__ packed,
                                                     const uint16_t* __restrict__ scale, int N, int K, int g,
                                                     const float* __restrict__ a, float* __restrict__ out) {
    const int j = blockIdx.x * 256 + threadIdx.x, m = blockIdx.y;
    const int jj = min(j, N - 1);  // clamped: the loads stay unconditional, the store is guarded
    const int nc = K / 32, ng = K / g;
    const uint4* prow = reinterpret_cast<const uint4*>(packed + (size_t)jj * (K / 2));
    const uint16_t* srow = scale + (size_t)jj * ng;
    const float4* arow = reinterpret_cast<const float4*>(a + (size_t)m * K);
    struct Chunk {
        uint4 w;
        float s;
        float4 av[8];
    };
    auto ld = [&](Chunk& c, int i) {
        c.w = prow[i];
        c.s = h2f(srow[(32 * i) / g]);
#pragma unroll
        for (int u = 0; u < 8; ++u) c.av[u] = arow[8 * i + u];
    };
    float acc = 0.0f;
    auto chain = [&](const Chunk& c) {
        const uint32_t ws[4] = {c.w.x, c.w.y, c.w.z, c.w.w};
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
            const float x[8] = {c.av[2 * c4].x, c.av[2 * c4].y, c.av[2 * c4].z, c.av[2 * c4].w,
                                c.av[2 * c4 + 1].x, c.av[2 * c4 + 1].y, c.av[2 * c4 + 1].z, c.av[2 * c4 + 1].w};
#pragma unroll
            for (int q = 0; q < 8; ++q) acc = __builtin_fmaf(x[q], s4f(ws[c4], q) * c.s, acc);
        }
    };
    // a.dot's blocks: MM_KC / 32 chunks (an even count) each, so a block
    // starts on an even chunk, where the running block sum is folded in
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

constexpr float XMAX4 = 8323072.0f;  // 127 * 2^16

// Sign-extend the 8 nibbles of w (k = 0..7, low nibble first) into int8:
// lo = bytes for k = 0,2,4,6, hi = k = 1,3,5,7.  Per byte, with y = x ^ 8:
// ((y + 0x78) ^ 0x80) == x as a signed nibble, and y + 0x78 <= 0x87 never
// carries into the next byte.
__device__ __forceinline__ void nib_unpack(uint32_t w, uint32_t& lo, uint32_t& hi) {
    const uint32_t y = w ^ 0x88888888u;
    lo = ((y & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
    hi = (((y >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
}

// Activation digits, four threads (chunks q = 0..3 of 8 k) per (token m <
// 4*MT4, group g < 4*ng4).  The A operand of token group tg = m/4 and group
// g = 4*g4 + gi is, for lane l, the 8 bytes at ((tg*ng4 + g4)*64 + l)*32 +
// 8*gi (a lane's 4 groups of a quad are one 32-byte run); lane
// 16q + 4(m%4) + d holds digit d of token m at k = 8q + {0,2,4,6,1,3,5,7}
// (the nibble order of the unpacked weights), lane 16q + 4(m%4) + 3 is zero.
// so[(m*ng4 + g4)*4 + gi] = s, -1 for a group that takes the exact path, 0
// for padding tokens and groups.
__global__ void i4_digits_kernel(const float* __restrict__ a, int M, int Mp, int K, int ng4,
                                 uint8_t* __restrict__ adig, float* __restrict__ so_out) {
    const int ng = K / 32, ngp = 4 * ng4;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    const int mg = idx >> 2, q = idx & 3;  // the 4 threads of (m, g) are adjacent lanes
    const bool act = mg < Mp * ngp;
    const int m = act ? mg / ngp : 0, g = act ? mg % ngp : 0;
    const bool real = act && m < M && g < ng;
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (real) {
        const float4* ap = reinterpret_cast<const float4*>(a + (size_t)m * K + (size_t)g * 32 + 8 * q);
        const float4 x0 = ap[0], x1 = ap[1];
        v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
        v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
    }
    float mx = 0.0f;
    int nf = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        nf |= !(fabsf(v[k]) <= 3.0e38f);
        mx = fmaxf(mx, fabsf(v[k]));
    }
    mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
    nf |= __shfl_xor(nf, 1, 64);
    nf |= __shfl_xor(nf, 2, 64);
    if (!act) return;
    // |group sum| <= 32 * 8 * mx stays finite for s <= 1e28
    const float s = mx > 0.0f ? mx / XMAX4 : 1.0f;
    const bool ok = real && !nf && s >= 1.0e-30f && s <= 1.0e28f;
    uint32_t dw[3][2] = {{0, 0}, {0, 0}, {0, 0}};
    if (ok) {
        const float r = 1.0f / s;  // any rounding of a / s keeps |a - s X| <= ~s/2
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float xf = rintf(v[j] * r);
            xf = fminf(fmaxf(xf, -XMAX4), XMAX4);
            const int X = (int)xf;
            const int d0 = (int)(int8_t)(X & 0xFF);
            const int X1 = (X - d0) >> 8;
            const int d1 = (int)(int8_t)(X1 & 0xFF);
            const int d2 = (X1 - d1) >> 8;
            const int p = (j & 1) ? 4 + (j >> 1) : (j >> 1);  // byte within the lane's 8
            const int wsel = p >> 2, sh = 8 * (p & 3);
            dw[0][wsel] |= (uint32_t)(d2 & 0xFF) << sh;
            dw[1][wsel] |= (uint32_t)(d1 & 0xFF) << sh;
            dw[2][wsel] |= (uint32_t)(d0 & 0xFF) << sh;
        }
    }
    const int g4 = g >> 2, gi = g & 3;
    uint8_t* blk = adig + ((size_t)(m >> 2) * ng4 + g4) * 64 * 32 + 8 * gi;
    const int l0 = 16 * q + 4 * (m & 3);
#pragma unroll
    for (int d = 0; d < 3; ++d)
        *reinterpret_cast<uint2*>(blk + (l0 + d) * 32) = make_uint2(dw[d][0], dw[d][1]);
    *reinterpret_cast<uint2*>(blk + (l0 + 3) * 32) = make_uint2(0u, 0u);
    if (q == 0) so_out[((size_t)m * ng4 + g4) * 4 + gi] = real ? (ok ? s : -1.0f) : 0.0f;
}

// acc plus one group of a (token, weight row) in the reference arm's own
// order, for activations the digits cannot carry (non-finite or extreme):
// M == 1: scale * i4_dot_avx2 group sum; M > 1: a * (s4 * scale), k ascending.
template <bool INL = false>
__device__ __attribute__((noinline)) float exact_group(float acc, const uint8_t* wrow, const float* ag,
                                                       float sc, bool m1);
template <>
__device__ __attribute__((noinline)) float exact_group<false>(float acc, const uint8_t* wrow, const float* ag,
                                                              float sc, bool m1);
__device__ __forceinline__ float exact_group_body(float acc, const uint8_t* wrow, const float* ag,
                                                  float sc, bool m1) {
    const uint4 wr = *reinterpret_cast<const uint4*>(wrow);
    if (m1) return acc + sc * group_avx2(wr, ag);
    const uint32_t ws[4] = {wr.x, wr.y, wr.z, wr.w};
    float e = 0.0f;
    for (int k = 0; k < 32; ++k) e = __builtin_fmaf(ag[k], s4f(ws[k >> 3], k & 7) * sc, e);
    return acc + e;
}
template <>
__device__ __attribute__((noinline)) float exact_group<false>(float acc, const uint8_t* wrow, const float* ag,
                                                              float sc, bool m1) {
    return exact_group_body(acc, wrow, ag, sc, m1);
}

// Dot of one group for the MT4 token groups of a wave, acc += scale * gsum.
template <int MT4, bool INL = false>
__device__ __forceinline__ void group_mfma(float (&acc)[MT4], uint32_t wd, float sc, const long* aop,
                                           const float* so, int g, int row, int N, int K, int M,
                                           const uint8_t* __restrict__ raw, const float* __restrict__ a,
                                           int ml) {
    uint32_t lo, hi;
    nib_unpack(wd, lo, hi);
    const long bop = (long)(((unsigned long long)hi << 32) | lo);
#pragma unroll
    for (int t = 0; t < MT4; ++t) {
        const v4i cr = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop[t], bop, v4i{0, 0, 0, 0}, 0, 0, 0);
        if (__builtin_amdgcn_ballot_w64(so[t] < 0.0f)) {  // wave-uniform, rare
            if (so[t] < 0.0f && row < N) {
                const uint8_t* wr = raw + (size_t)row * (K / 2) + (size_t)g * 16;
                const float* ag = a + (size_t)(4 * t + ml) * K + (size_t)g * 32;
                if constexpr (INL) acc[t] = exact_group_body(acc[t], wr, ag, sc, M == 1);
                else acc[t] = exact_group<false>(acc[t], wr, ag, sc, M == 1);
                continue;
            }
        }
        const float gs = so[t] * ((float)cr[0] * 65536.0f + ((float)cr[1] * 256.0f + (float)cr[2]));
        acc[t] = acc[t] + sc * gs;
    }
}

// int4 x f32 on the int8 MFMA.  A workgroup of KS waves covers 16-row
// blocks rb = blockIdx.x, + gridDim.x, ...; wave ks owns the ks-th part (at
// most GQ group quads) of K.  It loads that part's activation operands once
// (only the lanes whose A rows carry a token's digit; with M == 1 the digit
// scales are wave-uniform) and keeps them in registers; per block it issues
// all of the part's weight loads at once.  The KS partial sums of a block are
// added in part order through LDS.  MT4 = token groups of 4 (M <= 4 * MT4).
template <int MT4, int KS, int GQ, bool M1>
__global__ __launch_bounds__(64 * KS) void i4_mfma_kernel(
    const uint8_t* __restrict__ q4m, const uint16_t* __restrict__ s4m,
    const uint8_t* __restrict__ raw, const float* __restrict__ a,
    const uint8_t* __restrict__ adig, const float* __restrict__ sog, int M, int K,
    int N, int ng4, float* __restrict__ out) {
    __shared__ float red[2][KS][MT4][64];
    const int lane = threadIdx.x & 63;
    const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nrb = (N + 15) / 16, ng = K / 32;
    const int q0 = (int)((long)ng4 * ks / KS), q1 = (int)((long)ng4 * (ks + 1) / KS);
    const int col = lane & 15, ml = M1 ? 0 : lane >> 4;
    // resident activation operands and digit scales of this part
    long ao[GQ][4][MT4];
    float sv[GQ][4][MT4];
#pragma unroll
    for (int i = 0; i < GQ; ++i)
#pragma unroll
        for (int t = 0; t < MT4; ++t) {
            const int mt = M1 ? 1 : min(M - 4 * t, 4);  // tokens in this token group
            const bool need = ((col >> 2) < mt) && ((col & 3) < 3) && q0 + i < q1;
            uint4 h0 = make_uint4(0, 0, 0, 0), h1 = make_uint4(0, 0, 0, 0);
            if (need) {
                const uint4* ap = reinterpret_cast<const uint4*>(adig + (((size_t)t * ng4 + q0 + i) * 64 + lane) * 32);
                h0 = ap[0];
                h1 = ap[1];
            }
            ao[i][0][t] = (long)(((unsigned long long)h0.y << 32) | h0.x);
            ao[i][1][t] = (long)(((unsigned long long)h0.w << 32) | h0.z);
            ao[i][2][t] = (long)(((unsigned long long)h1.y << 32) | h1.x);
            ao[i][3][t] = (long)(((unsigned long long)h1.w << 32) | h1.z);
            float4 s4v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (q0 + i < q1 && (M1 || 4 * t + ml < M))
                s4v = *reinterpret_cast<const float4*>(sog + ((size_t)(4 * t + ml) * ng4 + q0 + i) * 4);
            sv[i][0][t] = s4v.x; sv[i][1][t] = s4v.y; sv[i][2][t] = s4v.z; sv[i][3][t] = s4v.w;
        }

    int buf = 0;
    for (int rb = blockIdx.x; rb < nrb; rb += gridDim.x) {  // workgroup-uniform
        const int row = 16 * rb + col;
        uint4 wq[GQ];
        uint2 wsc[GQ];
#pragma unroll
        for (int i = 0; i < GQ; ++i)
            if (q0 + i < q1) {
                const size_t blk = (size_t)rb * ng4 + q0 + i;
                wq[i] = *reinterpret_cast<const uint4*>(q4m + (blk * 64 + lane) * 16);
                wsc[i] = *reinterpret_cast<const uint2*>(s4m + (blk * 16 + col) * 4);
            }
        float acc[MT4];
#pragma unroll
        for (int t = 0; t < MT4; ++t) acc[t] = 0.0f;
#pragma unroll
        for (int i = 0; i < GQ; ++i) {
            if (q0 + i >= q1) continue;  // no break, so the loop unrolls
            const uint32_t wd[4] = {wq[i].x, wq[i].y, wq[i].z, wq[i].w};
            const uint32_t sd[2] = {wsc[i].x, wsc[i].y};
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                const int g = 4 * (q0 + i) + gi;
                if (g >= ng) continue;  // zero padding groups of the last quad
                const float sc = h2f((uint16_t)(sd[gi >> 1] >> (16 * (gi & 1))));
                group_mfma<MT4>(acc, wd[gi], sc, ao[i][gi], sv[i][gi], g, row, N, K, M, raw, a, ml);
            }
        }
        if (KS == 1) {
#pragma unroll
            for (int t = 0; t < MT4; ++t) {
                const int m = 4 * t + (lane >> 4);
                if (m < M && row < N) out[(size_t)m * N + row] = acc[t];
            }
            continue;
        }
        // parts of this block through LDS; the two buffers alternate between
        // consecutive blocks, so one barrier per block suffices
#pragma unroll
        for (int t = 0; t < MT4; ++t) red[buf][ks][t][lane] = acc[t];
        __syncthreads();
        if (ks == 0) {
#pragma unroll
            for (int t = 0; t < MT4; ++t) {
                float v = red[buf][0][t][lane];
#pragma unroll
                for (int q = 1; q < KS; ++q) v = v + red[buf][q][t][lane];
                const int m = 4 * t + (lane >> 4);
                if (m < M && row < N) out[(size_t)m * N + row] = v;
            }
        }
        buf ^= 1;
    }
}

// Fused M <= 4 path (one launch, one 16-row block per workgroup).  The
// workgroup first writes the activation digits of all K into LDS in compact
// form: for group g < 4*ng4 (groups past K are zero), chunk q (k = 8q..8q+7),
// token m and digit d, the 8 bytes at (((g*4 + q)*M + m)*3 + d)*8, plus
// so[g*M + m] (-1: a group the digits cannot carry), and one zero slot.
// Then its KS waves, wave ks owning the ks-th part (at most GQ quads) of K,
// issue all of their part's weight loads at once (before the digit pass, so
// the latencies overlap); the A operand of a group is an 8-byte LDS read (the
// zero slot for lanes whose A row 4m + d has m >= M or d == 3).  The KS
// partial sums are added in part order through LDS.
template <int M, int KS, int GQ>
__global__ __launch_bounds__(64 * KS) void i4_fused_kernel(
    const uint8_t* __restrict__ q4m, const uint16_t* __restrict__ s4m,
    const uint8_t* __restrict__ raw, const float* __restrict__ a, int K, int N,
    int ng4, float* __restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int ng = K / 32, ngp = 4 * ng4;
    uint2* adl = reinterpret_cast<uint2*>(smem);  // [ngp*4*M*3 + 1 zero slot]
    const int zslot = ngp * 4 * M * 3;
    float* sol = reinterpret_cast<float*>(smem + (size_t)(zslot + 2) * 8);  // [ngp*M]
    float* red = sol + ((ngp * M + 3) & ~3);                                // [KS][64]
    const int tid = threadIdx.x, lane = tid & 63;
    const int ks = __builtin_amdgcn_readfirstlane(tid >> 6);

    // the weight loads of this wave's part do not depend on the digits: issue
    // them first, so their latency overlaps the digit pass
    const int rb = blockIdx.x;
    const int q0 = (int)((long)ng4 * ks / KS), q1 = (int)((long)ng4 * (ks + 1) / KS);
    const int nq = q1 - q0;  // <= GQ
    const int col = lane & 15, ml = lane >> 4;
    uint4 wq[GQ];
    uint2 wsc[GQ];
#pragma unroll
    for (int i = 0; i < GQ; ++i)
        if (i < nq) {
            const size_t blk = (size_t)rb * ng4 + q0 + i;
            wq[i] = *reinterpret_cast<const uint4*>(q4m + (blk * 64 + lane) * 16);
            wsc[i] = *reinterpret_cast<const uint2*>(s4m + (blk * 16 + col) * 4);
        }

    // 1. digits: four adjacent threads per (m, g), one chunk q each; a
    //    thread's items of a pass are loaded together, then digitised
    constexpr int IPT = 2;
    const int nitems = 4 * M * ngp;
    if (tid == 0) adl[zslot] = make_uint2(0u, 0u);
    for (int base = 0; base < nitems; base += 64 * KS * IPT) {  // uniform trip count
        float v[IPT][8];
#pragma unroll
        for (int it = 0; it < IPT; ++it) {
            const int idx = base + it * 64 * KS + tid;
            const int mg = idx >> 2, q = idx & 3;
            const int m = mg / ngp, g = mg % ngp;
#pragma unroll
            for (int k = 0; k < 8; ++k) v[it][k] = 0.0f;
            if (mg < M * ngp && g < ng) {
                const float4* ap = reinterpret_cast<const float4*>(a + (size_t)m * K + (size_t)g * 32 + 8 * q);
                const float4 x0 = ap[0], x1 = ap[1];
                v[it][0] = x0.x; v[it][1] = x0.y; v[it][2] = x0.z; v[it][3] = x0.w;
                v[it][4] = x1.x; v[it][5] = x1.y; v[it][6] = x1.z; v[it][7] = x1.w;
            }
        }
#pragma unroll
        for (int it = 0; it < IPT; ++it) {
            const int idx = base + it * 64 * KS + tid;
            const int mg = idx >> 2, q = idx & 3;
            const bool act = mg < M * ngp;
            const int m = act ? mg / ngp : 0, g = act ? mg % ngp : 0;
            float mx = 0.0f;
            int nf = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                nf |= !(fabsf(v[it][k]) <= 3.0e38f);
                mx = fmaxf(mx, fabsf(v[it][k]));
            }
            mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
            nf |= __shfl_xor(nf, 1, 64);
            nf |= __shfl_xor(nf, 2, 64);
            if (!act) continue;
            // |group sum| <= 32 * 8 * mx stays finite for s <= 1e28
            const float sg = mx > 0.0f ? mx / XMAX4 : 1.0f;
            const bool ok = !nf && sg >= 1.0e-30f && sg <= 1.0e28f;
            uint32_t dw[3][2] = {{0, 0}, {0, 0}, {0, 0}};
            if (ok) {
                const float r = 1.0f / sg;  // any rounding of a / s keeps |a - s X| <= ~s/2
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    float xf = rintf(v[it][j] * r);
                    xf = fminf(fmaxf(xf, -XMAX4), XMAX4);
                    const int X = (int)xf;
                    const int d0 = (int)(int8_t)(X & 0xFF);
                    const int X1 = (X - d0) >> 8;
                    const int d1 = (int)(int8_t)(X1 & 0xFF);
                    const int d2 = (X1 - d1) >> 8;
                    const int p = (j & 1) ? 4 + (j >> 1) : (j >> 1);
                    const int wsel = p >> 2, sh = 8 * (p & 3);
                    dw[0][wsel] |= (uint32_t)(d2 & 0xFF) << sh;
                    dw[1][wsel] |= (uint32_t)(d1 & 0xFF) << sh;
                    dw[2][wsel] |= (uint32_t)(d0 & 0xFF) << sh;
                }
            }
#pragma unroll
            for (int d = 0; d < 3; ++d) adl[((g * 4 + q) * M + m) * 3 + d] = make_uint2(dw[d][0], dw[d][1]);
            if (q == 0) sol[g * M + m] = g < ng ? (ok ? sg : -1.0f) : 0.0f;
        }
    }
    __syncthreads();

    // 2. this workgroup's 16-row block, the groups of the wave's part in order
    const int am = col >> 2, ad = col & 3;  // A row of this lane: token am, digit ad
    const int row = 16 * rb + col;
    const int mtok = ml < M ? ml : 0;       // token of this lane's result (lanes >= M: junk)
    // LDS slot of the lane's A operand for group g: abase + g * 12M (the zero
    // slot, stride 0, for lanes without a digit row)
    const bool arow = am < M && ad < 3;
    const int abase = arow ? (ml * M + am) * 3 + ad : zslot;
    const int astep = arow ? 12 * M : 0;
    const int g0 = 4 * q0;
    // any group of the part that the digits cannot carry?  (wave-uniform)
    int xg = 0;
    for (int i = lane; i < 4 * nq * M; i += 64) xg |= sol[g0 * M + i] < 0.0f;
    float acc = 0.0f;
    if (__builtin_amdgcn_ballot_w64(xg) == 0) {
        // fast path: straight-line digit MFMAs, four groups per weight quad
#pragma unroll
        for (int i = 0; i < GQ; ++i) {
            if (i >= nq) continue;  // wave-uniform; no break, so the loop unrolls
            const int gq = 4 * (q0 + i);
            const uint32_t wd[4] = {wq[i].x, wq[i].y, wq[i].z, wq[i].w};
            v4i cr[4];
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                uint32_t lo, hi;
                nib_unpack(wd[gi], lo, hi);
                const long bop = (long)(((unsigned long long)hi << 32) | lo);
                const uint2 av = adl[abase + (gq + gi) * astep];
                const long aop = (long)(((unsigned long long)av.y << 32) | av.x);
                cr[gi] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, v4i{0, 0, 0, 0}, 0, 0, 0);
            }
            const uint32_t sd[2] = {wsc[i].x, wsc[i].y};
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                const float sgi = sol[(gq + gi) * M + mtok];
                const float sc = h2f((uint16_t)(sd[gi >> 1] >> (16 * (gi & 1))));
                const float gs = sgi * ((float)cr[gi][0] * 65536.0f + ((float)cr[gi][1] * 256.0f + (float)cr[gi][2]));
                acc = acc + sc * gs;
            }
        }
    } else {
        // some group needs the exact path: a compact loop over the part, the
        // weights read again from global memory
        for (int g = g0; g < min(4 * q1, ng); ++g) {
            const size_t blk = (size_t)rb * ng4 + (g >> 2);
            const uint32_t wd = *reinterpret_cast<const uint32_t*>(q4m + (blk * 64 + lane) * 16 + 4 * (g & 3));
            const uint16_t sh = s4m[(blk * 16 + col) * 4 + (g & 3)];
            const uint2 av = adl[abase + g * astep];
            const long aop[1] = {(long)(((unsigned long long)av.y << 32) | av.x)};
            const float so[1] = {sol[g * M + mtok]};
            float a1[1] = {acc};
            group_mfma<1, true>(a1, wd, h2f(sh), aop, so, g, row, N, K, M, raw, a, ml);
            acc = a1[0];
        }
    }
    if (KS == 1) {
        if (ml < M && row < N) out[(size_t)ml * N + row] = acc;
        return;
    }
    red[ks * 64 + lane] = acc;
    __syncthreads();
    if (ks == 0) {
        float v = red[lane];
#pragma unroll
        for (int q = 1; q < KS; ++q) v = v + red[q * 64 + lane];
        if (ml < M && row < N) out[(size_t)ml * N + row] = v;
    }
}

// LDS bytes of the fused path (compact digits + zero slot + scales + reduction).
size_t fused_lds(size_t m, size_t k, int ks) {
    const size_t ngp = 4 * ((k / 32 + 3) / 4);
    return (ngp * 4 * m * 3 + 2) * 8 + ((ngp * m + 3) & ~(size_t)3) * 4 + (size_t)ks * 64 * 4;
}

// (N, K/2) packed nibbles + (N, ng) f16 scales -> the MFMA layout: for row
// block rb and group quad g4, lane l = 16q + r holds, for groups 4g4..4g4+3,
// the 4 bytes of row 16rb + r at k = 8q..8q+7 of each group (16 bytes at
// ((rb*ng4 + g4)*64 + l)*16), and the scales (rb, g4, r) as 4 halves.
// Rows >= N and groups >= ng are zero.
__global__ void i4_block_kernel(const uint8_t* __restrict__ raw, const uint16_t* __restrict__ sraw,
                                int N, int K, int ng4, uint8_t* __restrict__ q4m,
                                uint16_t* __restrict__ s4m) {
    const int ng = K / 32, nrb = (N + 15) / 16;
    const size_t total = (size_t)nrb * ng4 * 64;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int l = (int)(i % 64);
        const size_t bg = i / 64;
        const int g4 = (int)(bg % ng4), rb = (int)(bg / ng4);
        const int r = l & 15, q = l >> 4, row = 16 * rb + r;
        uint32_t v[4] = {0, 0, 0, 0};
        for (int gi = 0; gi < 4; ++gi) {
            const int g = 4 * g4 + gi;
            if (row < N && g < ng)
                v[gi] = *reinterpret_cast<const uint32_t*>(raw + (size_t)row * (K / 2) + (size_t)g * 16 + 4 * q);
        }
        reinterpret_cast<uint4*>(q4m)[i] = make_uint4(v[0], v[1], v[2], v[3]);
        if (q == 0) {
            for (int gi = 0; gi < 4; ++gi) {
                const int g = 4 * g4 + gi;
                s4m[(bg * 16 + r) * 4 + gi] = (row < N && g < ng) ? sraw[(size_t)row * ng + g] : (uint16_t)0;
            }
        }
    }
}

}  // namespace

static bool mfma_fits(size_t k, size_t m);

static bool fused_fits(size_t k, size_t m);

size_t i4_ws_floats(const Weight& w, size_t m) {
    if (!w.i4_blocked || fused_fits(w.k, m) || !mfma_fits(w.k, m)) return 0;
    const size_t mp = round_up(m, 4), ng4 = (w.k / 32 + 3) / 4;
    return (mp / 4) * ng4 * 64 * 32 / sizeof(float) + mp * ng4 * 4 + 64;  // digits + scales
}

size_t i4_blocked_bytes(size_t n, size_t k) {
    return (n + 15) / 16 * ((k / 32 + 3) / 4) * 1024;
}

hipError_t launch_i4_block(const uint8_t* raw, const uint16_t* sraw, size_t n,
                           size_t k, uint8_t* blk, uint16_t* sblk,
                           hipStream_t s) {
    const int ng4 = (int)((k / 32 + 3) / 4);
    i4_block_kernel<<<dim3(1024), dim3(256), 0, s>>>(raw, sraw, (int)n, (int)k, ng4, blk, sblk);
    return hipGetLastError();
}

template <int MT4, int KS, int GQ>
static hipError_t launch_mfma_t(const Weight& w, size_t m, const float* a, const uint8_t* adig,
                                const float* sog, float* out, hipStream_t s) {
    const size_t ng4 = (w.k / 32 + 3) / 4, nrb = (w.n + 15) / 16;
    // about 8 waves per CU on 256 CUs, the blocks spread evenly
    const size_t want = 2048 / KS;
    const size_t per = (nrb + want - 1) / want;
    const size_t grid = (nrb + per - 1) / per;
    if constexpr (MT4 == 1)
        if (m == 1) {
            i4_mfma_kernel<1, KS, GQ, true><<<dim3((unsigned)grid), dim3(64 * KS), 0, s>>>(
                w.q4, w.s4, w.q4raw, a, adig, sog, (int)m, (int)w.k, (int)w.n, (int)ng4, out);
            return hipGetLastError();
        }
    i4_mfma_kernel<MT4, KS, GQ, false><<<dim3((unsigned)grid), dim3(64 * KS), 0, s>>>(
        w.q4, w.s4, w.q4raw, a, adig, sog, (int)m, (int)w.k, (int)w.n, (int)ng4, out);
    return hipGetLastError();
}

// Group quads per K part (register budget: GQ * 4 * MT4 resident operands).
constexpr int gq_of(int mt4) { return mt4 == 1 ? 9 : (mt4 == 2 ? 5 : 3); }

// KS waves per workgroup, the fewest whose parts hold at most GQ quads.
template <int MT4>
static hipError_t launch_mfma(const Weight& w, size_t m, const float* a, const uint8_t* adig,
                              const float* sog, float* out, hipStream_t s) {
    constexpr int GQ = gq_of(MT4);
    const size_t ng4 = (w.k / 32 + 3) / 4;
    if (ng4 <= GQ) return launch_mfma_t<MT4, 1, GQ>(w, m, a, adig, sog, out, s);
    if (ng4 <= 2 * GQ) return launch_mfma_t<MT4, 2, GQ>(w, m, a, adig, sog, out, s);
    if (ng4 <= 4 * GQ) return launch_mfma_t<MT4, 4, GQ>(w, m, a, adig, sog, out, s);
    if (ng4 <= 8 * GQ) return launch_mfma_t<MT4, 8, GQ>(w, m, a, adig, sog, out, s);
    return hipErrorInvalidValue;  // mfma_fits() sends longer K to the generic path
}

// Shapes the MFMA path takes at m tokens: m <= 16 and K in at most 8 parts.
static bool mfma_fits(size_t k, size_t m) {
    if (m < 1 || m > 16) return false;
    const size_t ng4 = (k / 32 + 3) / 4, mt4 = (m + 3) / 4;
    return ng4 <= 8 * (size_t)gq_of((int)mt4);
}

template <int M, int KS>
static hipError_t launch_fused_t(const Weight& w, const float* a, float* out, hipStream_t s) {
    constexpr int GQ = 9;
    const size_t ng4 = (w.k / 32 + 3) / 4, nrb = (w.n + 15) / 16;
    const size_t lds = fused_lds(M, w.k, KS);
    i4_fused_kernel<M, KS, GQ><<<dim3((unsigned)nrb), dim3(64 * KS), lds, s>>>(
        w.q4, w.s4, w.q4raw, a, (int)w.k, (int)w.n, (int)ng4, out);
    return hipGetLastError();
}

// KS waves per workgroup: parts of at most 5 group quads (more waves per CU
// to overlap the MFMA -> VALU chains), at most 9 when K needs 16 parts.
template <int M>
static hipError_t launch_fused_m(const Weight& w, const float* a, float* out, hipStream_t s) {
    const size_t ng4 = (w.k / 32 + 3) / 4;
    if (ng4 <= 5) return launch_fused_t<M, 1>(w, a, out, s);
    if (ng4 <= 10) return launch_fused_t<M, 2>(w, a, out, s);
    if (ng4 <= 20) return launch_fused_t<M, 4>(w, a, out, s);
    if (ng4 <= 40) return launch_fused_t<M, 8>(w, a, out, s);
    return launch_fused_t<M, 16>(w, a, out, s);
}

// The fused path: M <= 4, K in at most 16 parts of 9 quads, digits within 64 KB of LDS.
static bool fused_fits(size_t k, size_t m) {
    const size_t ng4 = (k / 32 + 3) / 4;
    return m >= 1 && m <= 4 && ng4 <= 144 && fused_lds(m, k, 16) <= 64 * 1024;
}

static hipError_t launch_fused(const Weight& w, size_t m, const float* a, float* out, hipStream_t s) {
    switch (m) {
        case 1: return launch_fused_m<1>(w, a, out, s);
        case 2: return launch_fused_m<2>(w, a, out, s);
        case 3: return launch_fused_m<3>(w, a, out, s);
        default: return launch_fused_m<4>(w, a, out, s);
    }
}

template <int G4, int IPT, int NT>
hipError_t launch_stream_t(const Weight& w, int R, unsigned grid, size_t lds, const float* a, float* out,
                           hipStream_t s) {
    // the attribute once per instantiation, at the full 160 KB (later calls
    // issue the launch only)
    static bool attr = false;
    if (lds > 64 * 1024 && !attr) {
        const hipError_t e = hipFuncSetAttribute((const void*)i4_m1_stream<G4, IPT, NT>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        attr = true;
    }
    i4_m1_stream<G4, IPT, NT><<<dim3(grid), dim3(NT), lds, s>>>(w.q4raw, w.s4raw, (int)w.n, (int)w.k, R, a, out);
    return hipGetLastError();
}

template <int G4, int NT>
hipError_t launch_stream_g(const Weight& w, int ipt, int R, unsigned grid, size_t lds, const float* a, float* out,
                           hipStream_t s) {
    switch (ipt) {
        case 2: return launch_stream_t<G4, 2, NT>(w, R, grid, lds, a, out, s);
        case 4: return launch_stream_t<G4, 4, NT>(w, R, grid, lds, a, out, s);
        case 6: return launch_stream_t<G4, 6, NT>(w, R, grid, lds, a, out, s);
        case 8: return launch_stream_t<G4, 8, NT>(w, R, grid, lds, a, out, s);
        case 12: return launch_stream_t<G4, 12, NT>(w, R, grid, lds, a, out, s);
        default: return launch_stream_t<G4, 16, NT>(w, R, grid, lds, a, out, s);
    }
}

// The streamed M == 1 kernel: rows split evenly over the workgroups (one a
// CU, of 512 threads; more where a thread would hold over 16 items),
// the activation row and the terms within 160 KB of LDS (else
// hipErrorNotSupported).
hipError_t launch_i4_stream(const Weight& w, const float* a, float* out, hipStream_t s) {
    if (w.k % 32 || (w.g != 32 && w.g != 64) || w.k % w.g || w.k > (1u << 24) || w.n > (size_t)INT32_MAX ||
        ((uintptr_t)a & 15))
        return hipErrorNotSupported;
    const size_t ng = w.k / w.g, n = w.n;
    constexpr int nt = 512;  // 8 waves: two a SIMD, one activation row staged a CU
    const size_t nwg = (size_t)device_cus(w.device);
    size_t R = (n + nwg - 1) / nwg;
    if (R * ng > (size_t)nt * 16) R = std::max<size_t>(1, (size_t)nt * 16 / ng);
    const size_t items = R * ng, ipt0 = (items + nt - 1) / nt;
    const int ipt = ipt0 <= 2 ? 2 : ipt0 <= 4 ? 4 : ipt0 <= 6 ? 6 : ipt0 <= 8 ? 8 : ipt0 <= 12 ? 12 : 16;
    if (ipt0 > 16) return hipErrorNotSupported;
    const size_t lds = i4_stream_as_bytes((int)w.k) + (R * ((ng + 3) & ~(size_t)3) + 4) * sizeof(float);
    if (lds > 160 * 1024) return hipErrorNotSupported;
    const unsigned grid = (unsigned)((n + R - 1) / R);
    return w.g == 32 ? launch_stream_g<1, nt>(w, ipt, (int)R, grid, lds, a, out, s)
                     : launch_stream_g<2, nt>(w, ipt, (int)R, grid, lds, a, out, s);
}

// The exact M == 1 kernel when the shape allows it (else hipErrorNotSupported).
hipError_t launch_i4_terms(const Weight& w, const float* a, float* out, hipStream_t s) {
    {
        const hipError_t e = launch_i4_stream(w, a, out, s);
        if (e != hipErrorNotSupported) return e;
    }
    if (w.k % 32 || (w.g != 32 && w.g != 64) || w.k > (size_t)INT32_MAX || w.n > (size_t)INT32_MAX)
        return hipErrorNotSupported;
    const int ng = (int)(w.k / w.g);
    int rb = std::min(64, std::max(1, 8192 / std::max(ng, 1)));
    while (rb > 8 && (w.n + rb - 1) / rb < 512) rb /= 2;
    const size_t cgb = (size_t)rb * ((ng + 3) & ~3) * sizeof(float);
    const size_t asb = (w.k / 32) * 36 * sizeof(float);
    if (cgb + asb > 64 * 1024) return hipErrorNotSupported;
    const unsigned grid = (unsigned)((w.n + rb - 1) / rb);
    if (w.g == 32)
        i4_gemv_terms<1><<<dim3(grid), dim3(256), cgb + asb, s>>>(w.q4raw, w.s4raw, (int)w.n, (int)w.k, rb, a, out);
    else
        i4_gemv_terms<2><<<dim3(grid), dim3(256), cgb + asb, s>>>(w.q4raw, w.s4raw, (int)w.n, (int)w.k, rb, a, out);
    return hipGetLastError();
}

// Whether launch_i4_rows_a4 takes this weight (else launch_i4_m1_rows runs
// the rows one M == 1 launch at a time).
bool i4_rows_a4_ok(const Weight& w) {
    return (w.g == 32 || w.g == 64) && w.k % w.g == 0 && w.k <= (size_t)INT32_MAX &&
           w.n <= (size_t)INT32_MAX && w.n * w.k / 2 < ((size_t)1 << 32);
}

size_t i4_a4_floats(size_t k) { return 16 * k; }

hipError_t launch_rows_to_a4(const float* a, size_t m, size_t k, float* a4, hipStream_t s) {
    const size_t n4 = 4 * k;  // float4 of a4
    rows_to_a4_kernel<<<dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s>>>(a, (int)m, (int)k, a4);
    return hipGetLastError();
}

namespace {
template <int G4, int R>
hipError_t rows_dpp(const Weight& w, int nw, size_t m, const float* a4, float* out, hipStream_t s) {
    const unsigned grid = (unsigned)((w.n + R - 1) / R);
    if (nw == 3)
        i4_rows_dpp<G4, R, 3><<<dim3(grid), dim3(192), 0, s>>>(w.q4raw, w.s4raw, (int)w.n, (int)w.k, a4, (int)m, out);
    else
        i4_rows_dpp<G4, R, 4><<<dim3(grid), dim3(256), 0, s>>>(w.q4raw, w.s4raw, (int)w.n, (int)w.k, a4, (int)m, out);
    return hipGetLastError();
}
}  // namespace

// m <= 16 rows in the a4 layout (launch_rows_to_a4), each in the M == 1
// order.  Workgroups of 3 or 4 waves (12 or 16 DPP rows, whichever leaves
// the fewer idle groups in the last slice; 4 on a tie) and 6 rows (each
// activation register used 6 times) for wide outputs, 4 below 8192 rows,
// where more workgroups matter more (measured on the Gemma-2 2B shapes).
hipError_t launch_i4_rows_a4(const Weight& w, size_t m, const float* a4, float* out, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    if (m > 16 || !i4_rows_a4_ok(w)) return hipErrorNotSupported;
    const size_t ng = w.k / w.g, gps = w.g == 32 ? 2 : 1;  // groups a DPP row takes a slice
    const int nw = (ng + 12 * gps - 1) / (12 * gps) * 12 < (ng + 16 * gps - 1) / (16 * gps) * 16 ? 3 : 4;
    const bool r6 = w.n >= 8192;
    if (w.g == 32) return r6 ? rows_dpp<1, 6>(w, nw, m, a4, out, s) : rows_dpp<1, 4>(w, nw, m, a4, out, s);
    return r6 ? rows_dpp<2, 6>(w, nw, m, a4, out, s) : rows_dpp<2, 4>(w, nw, m, a4, out, s);
}

// m rows, each in the M == 1 order (bit-identical to m launches at M == 1);
// a4 is scratch of i4_a4_floats(K) floats (16-byte aligned).
hipError_t launch_i4_m1_rows(const Weight& w, size_t m, const float* a, float* out, float* a4, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    for (size_t r0 = 0; r0 < m; r0 += 16) {
        const size_t mm = std::min<size_t>(16, m - r0);
        if (a4 && i4_rows_a4_ok(w)) {
            if (hipError_t e = launch_rows_to_a4(a + r0 * w.k, mm, w.k, a4, s)) return e;
            if (hipError_t e = launch_i4_rows_a4(w, mm, a4, out + r0 * w.n, s)) return e;
            continue;
        }
        for (size_t i = r0; i < r0 + mm; ++i)
            if (hipError_t e = launch_i4_exact(w, 1, a + i * w.k, out + i * w.n, s)) return e;
    }
    return hipSuccess;
}

hipError_t launch_i4_exact(const Weight& w, size_t m, const float* a, float* out, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    if (m == 1) {
        const hipError_t e = launch_i4_terms(w, a, out, s);
        if (e != hipErrorNotSupported) return e;
        i4_gemv_generic<<<dim3((unsigned)((w.n + 255) / 256)), dim3(256), 0, s>>>(
            w.q4raw, w.s4raw, (int)w.n, (int)w.k, (int)w.g, a, out);
        return hipGetLastError();
    }
    if (w.k % 32 == 0 && w.g % 16 == 0 && ((uintptr_t)a & 15) == 0 && (m + 15) / 16 <= 65535 &&
        w.k <= (size_t)INT32_MAX && w.n <= (size_t)INT32_MAX && w.n * w.k / 2 < ((size_t)1 << 32)) {
        // workgroups of NW waves (4 NW DPP rows) in BP block phases: the
        // most blocks used of the slices run, then the longer slice (fewer
        // rows a workgroup, fewer barriers), then four waves
        const int nb = (int)((w.k + MM_KC - 1) / MM_KC);
        int bnw = 4, bbp = 1;
        double best = -1.0;
        for (int nw : {4, 3})
            for (int bp = 1; bp <= 4 * nw; ++bp) {
                if ((4 * nw) % bp) continue;
                const double eff = (double)nb / ((nb + bp - 1) / bp * bp);
                if (eff > best + 1e-9 || (eff > best - 1e-9 && bp > bbp)) {
                    best = eff;
                    bnw = nw;
                    bbp = bp;
                }
            }
        const unsigned rows = (unsigned)(4 * bnw / bbp * 8);
        const dim3 grid((unsigned)((w.n + rows - 1) / rows), (unsigned)((m + 15) / 16));
        if (bnw == 3)
            i4_mm_dpp<3><<<grid, dim3(192), 0, s>>>(w.q4raw, w.s4raw, (int)w.n, (int)w.k, (int)w.g, a, (int)m, out,
                                                    bbp);
        else
            i4_mm_dpp<4><<<grid, dim3(256), 0, s>>>(w.q4raw, w.s4raw, (int)w.n, (int)w.k, (int)w.g, a, (int)m, out,
                                                    bbp);
        return hipGetLastError();
    }
    if (w.k % 32 == 0 && w.g % 32 == 0 && ((uintptr_t)a & 15) == 0 && m <= 65535) {
        i4_rows_chain<<<dim3((unsigned)((w.n + 255) / 256), (unsigned)m), dim3(256), 0, s>>>(
            w.q4raw, w.s4raw, (int)w.n, (int)w.k, (int)w.g, a, out);
        return hipGetLastError();
    }
    dim3 grid((unsigned)((w.n + 255) / 256), (unsigned)((m + 15) / 16));
    i4_gemm_rows<16><<<grid, dim3(256), 0, s>>>(w.q4raw, w.s4raw, (int)w.n, (int)w.k, (int)w.g, a, (int)m, out);
    return hipGetLastError();
}

hipError_t launch_i4(const Weight& w, size_t m, const float* a, float* out,
                     float* wsf, hipStream_t s) {
    if (m == 0) return hipSuccess;
    if (m == 1) {  // the reference's decode order, bit for bit, where the shape allows
        const hipError_t e = launch_i4_terms(w, a, out, s);
        if (e != hipErrorNotSupported) return e;
    }
    if (w.i4_blocked && fused_fits(w.k, m)) return launch_fused(w, m, a, out, s);
    if (w.i4_blocked && mfma_fits(w.k, m)) {
        const size_t mp = round_up(m, 4), ng4 = (w.k / 32 + 3) / 4;
        uint8_t* adig = reinterpret_cast<uint8_t*>(wsf);
        float* sog = reinterpret_cast<float*>(adig + (mp / 4) * ng4 * 64 * 32);
        const size_t nth = 4 * mp * 4 * ng4;
        i4_digits_kernel<<<dim3((unsigned)((nth + 255) / 256)), dim3(256), 0, s>>>(
            a, (int)m, (int)mp, (int)w.k, (int)ng4, adig, sog);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        switch (mp / 4) {
            case 1: return launch_mfma<1>(w, m, a, adig, sog, out, s);
            case 2: return launch_mfma<2>(w, m, a, adig, sog, out, s);
            case 3: return launch_mfma<3>(w, m, a, adig, sog, out, s);
            default: return launch_mfma<4>(w, m, a, adig, sog, out, s);
        }
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
