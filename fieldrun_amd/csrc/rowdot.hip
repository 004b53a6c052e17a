// rowdot.hip — the row-major unembed dot Bundle::rowdot_f32, gfx950.
//
// Restates /root/reference/src/bundle.rs:958-987 (rowdot_f32) and 995-1015
// (rowdot_f32_subset): out[r] = dot(W[r], x) for a (rows, d) matrix stored
// row-major as f32, f16, or rowi8 with an f32 scale per row, in the
// reference's operation order, bit for bit:
//   f32 / f16      a fold of w * x (w.to_f32() for f16; a mul, then an
//                  add) from -0.0 (Rust's f32 Sum), k ascending;
//   rowi8, full    s * rowi8_dot_avx2 (158-178), the order of the x86
//                  build (AVX2 + FMA hosts, 975-978): eight lane
//                  accumulators from +0.0, lane q an FMA chain over
//                  k = 8i + q, then hsum256 ((l0+l4)+(l2+l6)) + ((l1+l5)+
//                  (l3+l7)) (146-153), then a mul + add tail from 8*(d/8);
//   rowi8, subset  s * the fold from -0.0 (1009-1012).
// The subset form scores rows cand[i]; an id < 0 or >= rows gives -inf.
//
// HBM-bound: the matrix streams once.  One lane per row keeps each row's
// chain in order.  A wave owns 64 rows and walks d in 128-byte chunks: the
// chunk tile (64 rows x 128 B) is loaded coalesced (8 lanes per row, 16 B
// each), staged through the wave's padded LDS tile (row stride 144 B, so the
// lanes' row reads are conflict-free), and each lane reads back its own row;
// the next one or two chunks' loads are in flight meanwhile.  x is wave-uniform: its
// reads are scalar loads.  Rows are padded to a multiple of 128 bytes at
// upload, so chunk loads never run past a row.
#include "frq_internal.h"

#include <type_traits>

namespace frq {

namespace {

constexpr int TP = 144;  // LDS tile row stride (bytes)

// The argmax of the full-table form (ARG): each wave folds its 64 outputs'
// keys (order-preserving bits of the value, -0 as +0, above the row id, so
// ties go to the larger id) into *best with a 64-bit atomic max; a NaN
// output sets *err.
__device__ __forceinline__ unsigned long long argmax_key(float v, int row) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    if (u == 0x80000000u) u = 0;
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (uint32_t)row;
}

// NX x vectors at once (outputs out + v os, argmax best[v], v < nv): each
// lane runs NX chains of its row, one per vector, so the table streams once
// for all of them; every chain is the one-vector order.  For NX > 1, x is
// the vectors transposed, x[k NX + v] (zero for v >= nv): element k's NX
// values are adjacent, one wide scalar load feeding 2 NX VALU operations.
template <int DT, bool SUB, int DEPTH, int WPB, bool ARG, int NX = 1>  // DT: 0 f32, 1 f16, 2 rowi8; DEPTH
                                                                      // chunks in registers; WPB waves
__global__ __launch_bounds__(64 * WPB) void rowdot_kernel(
    const uint8_t* __restrict__ W, const float* __restrict__ rs, int rows, int d, size_t pitch,
    const float* __restrict__ x, const int64_t* __restrict__ cand, int nout, float* __restrict__ out,
    unsigned long long* __restrict__ best, int* __restrict__ err, size_t os = 0, int nv = NX) {
    constexpr int ES = DT == 0 ? 4 : (DT == 1 ? 2 : 1);  // bytes per element
    constexpr int CE = 128 / ES;                         // elements per chunk
    __shared__ __attribute__((aligned(16))) uint8_t tile[WPB][64 * TP];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int o0 = ((int)blockIdx.x * WPB + wave) * 64;
    if (o0 >= nout) return;  // wave-uniform; no block-wide barrier below
    uint8_t* tw = tile[wave];
    auto xat = [&](int u, int k) __attribute__((always_inline)) -> float { return NX == 1 ? x[k] : x[(size_t)k * NX + u]; };

    // the row an output scores (row 0 stands in for invalid ones)
    auto row_of = [&](int o, bool& ok) __attribute__((always_inline)) -> int {
        ok = o < nout;
        if constexpr (SUB) {
            const int64_t c = ok ? cand[o] : 0;
            ok = ok && c >= 0 && c < (int64_t)rows;
            return ok ? (int)c : 0;
        } else {
            return ok ? o : 0;
        }
    };
    // load instruction i of a chunk: lane l reads 16 bytes (l % 8) of the
    // row of output o0 + 8i + l / 8
    const uint8_t* src[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        bool ok;
        const int r = row_of(o0 + 8 * i + (lane >> 3), ok);
        src[i] = W + (size_t)r * pitch + (lane & 7) * 16;
    }
    bool own_ok;
    const int own_row = row_of(o0 + lane, own_ok);

    const int nch = (int)(pitch / 128);
    float acc[NX];  // the fold (f32, f16, subset rowi8)
    float l8[NX][8];  // the AVX2 lanes (full rowi8)
#pragma unroll
    for (int v = 0; v < NX; ++v) {
        acc[v] = -0.0f;
#pragma unroll
        for (int q = 0; q < 8; ++q) l8[v][q] = 0.0f;
    }
    auto load = [&](uint4 (&b)[8], int c) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 8; ++i) b[i] = ntload16u(src[i] + (size_t)c * 128);
    };
    // the elements k0 .. k0 + CE of this lane's row, in order; CHECK: only
    // those below d (the last, partial chunk)
    auto run = [&](const uint32_t (&v)[32], int k0, auto check) __attribute__((always_inline)) {
        constexpr bool CHECK = decltype(check)::value;
        if constexpr (DT == 0) {
#pragma unroll
            for (int e = 0; e < CE; ++e)
                if (!CHECK || k0 + e < d) {
                    const float w = __builtin_bit_cast(float, v[e]);
#pragma unroll
                    for (int u = 0; u < NX; ++u) acc[u] = acc[u] + w * xat(u, k0 + e);
                }
        } else if constexpr (DT == 1) {
#pragma unroll
            for (int e = 0; e < CE; ++e)
                if (!CHECK || k0 + e < d) {
                    const float w = h2f((uint16_t)(v[e >> 1] >> (16 * (e & 1))));
#pragma unroll
                    for (int u = 0; u < NX; ++u) acc[u] = acc[u] + w * xat(u, k0 + e);
                }
        } else if constexpr (SUB) {
#pragma unroll
            for (int e = 0; e < CE; ++e)
                if (!CHECK || k0 + e < d) {
                    const float w = (float)(int8_t)(v[e >> 2] >> (8 * (e & 3)));
#pragma unroll
                    for (int u = 0; u < NX; ++u) acc[u] = acc[u] + w * xat(u, k0 + e);
                }
        } else {
            // full 8-element groups only; the tail follows the lane sum
#pragma unroll
            for (int gi = 0; gi < CE / 8; ++gi) {
                const int kb = k0 + 8 * gi;
                if (!CHECK || kb + 8 <= d) {
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        const float w = (float)(int8_t)(v[2 * gi + (q >> 2)] >> (8 * (q & 3)));
#pragma unroll
                        for (int u = 0; u < NX; ++u) l8[u][q] = __builtin_fmaf(w, xat(u, kb + q), l8[u][q]);
                    }
                }
            }
        }
    };
    // one chunk: through the tile, then this lane's row
    auto consume = [&](const uint4 (&b)[8], int c) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            *reinterpret_cast<uint4*>(tw + (8 * i + (lane >> 3)) * TP + (lane & 7) * 16) = b[i];
        wave_sync();
        uint32_t v[32];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint4 q = *reinterpret_cast<const uint4*>(tw + lane * TP + 16 * j);
            v[4 * j] = q.x; v[4 * j + 1] = q.y; v[4 * j + 2] = q.z; v[4 * j + 3] = q.w;
        }
        wave_sync();  // the tile is read before the next chunk is written
        const int k0 = c * CE;
        if (k0 + CE <= d) run(v, k0, std::false_type{});  // wave-uniform
        else run(v, k0, std::true_type{});
        if constexpr (DT == 2 && !SUB) {
            if (c == nch - 1) {
#pragma unroll
                for (int u = 0; u < NX; ++u) {
                    const float q0 = l8[u][0] + l8[u][4], q1 = l8[u][1] + l8[u][5];
                    const float q2 = l8[u][2] + l8[u][6], q3 = l8[u][3] + l8[u][7];
                    acc[u] = (q0 + q2) + (q1 + q3);
                }
                const int kt = d & ~7;  // the tail lies in this chunk
                if (kt < d) {
#pragma unroll
                    for (int e = 0; e < CE; ++e)
                        if (k0 + e >= kt && k0 + e < d) {
                            const float w = (float)(int8_t)(v[e >> 2] >> (8 * (e & 3)));
#pragma unroll
                            for (int u = 0; u < NX; ++u) acc[u] = acc[u] + w * xat(u, k0 + e);
                        }
                }
            }
        }
    };
    // DEPTH - 1 chunks in flight ahead of the one consumed: a ring of DEPTH
    // register buffers, rotated by unrolling (static indices).  Every load
    // is issued unconditionally (the index clamped to the last chunk, whose
    // re-reads hit L2), so the waits before a buffer's use count exactly
    // the loads issued after it.
    uint4 b0[8], b1[8], b2[8];
    if (nch > 0) {
        const int last = nch - 1;
        load(b0, 0);
        load(b1, min(1, last));
        if constexpr (DEPTH == 2) {
            for (int c = 0; c < nch; c += 2) {
                consume(b0, c);
                load(b0, min(c + 2, last));
                if (c + 1 < nch) consume(b1, c + 1);
                load(b1, min(c + 3, last));
            }
        } else {
            load(b2, min(2, last));
            for (int c = 0; c < nch; c += 3) {
                consume(b0, c);
                load(b0, min(c + 3, last));
                if (c + 1 < nch) consume(b1, c + 1);
                load(b1, min(c + 4, last));
                if (c + 2 < nch) consume(b2, c + 2);
                load(b2, min(c + 5, last));
            }
        }
    }
    const int o = o0 + lane;
#pragma unroll
    for (int u = 0; u < NX; ++u) {
        float a = acc[u];
        if constexpr (DT == 2) {
            if (!SUB && nch == 0) a = 0.0f;  // d == 0: hsum of zero lanes
            a = rs[own_row] * a;
        }
        if (NX > 1 && u >= nv) break;  // the zero padding of the transposed x
        if (o < nout) out[u * os + o] = own_ok ? a : -__builtin_inff();
        if constexpr (ARG) {
            unsigned long long key = o < nout ? argmax_key(a, o) : 0ull;
            const bool nan = o < nout && a != a;
#pragma unroll
            for (int sh = 32; sh > 0; sh >>= 1) {
                const unsigned long long ok = __shfl_xor(key, sh);
                key = ok > key ? ok : key;
            }
            if (__builtin_amdgcn_ballot_w64(nan) && lane == 0) atomicOr(err, 1);
            if (lane == 0) atomicMax(best + u, key);
        }
    }
}

template <int DT, bool ARG>
hipError_t launch_dt(const Weight& w, const float* x, const int64_t* cand, size_t nout, float* out,
                     unsigned long long* best, int* err, hipStream_t s) {
    // fewer waves than about four per SIMD: keep three chunks in flight per
    // wave (latency-bound), else two (the occupancy carries the load)
    const bool deep = nout < 4 * 1024 * 64;
    const unsigned g4 = (unsigned)((nout + 255) / 256);
#define FRQ_ROWDOT(SUBV, DEPTHV, WPBV)                                                                   \
    rowdot_kernel<DT, SUBV, DEPTHV, WPBV, ARG><<<dim3(g4), dim3(64 * WPBV), 0, s>>>(                   \
        w.rowp, w.scale, (int)w.n, (int)w.k, w.rpitch, x, cand, (int)nout, out, best, err)
    if (cand) {
        if (deep) FRQ_ROWDOT(true, 3, 4);
        else FRQ_ROWDOT(true, 2, 4);
    } else {
        if (deep) FRQ_ROWDOT(false, 3, 4);
        else FRQ_ROWDOT(false, 2, 4);
    }
#undef FRQ_ROWDOT
    return hipGetLastError();
}

// Products w * x[u] for vectors u = U, U + 1 of one element: x (a VGPR)
// holds vector u's value in lane u of each 16-lane DPP row, and
// v_mul_f32_dpp row_newbcast:u hands every lane that value times its own w.
// NOP: the two wait states a DPP read needs after a VALU write of x (the
// compiler does not see into the asm).
#define FRQ_DPPM(dst, n) "v_mul_f32_dpp %" #dst ", %2, %3 row_newbcast:" #n " row_mask:0xf bank_mask:0xf\n\t"
template <int U, bool NOP>
__device__ __forceinline__ void dpp_mul2(float& p0, float& p1, float x, float w) {
    static_assert(U >= 0 && U <= 14 && U % 2 == 0, "lane pair");
#define FRQ_DPPM_CASE(u0, u1)                                                                        \
    if constexpr (U == u0) {                                                                         \
        if constexpr (NOP) asm("s_nop 1\n\t" FRQ_DPPM(0, u0) FRQ_DPPM(1, u1) : "=&v"(p0), "=&v"(p1) : "v"(x), "v"(w)); \
        else asm(FRQ_DPPM(0, u0) FRQ_DPPM(1, u1) : "=&v"(p0), "=&v"(p1) : "v"(x), "v"(w));              \
    }
    FRQ_DPPM_CASE(0, 1) FRQ_DPPM_CASE(2, 3) FRQ_DPPM_CASE(4, 5) FRQ_DPPM_CASE(6, 7)
    FRQ_DPPM_CASE(8, 9) FRQ_DPPM_CASE(10, 11) FRQ_DPPM_CASE(12, 13) FRQ_DPPM_CASE(14, 15)
#undef FRQ_DPPM_CASE
}
#undef FRQ_DPPM

// The f32 / f16 fold for 2 <= NX <= 16 vectors with the argmax (the
// batched head): each output is rowdot_kernel's fold (acc = acc + w * x
// from -0.0, k ascending).  A lane owns a row (read from the LDS tile 16
// bytes at a time); an element's NX products come from dpp_mul2 (x
// broadcast from a register, no scalar loads: their latency, not the
// arithmetic, bounded the scalar-x form), then its NX adds.  x is in the
// k-quad interleaved layout xq[64 (k / 4) + 4 v + k % 4] (16 vector slots,
// k < d + 4; lane l loads the quad of vector l % 16), one quad ahead.  The
// next chunk's row tile loads into the registers the current one was
// staged from.
template <int DT, int NX>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void rowdot_nx_kernel(const uint8_t* __restrict__ W, int rows, int d, size_t pitch,
                                                        const float* __restrict__ xq, float* __restrict__ out,
                                                        unsigned long long* __restrict__ best, int* __restrict__ err,
                                                        size_t os, int nv) {
    static_assert(DT == 0 || DT == 1, "the fold arms");
    static_assert(NX >= 2 && NX <= 16 && NX % 2 == 0, "vector pairs");
    constexpr int ES = DT == 0 ? 4 : 2;  // bytes per element
    constexpr int EQ = 16 / ES;          // elements per 16-byte piece
    __shared__ __attribute__((aligned(16))) uint8_t tile[4][64 * TP];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int o0 = ((int)blockIdx.x * 4 + wave) * 64;
    if (o0 >= rows) return;  // wave-uniform; no block-wide barrier below
    uint8_t* tw = tile[wave];
    // load instruction i of a chunk: row o0 + 8 i + lane / 8 (the last row
    // past the end), bytes 16 (lane % 8); 32-bit offsets from the wave's
    // first row (64 rows of one table)
    const uint8_t* wb = W + (size_t)o0 * pitch;
    uint32_t lo[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        lo[i] = (uint32_t)min(8 * i + (lane >> 3), rows - 1 - o0) * (uint32_t)pitch + (lane & 7) * 16;
    const int nch = (int)(pitch / 128);
    const float* xl = xq + 4 * (lane & 15);
    const int nq = (d + 3) / 4;  // quads of x
    float acc[NX];
#pragma unroll
    for (int u = 0; u < NX; ++u) acc[u] = -0.0f;
    // element e of piece q (a uint4 of the lane's row) as f32
    auto elem = [&](const uint4& q, int e) __attribute__((always_inline)) -> float {
        const uint32_t wd = e / (4 / ES) == 0 ? q.x : e / (4 / ES) == 1 ? q.y : e / (4 / ES) == 2 ? q.z : q.w;
        if constexpr (DT == 0) return __builtin_bit_cast(float, wd);
        else return h2f((uint16_t)(wd >> (16 * (e & 1))));
    };
    // one element: w times its x (component i of the quad xv); ADD: k < d
    auto fold = [&](float w, const float4& xv, int i, bool add) __attribute__((always_inline)) {
        const float xi = i == 0 ? xv.x : i == 1 ? xv.y : i == 2 ? xv.z : xv.w;
        float pr[NX];
        dpp_mul2<0, true>(pr[0], pr[1], xi, w);
        if constexpr (NX > 2) dpp_mul2<2, false>(pr[2], pr[3], xi, w);
        if constexpr (NX > 4) {
            dpp_mul2<4, false>(pr[4], pr[5], xi, w);
            dpp_mul2<6, false>(pr[6], pr[7], xi, w);
        }
        if constexpr (NX > 8) {
            dpp_mul2<8, false>(pr[8], pr[9], xi, w);
            dpp_mul2<10, false>(pr[10], pr[11], xi, w);
            dpp_mul2<12, false>(pr[12], pr[13], xi, w);
            dpp_mul2<14, false>(pr[14], pr[15], xi, w);
        }
        if (add) {
#pragma unroll
            for (int u = 0; u < NX; ++u) acc[u] = acc[u] + pr[u];
        }
    };
    auto xload = [&](int kq) __attribute__((always_inline)) {
        return *reinterpret_cast<const float4*>(xl + (size_t)min(kq, nq - 1) * 64);
    };
    // a chunk's elements k0 .. k0 + 128 / ES; CHECK: only k < d.  The quads
    // alternate two register sets (an even count a chunk).
    float4 xa = xload(0), xb;
    auto run = [&](auto check, int k0) __attribute__((always_inline)) {
        constexpr bool CHECK = decltype(check)::value;
        const int kq0 = k0 / 4;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint4 q = *reinterpret_cast<const uint4*>(tw + lane * TP + 16 * j);
#pragma unroll
            for (int h = 0; h < EQ / 4; ++h) {
                const int qi = j * (EQ / 4) + h;  // quad of the chunk
                if (qi % 2 == 0) {
                    xb = xload(kq0 + qi + 1);
#pragma unroll
                    for (int i = 0; i < 4; ++i) fold(elem(q, 4 * h + i), xa, i, !CHECK || k0 + 4 * qi + i < d);
                } else {
                    xa = xload(kq0 + qi + 1);
#pragma unroll
                    for (int i = 0; i < 4; ++i) fold(elem(q, 4 * h + i), xb, i, !CHECK || k0 + 4 * qi + i < d);
                }
            }
        }
    };
    uint4 b[8];
    auto load = [&](int c) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 8; ++i) b[i] = ntload16u(wb + (size_t)c * 128 + lo[i]);
    };
    if (nch > 0) {
        load(0);
        for (int c = 0; c < nch; ++c) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                *reinterpret_cast<uint4*>(tw + (8 * i + (lane >> 3)) * TP + (lane & 7) * 16) = b[i];
            load(min(c + 1, nch - 1));  // the next chunk, under this one's arithmetic
            wave_sync();
            const int k0 = c * (128 / ES);
            if (k0 + 128 / ES <= d) run(std::false_type{}, k0);  // wave-uniform
            else run(std::true_type{}, k0);
            wave_sync();  // the tile is read before the next chunk is written
        }
    }
    const int o = o0 + lane;
#pragma unroll
    for (int u = 0; u < NX; ++u) {
        if (u >= nv) break;  // the zero padding of the transposed x
        const float a = acc[u];
        if (o < rows) out[u * os + o] = a;
        unsigned long long key = o < rows ? argmax_key(a, o) : 0ull;
        const bool nan = o < rows && a != a;
#pragma unroll
        for (int sh = 32; sh > 0; sh >>= 1) {
            const unsigned long long ok = __shfl_xor(key, sh);
            key = ok > key ? ok : key;
        }
        if (__builtin_amdgcn_ballot_w64(nan) && lane == 0) atomicOr(err, 1);
        if (lane == 0) atomicMax(best + u, key);
    }
}

// xq[64 (k / 4) + 4 v + k % 4] = x[v xs + k] for v < nv and k < d, else 0,
// over the (d + 3) / 4 quads (rowdot_nx_kernel's x layout)
__global__ __launch_bounds__(256) void quad_x_kernel(const float* __restrict__ x, size_t xs, int nv, int d,
                                                     float* __restrict__ xq) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t nq = ((size_t)d + 3) / 4;
    if (i >= nq * 64) return;
    const int kq = (int)(i / 64), v = (int)(i % 64) / 4, k = 4 * kq + (int)(i % 4);
    xq[i] = v < nv && k < d ? x[(size_t)v * xs + k] : 0.0f;
}

// xt[k NX + v] = x[v xs + k] for v < nv, 0 for nv <= v < NX
template <int NX>
__global__ __launch_bounds__(256) void transpose_x_kernel(const float* __restrict__ x, size_t xs, int nv, int d,
                                                          float* __restrict__ xt) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)d * NX) return;
    const int k = (int)(i / NX), v = (int)(i % NX);
    xt[i] = v < nv ? x[(size_t)v * xs + k] : 0.0f;
}

template <int DT, int NX>
hipError_t launch_argmax_nx(const Weight& w, size_t nv, const float* x, size_t xs, float* xt, float* out, size_t os,
                            unsigned long long* best, int* err, hipStream_t s) {
    const unsigned g4 = (unsigned)((w.n + 255) / 256);
    if constexpr (NX > 1 && DT != 2) {
        const size_t nq = (w.k + 3) / 4;
        quad_x_kernel<<<dim3((unsigned)((nq * 64 + 255) / 256)), dim3(256), 0, s>>>(x, xs, (int)nv, (int)w.k, xt);
        rowdot_nx_kernel<DT, NX><<<dim3(g4), dim3(256), 0, s>>>(w.rowp, (int)w.n, (int)w.k, w.rpitch, xt, out, best,
                                                                 err, os, (int)nv);
    } else {
        const float* xv = x;
        if constexpr (NX > 1) {
            const size_t tot = w.k * NX;
            transpose_x_kernel<NX><<<dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s>>>(x, xs, (int)nv,
                                                                                             (int)w.k, xt);
            xv = xt;
        }
        rowdot_kernel<DT, false, 2, 4, true, NX><<<dim3(g4), dim3(256), 0, s>>>(
            w.rowp, w.scale, (int)w.n, (int)w.k, w.rpitch, xv, nullptr, (int)w.n, out, best, err, os, (int)nv);
    }
    return hipGetLastError();
}

template <int DT>
hipError_t launch_argmax_batch(const Weight& w, size_t nx, const float* x, size_t xs, float* xt, float* out,
                               size_t os, unsigned long long* best, int* err, hipStream_t s) {
    // up to 16 vectors a pass (each a chain per lane), further passes for
    // more; a count between the powers of two runs zero-padded
    for (size_t v0 = 0; v0 < nx; v0 += 16) {
        const size_t k = nx - v0 < 16 ? nx - v0 : 16;
        const float* xv = x + v0 * xs;
        float* ov = out + v0 * os;
        hipError_t e;
        if (k == 1) e = launch_argmax_nx<DT, 1>(w, 1, xv, xs, xt, ov, os, best + v0, err, s);
        else if (k == 2) e = launch_argmax_nx<DT, 2>(w, k, xv, xs, xt, ov, os, best + v0, err, s);
        else if (k <= 4) e = launch_argmax_nx<DT, 4>(w, k, xv, xs, xt, ov, os, best + v0, err, s);
        else if (k <= 8) e = launch_argmax_nx<DT, 8>(w, k, xv, xs, xt, ov, os, best + v0, err, s);
        else e = launch_argmax_nx<DT, 16>(w, k, xv, xs, xt, ov, os, best + v0, err, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

// rowdot_f32 with the argmax fold for nx vectors x + v xs at once (outputs
// out + v os, best[v]); each output's arithmetic is launch_rowdot_argmax's.
// xt: device scratch of 16 (w.k + 4) floats (the vectors of a pass, transposed or in quads).
hipError_t launch_rowdot_argmax_batch(const Weight& w, size_t nx, const float* x, size_t xs, float* xt, float* out,
                                      size_t os, unsigned long long* best, int* err, hipStream_t s) {
    if (!w.n || !nx) return hipSuccess;
    if (w.n > (size_t)INT32_MAX - 256 || w.k > (size_t)INT32_MAX) return hipErrorInvalidValue;
    switch (w.dtype) {
        case FRQ_DT_F32: return launch_argmax_batch<0>(w, nx, x, xs, xt, out, os, best, err, s);
        case FRQ_DT_F16: return launch_argmax_batch<1>(w, nx, x, xs, xt, out, os, best, err, s);
        case FRQ_DT_ROWI8: return launch_argmax_batch<2>(w, nx, x, xs, xt, out, os, best, err, s);
        default: return hipErrorInvalidValue;
    }
}

size_t row_pitch(int dtype, size_t d) {
    const size_t es = dtype == FRQ_DT_F32 ? 4 : (dtype == FRQ_DT_F16 ? 2 : 1);
    return (d * es + 127) / 128 * 128;
}

hipError_t launch_rowdot(const Weight& w, const float* x, const int64_t* cand, size_t nout, float* out,
                         hipStream_t s) {
    if (!nout) return hipSuccess;
    if (nout > (size_t)INT32_MAX - 256 || w.n > (size_t)INT32_MAX || w.k > (size_t)INT32_MAX)
        return hipErrorInvalidValue;
    switch (w.dtype) {
        case FRQ_DT_F32: return launch_dt<0, false>(w, x, cand, nout, out, nullptr, nullptr, s);
        case FRQ_DT_F16: return launch_dt<1, false>(w, x, cand, nout, out, nullptr, nullptr, s);
        case FRQ_DT_ROWI8: return launch_dt<2, false>(w, x, cand, nout, out, nullptr, nullptr, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_rowdot_argmax(const Weight& w, const float* x, float* out, unsigned long long* best, int* err,
                                hipStream_t s) {
    if (!w.n) return hipSuccess;
    if (w.n > (size_t)INT32_MAX - 256 || w.k > (size_t)INT32_MAX) return hipErrorInvalidValue;
    switch (w.dtype) {
        case FRQ_DT_F32: return launch_dt<0, true>(w, x, nullptr, w.n, out, best, err, s);
        case FRQ_DT_F16: return launch_dt<1, true>(w, x, nullptr, w.n, out, best, err, s);
        case FRQ_DT_ROWI8: return launch_dt<2, true>(w, x, nullptr, w.n, out, best, err, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace frq
