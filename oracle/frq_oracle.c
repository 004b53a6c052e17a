/*
 * frq_oracle.c — CPU restatement of fieldrun's quantised-linear hot path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker + CPU baseline); see
 * frq_oracle.h for who may load it and how each function is pinned.
 *
 * Build: gcc -O3 -march=x86-64 -ffp-contract=off -fPIC -shared (oracle/Makefile).
 * -march=x86-64 mirrors the reference's release target (no target-cpu
 * override anywhere in its tree), -ffp-contract=off mirrors Rust, which never
 * contracts a*b+c into an FMA unless the source calls mul_add/_mm*_fmadd.
 *
 * All citations are to /root/reference (fieldrun 0.1.0).
 */
#include "frq_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* f16 <-> f32.  The reference upcasts with half::f16::to_f32 / F16C         */
/* (src/bundle.rs:921-933, 1131-1160; exact) and downcasts with               */
/* half::f16::from_f32 (src/convert.rs:147-155; round-to-nearest-even).       */
/* ------------------------------------------------------------------------ */
static size_t nz(size_t x) { return x ? x : 1; }
/* The reference's FMA code paths are compiled for FMA hardware
 * (#[target_feature(enable = "avx2,fma")] on i4_dot_avx2 / q4a_dot_avx2 /
 * rowi8_dot_avx2, src/bundle.rs:158-258; matrixmultiply selects its FMA
 * micro-kernel at run time): the functions that restate them use the FMA
 * instruction for fmaf too (same values as the libm call, which is exact). */
#define FRO_FMA __attribute__((target("fma")))
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float fro_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0x1F) /* inf / nan: keep payload */
        return u2f(sign | 0x7F800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: value = man * 2^-24, exact in f32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t fro_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) {
        if (man) return (uint16_t)(sign | 0x7E00u | (man >> 13));
        return (uint16_t)(sign | 0x7C00u);
    }
    int32_t he = (int32_t)exp - 127 + 15;
    if (he >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (he <= 0) {
        if (14 - he > 24) return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t hm = man >> (14 - he);
        uint32_t rb = 1u << (13 - he);
        /* round half to even: round bit set and (sticky or lsb) */
        if ((man & rb) && (man & (3u * rb - 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)he << 10) | (man >> 13);
    uint32_t rb = 0x1000u;
    if ((man & rb) && (man & (3u * rb - 1u))) h++;
    return (uint16_t)h;
}

void fro_f16_to_f32_n(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = fro_f16_to_f32(src[i]);
}

/* Rust `f32::round_ties_even` (src/convert.rs:351, 208): rintf under the
 * default FE_TONEAREST mode. */
static float round_ties_even(float v) { return rintf(v); }

static float clampf(float v, float lo, float hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

/* put_i8: src/convert.rs:344-360.  scale_j = max(amax_j/127, 1e-8) (f32),
 * q = clamp(round_ties_even(w/s), -127, 127), stored (in,out); the scale is
 * written as f16 (put_f16, 147-155). */
void fro_put_i8(const float* data, size_t rows, size_t cols, int transpose,
                int8_t* w_in_out, uint16_t* scale_f16) {
    size_t out = transpose ? rows : cols, inp = transpose ? cols : rows;
#define AT(i, j) (transpose ? data[(j) * inp + (i)] : data[(i) * out + (j)])
    float* sc = (float*)malloc(nz(out) * sizeof(float));
    for (size_t j = 0; j < out; j++) {
        float m = 0.0f;
        for (size_t i = 0; i < inp; i++) m = fmaxf(m, fabsf(AT(i, j)));
        float s = m / 127.0f;
        sc[j] = s > 1e-8f ? s : 1e-8f; /* f32::max(x, 1e-8) */
    }
    for (size_t i = 0; i < inp; i++)
        for (size_t j = 0; j < out; j++)
            w_in_out[i * out + j] =
                (int8_t)clampf(round_ties_even(AT(i, j) / sc[j]), -127.0f, 127.0f);
    for (size_t j = 0; j < out; j++) scale_f16[j] = fro_f32_to_f16(sc[j]);
    free(sc);
#undef AT
}

/* put_i4: src/convert.rs:189-216.  g = min(32, in); scale (out, ng) =
 * max(amax/7, 1e-8); q = clamp(round_ties_even(w/s), -7, 7) as a two's-
 * complement nibble, even input index in the low nibble.  Returns g. */
size_t fro_put_i4(const float* data, size_t rows, size_t cols, int transpose,
                  uint8_t* packed, uint16_t* scale_f16) {
    size_t out = transpose ? rows : cols, inp = transpose ? cols : rows;
#define AT(i, j) (transpose ? data[(j) * inp + (i)] : data[(i) * out + (j)])
    size_t g = 32 < nz(inp) ? 32 : nz(inp);
    size_t ng = (inp + g - 1) / g, rb = (inp + 1) / 2;
    float* sc = (float*)malloc(nz(out * ng) * sizeof(float));
    for (size_t j = 0; j < out; j++)
        for (size_t gi = 0; gi < ng; gi++) {
            size_t lo = gi * g, hi = (gi + 1) * g < inp ? (gi + 1) * g : inp;
            float m = 0.0f;
            for (size_t i = lo; i < hi; i++) m = fmaxf(m, fabsf(AT(i, j)));
            float s = m / 7.0f;
            sc[j * ng + gi] = s > 1e-8f ? s : 1e-8f;
        }
    memset(packed, 0, out * rb);
    for (size_t j = 0; j < out; j++)
        for (size_t i = 0; i < inp; i++) {
            float s = sc[j * ng + i / g];
            int8_t q = (int8_t)clampf(round_ties_even(AT(i, j) / s), -7.0f, 7.0f);
            uint8_t nib = (uint8_t)q & 0x0F;
            packed[j * rb + i / 2] |= (i % 2 == 0) ? nib : (uint8_t)(nib << 4);
        }
    for (size_t i = 0; i < out * ng; i++) scale_f16[i] = fro_f32_to_f16(sc[i]);
    free(sc);
    return g;
#undef AT
}

/* put_embed_i8: src/convert.rs:265-279 (row-major per-row int8). */
void fro_put_embed_i8(const float* data, size_t vocab, size_t d, int8_t* q,
                      uint16_t* scale_f16) {
    for (size_t r = 0; r < vocab; r++) {
        float m = 0.0f;
        for (size_t c = 0; c < d; c++) m = fmaxf(m, fabsf(data[r * d + c]));
        float s = m / 127.0f;
        s = s > 1e-8f ? s : 1e-8f;
        for (size_t c = 0; c < d; c++)
            q[r * d + c] = (int8_t)clampf(round_ties_even(data[r * d + c] / s), -127.0f, 127.0f);
        scale_f16[r] = fro_f32_to_f16(s);
    }
}

/* Bundle::load i8 arm: src/bundle.rs:345-355, wt[j*k+kk] = raw[kk*n+j]. */
void fro_i8_transpose(const int8_t* w_kn, size_t k, size_t n, int8_t* wt_nk) {
    for (size_t kk = 0; kk < k; kk++)
        for (size_t j = 0; j < n; j++) wt_nk[j * k + kk] = w_kn[kk * n + j];
}

/* i8dot scalar fallback: src/bundle.rs:1052 (the `_scalar_i8_bench` path,
 * Cargo.toml:19-21).  Every SIMD variant equals it (1359-1382). */
int32_t fro_i8dot(const int8_t* a, const int8_t* w, size_t n) {
    int32_t s = 0;
    for (size_t i = 0; i < n; i++) s += (int32_t)a[i] * (int32_t)w[i];
    return s;
}

/* i8dot_avx512bw: src/bundle.rs:1107-1126, the dot the production x86 build
 * dispatches to when the host has avx512bw + avx512f (1044-1047): 32 lanes
 * a step (sign-extend to i16, madd to 16 i32 pairwise sums, add), a
 * horizontal add of the 16 lanes, then the scalar tail.  Integer and
 * overflow-free at these lengths, so it equals fro_i8dot (the reference's
 * own test, 1359-1382).  Used for the CPU baseline's second figure. */
__attribute__((target("avx512bw,avx512f")))
int32_t fro_i8dot_avx512bw(const int8_t* a, const int8_t* w, size_t n) {
    const size_t chunks = n / 32;
    __m512i acc = _mm512_setzero_si512();
    for (size_t c = 0; c < chunks; c++) {
        const __m256i av = _mm256_loadu_si256((const __m256i*)(a + c * 32));
        const __m256i wv = _mm256_loadu_si256((const __m256i*)(w + c * 32));
        acc = _mm512_add_epi32(acc, _mm512_madd_epi16(_mm512_cvtepi8_epi16(av), _mm512_cvtepi8_epi16(wv)));
    }
    int32_t s = _mm512_reduce_add_epi32(acc);
    for (size_t k = chunks * 32; k < n; k++) s += (int32_t)a[k] * (int32_t)w[k];
    return s;
}

/* The dot the int8 linears below use: the scalar fallback (the
 * `_scalar_i8_bench` build, the default here) or, after
 * fro_set_i8dot(1) on a host with AVX-512BW, i8dot_avx512bw. */
static int32_t (*g_i8dot)(const int8_t*, const int8_t*, size_t) = fro_i8dot;

int fro_set_i8dot(int variant) {
    if (variant == 1) {
        __builtin_cpu_init();
        if (!__builtin_cpu_supports("avx512bw") || !__builtin_cpu_supports("avx512f")) return 0;
        g_i8dot = fro_i8dot_avx512bw;
        return 1;
    }
    g_i8dot = fro_i8dot;
    return 1;
}

/* Rust `f as i32` saturates and maps NaN to 0. */
static int32_t sat_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483647.0f) return 2147483647;
    if (v <= -2147483648.0f) return (-2147483647 - 1);
    return (int32_t)v;
}

/* Quickselect: the value at rank `r` (0-based) of v[0..n) in DESCENDING
 * order; reorders v.  Stands in for select_nth_unstable_by
 * (src/bundle.rs:702-705); only the value at rank t is used, which is
 * unique even when the index permutation is not. */
static float select_desc(float* v, size_t n, size_t r) {
    size_t lo = 0, hi = n; /* rank r lies in [lo, hi) */
    while (hi - lo > 1) {
        float a = v[lo], b = v[lo + (hi - lo) / 2], c = v[hi - 1];
        float p = (a < b) ? ((b < c) ? b : (a < c ? c : a)) : ((a < c) ? a : (b < c ? c : b));
        /* 3-way partition: [lo,lt) > p, [lt,gt) == p, [gt,hi) < p */
        size_t lt = lo, i = lo, gt = hi;
        while (i < gt) {
            float x = v[i];
            if (x > p) { v[i] = v[lt]; v[lt] = x; lt++; i++; }
            else if (x < p) { gt--; v[i] = v[gt]; v[gt] = x; }
            else i++;
        }
        if (r < lt) hi = lt;
        else if (r >= gt) lo = gt;
        else return p;
    }
    return v[lo];
}

/* Outlier-aware per-token activation quant: src/bundle.rs:691 (t),
 * 699-708 (M>1) == 732-743 (M==1), OUTLIER_T at 309.
 *   bulk_max = (t+1)-th largest |a| (0 when t == k)
 *   sa = bulk_max > 0 ? bulk_max/127 : 1
 *   a8 = clamp(round(a/sa) as i32, -127, 127)   (round: half away from 0)
 *   the t largest-|a| channels are zeroed and kept as (idx, a) outliers.
 * The reference leaves the outliers in select_nth_unstable_by's order and
 * breaks ties at |a| == bulk_max arbitrarily; here outliers are all channels
 * with |a| > bulk_max plus the lowest-index ties, listed in ascending channel
 * order (the corr summation order the GPU kernels also use). */
int fro_quant_row(const float* a, size_t k, int8_t* a8, float* sa_out,
                  uint32_t* oidx, float* oval, size_t* t_out) {
    size_t t = FRO_OUTLIER_T < k ? FRO_OUTLIER_T : k;
    float bulk = 0.0f;
    if (t < k) {
        for (size_t i = 0; i < k; i++)
            if (a[i] != a[i]) return FRO_ERR_NAN; /* partial_cmp().unwrap() */
        float* tmp = (float*)malloc(k * sizeof(float));
        for (size_t i = 0; i < k; i++) tmp[i] = fabsf(a[i]);
        bulk = select_desc(tmp, k, t);
        free(tmp);
    }
    float sa = bulk > 0.0f ? bulk / 127.0f : 1.0f;
    for (size_t i = 0; i < k; i++) {
        int32_t q = sat_i32(roundf(a[i] / sa));
        q = q < -127 ? -127 : (q > 127 ? 127 : q);
        a8[i] = (int8_t)q;
    }
    size_t n = 0;
    if (t == k) {
        for (size_t i = 0; i < k; i++) { oidx[n] = (uint32_t)i; oval[n] = a[i]; a8[i] = 0; n++; }
    } else {
        size_t gt = 0;
        for (size_t i = 0; i < k; i++) gt += fabsf(a[i]) > bulk;
        size_t ties = t - gt; /* >= 1 by definition of the (t+1)-th value */
        for (size_t i = 0; i < k && n < t; i++) {
            float m = fabsf(a[i]);
            if (m > bulk || (m == bulk && ties > 0)) {
                if (m == bulk) ties--;
                oidx[n] = (uint32_t)i; oval[n] = a[i]; a8[i] = 0; n++;
            }
        }
    }
    *sa_out = sa;
    *t_out = t;
    return FRO_OK;
}

/* Epilogue of the I8 arm: src/bundle.rs:709-715 / 745-751.
 *   corr = sum over outliers of av * (wt[j,ch] as f32)   (fold from -0.0)
 *   out  = scale[j] * (sa * (acc as f32) + corr)          (no FMA) */
static void i8_row(const float* arow, size_t k, const int8_t* wt,
                   const float* scale, size_t j0, size_t j1, const int8_t* a8,
                   float sa, const uint32_t* oidx, const float* oval, size_t t,
                   float* orow, int32_t* accrow) {
    for (size_t j = j0; j < j1; j++) {
        const int8_t* w = wt + j * k;
        int32_t acc = g_i8dot(a8, w, k);
        float corr = -0.0f;
        for (size_t o = 0; o < t; o++) corr = corr + oval[o] * (float)w[oidx[o]];
        orow[j] = scale[j] * (sa * (float)acc + corr);
        if (accrow) accrow[j] = acc;
    }
    (void)arow;
}

int fro_mm_i8(const float* a, size_t m, size_t k, const int8_t* wt,
              const float* scale, size_t n, float* out, int32_t* acc) {
    int8_t* a8 = (int8_t*)malloc(nz(k));
    uint32_t oidx[FRO_OUTLIER_T];
    float oval[FRO_OUTLIER_T], sa;
    size_t t;
    for (size_t i = 0; i < m; i++) {
        int rc = fro_quant_row(a + i * k, k, a8, &sa, oidx, oval, &t);
        if (rc) { free(a8); return rc; }
        i8_row(a + i * k, k, wt, scale, 0, n, a8, sa, oidx, oval, t, out + i * n,
               acc ? acc + i * n : NULL);
    }
    free(a8);
    return FRO_OK;
}

/* Threaded variant with the reference's rayon split: M==1 fans out over
 * output columns (src/bundle.rs:744-752), M>1 over rows (695-718). */
typedef struct {
    const float* a; size_t m, k, n; const int8_t* wt; const float* scale;
    float* out; size_t lo, hi; int by_rows;
    const int8_t* a8; float sa; const uint32_t* oidx; const float* oval; size_t t;
    int rc;
} mt_job;

static void* mt_worker(void* p) {
    mt_job* J = (mt_job*)p;
    if (!J->by_rows) {
        i8_row(J->a, J->k, J->wt, J->scale, J->lo, J->hi, J->a8, J->sa, J->oidx, J->oval,
               J->t, J->out, NULL);
        return NULL;
    }
    int8_t* a8 = (int8_t*)malloc(nz(J->k));
    uint32_t oidx[FRO_OUTLIER_T];
    float oval[FRO_OUTLIER_T], sa;
    size_t t;
    for (size_t i = J->lo; i < J->hi; i++) {
        int rc = fro_quant_row(J->a + i * J->k, J->k, a8, &sa, oidx, oval, &t);
        if (rc) { J->rc = rc; break; }
        i8_row(J->a + i * J->k, J->k, J->wt, J->scale, 0, J->n, a8, sa, oidx, oval, t,
               J->out + i * J->n, NULL);
    }
    free(a8);
    return NULL;
}

int fro_mm_i8_mt(const float* a, size_t m, size_t k, const int8_t* wt,
                 const float* scale, size_t n, float* out, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    pthread_t th[256];
    mt_job jobs[256];
    if (nthreads > 256) nthreads = 256;
    int8_t* a8 = NULL;
    uint32_t oidx[FRO_OUTLIER_T];
    float oval[FRO_OUTLIER_T], sa = 1.0f;
    size_t t = 0;
    int rc = FRO_OK;
    if (m == 1) {
        a8 = (int8_t*)malloc(nz(k));
        rc = fro_quant_row(a, k, a8, &sa, oidx, oval, &t);
        if (rc) { free(a8); return rc; }
    }
    size_t total = (m == 1) ? n : m;
    for (int w = 0; w < nthreads; w++) {
        mt_job* J = &jobs[w];
        J->a = a; J->m = m; J->k = k; J->n = n; J->wt = wt; J->scale = scale;
        J->out = out; J->by_rows = (m != 1);
        J->lo = total * (size_t)w / (size_t)nthreads;
        J->hi = total * (size_t)(w + 1) / (size_t)nthreads;
        J->a8 = a8; J->sa = sa; J->oidx = oidx; J->oval = oval; J->t = t; J->rc = 0;
        pthread_create(&th[w], NULL, mt_worker, J);
    }
    for (int w = 0; w < nthreads; w++) {
        pthread_join(th[w], NULL);
        if (jobs[w].rc) rc = jobs[w].rc;
    }
    free(a8);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* int4 (W4A32)                                                              */
/* ------------------------------------------------------------------------ */
/* Sign-extended nibble i of a packed row: src/bundle.rs:61-66. */
static int nib_s4(const uint8_t* prow, size_t i) {
    uint8_t b = prow[i / 2];
    uint8_t v = (i % 2 == 0) ? (b & 0x0F) : (b >> 4);
    return (int)(int8_t)(uint8_t)(v << 4) >> 4;
}

/* i4_dot scalar fold: src/bundle.rs:90-113 (== jit.rs:362-378). */
float fro_i4_dot(const uint8_t* prow, const float* a, const float* scale,
                 size_t g, size_t k) {
    float sum = 0.0f;
    size_t gi = 0, kk = 0;
    while (kk < k) {
        size_t hi = kk + g < k ? kk + g : k;
        float gsum = 0.0f;
        for (; kk < hi; kk++) gsum = gsum + a[kk] * (float)nib_s4(prow, kk);
        sum = sum + scale[gi] * gsum;
        gi++;
    }
    return sum;
}

/* i4_dot_avx2: src/bundle.rs:199-225, the order the x86 production build
 * takes (dispatch at 91-96).  Per group: 8 lane accumulators, each an FMA
 * chain over the 8-nibble chunks (unpack8_nibbles 186-193 reads 4 bytes at
 * kk/2, i.e. nibbles 2*(kk/2)..+8), then hsum256 (146-153):
 * ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)), then a scalar mul+add tail, then
 * sum += scale*gsum. */
FRO_FMA float fro_i4_dot_avx2(const uint8_t* prow, const float* a, const float* scale,
                      size_t g, size_t k) {
    float sum = 0.0f;
    size_t gi = 0, kk = 0;
    while (kk < k) {
        size_t hi = kk + g < k ? kk + g : k;
        float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        while (kk + 8 <= hi) {
            size_t base = (kk / 2) * 2;
            for (int q = 0; q < 8; q++)
                l[q] = fmaf((float)nib_s4(prow, base + (size_t)q), a[kk + (size_t)q], l[q]);
            kk += 8;
        }
        float q0 = l[0] + l[4], q1 = l[1] + l[5], q2 = l[2] + l[6], q3 = l[3] + l[7];
        float d0 = q0 + q2, d1 = q1 + q3;
        float gsum = d0 + d1;
        for (; kk < hi; kk++) gsum = gsum + a[kk] * (float)nib_s4(prow, kk);
        sum = sum + scale[gi] * gsum;
        gi++;
    }
    return sum;
}

/* f32 GEMM where the reference calls ndarray's a.dot: ndarray 0.16.1 hands
 * every f32 Array2 product to matrixmultiply 0.3.10's sgemm (Cargo.lock:1108,
 * 1207; the default build has no BLAS feature, Cargo.toml:27).  That crate's
 * published algorithm (gemm.rs gemm_loop, the BLIS loop nest) fixes each
 * output element's summation order, whatever m, n and the strides:
 *   - k is split into blocks of KC = 256 (archparam S_KC), in order;
 *   - per block, the micro-kernel (the FMA one on an x86-64 host with
 *     avx + fma, selected at run time) accumulates each C element in its own
 *     register lane from +0, k ascending, one fused multiply-add a step;
 *   - the first block stores C = AB (beta = 0), every later one C = C + AB
 *     (beta = 1, alpha = 1: one rounding).
 * fro_mm_dot is that order for one element (x stride xs, w stride ws). */
FRO_FMA float fro_mm_dot(const float* x, size_t xs, const float* w, size_t ws, size_t k) {
    float c = 0.0f;
    for (size_t k0 = 0; k0 < k; k0 += FRO_MM_KC) {
        const size_t k1 = k - k0 > FRO_MM_KC ? k0 + FRO_MM_KC : k;
        float ab = 0.0f;
        for (size_t kk = k0; kk < k1; kk++) ab = fmaf(x[kk * xs], w[kk * ws], ab);
        c = k0 == 0 ? ab : c + ab;
    }
    return c;
}

void fro_sgemm(const float* x, size_t m, size_t k, const float* w, size_t n,
               float* y) {
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) y[i * n + j] = fro_mm_dot(x + i * k, 1, w + j, n, k);
}

/* Bundle::mm I4 arm: src/bundle.rs:760-799.  M==1 -> i4_dot per output
 * column (767-776, AVX2 order on x86); M>1 -> dequantise
 * w[kk,col] = s4 * scale[j, kk/g] (784-790) then a.dot(w). */
int fro_mm_i4(const float* a, size_t m, size_t k, const uint8_t* packed,
              const float* scale, size_t n, size_t g, float* out) {
    size_t ng = (k + g - 1) / g, rb = (k + 1) / 2;
    if (m == 1) {
        for (size_t j = 0; j < n; j++)
            out[j] = fro_i4_dot_avx2(packed + j * rb, a, scale + j * ng, g, k);
        return FRO_OK;
    }
    float* wcol = (float*)malloc(nz(k) * sizeof(float));
    for (size_t j = 0; j < n; j++) {
        for (size_t kk = 0; kk < k; kk++)
            wcol[kk] = (float)nib_s4(packed + j * rb, kk) * scale[j * ng + kk / g];
        for (size_t i = 0; i < m; i++) {
            out[i * n + j] = fro_mm_dot(a + i * k, 1, wcol, 1, k);
        }
    }
    free(wcol);
    return FRO_OK;
}

/* expert_f32 i8 arm + expert_mm: src/bundle.rs:410-420, 457-461.
 * v[i,j] = (raw[i,j] as f32) * scale[j]; y = x . v  (W8A32). */
void fro_expert_mm_i8(const float* x, size_t m, const int8_t* raw,
                      const float* scale, size_t inp, size_t out, float* y) {
    const fro_expert_t e = {FRO_DT_I8, raw, scale, NULL, 0};
    fro_expert_mm(&e, x, m, inp, out, y);
}

/* silu: src/qwen3moe.rs:38-40. */
float fro_silu(float x) { return x / (1.0f + expf(-x)); }

/* gelu_tanh: src/gemma4.rs:61-64 (c = sqrt(2/pi) computed in f32). */
float fro_gelu_tanh(float x) {
    float c = sqrtf(2.0f / 3.14159274101257324f);
    return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

/* Routing.  qwen3moe: softmax_rows (src/qwen3moe.rs:42-52; max, exp,
 * sequential sum, divide), stable sort desc (129; ties -> lower expert),
 * truncate to topk (130), w = p/denom with denom the sum over the top-k in
 * sorted order when norm_topk (131-134).  gemma4 (src/gemma4.rs:146-161)
 * always renormalises and multiplies by per_expert_scale[e]. */
typedef struct { float p; int32_t e; } pe_t;
static int pe_cmp(const void* x, const void* y) {
    const pe_t* a = (const pe_t*)x;
    const pe_t* b = (const pe_t*)y;
    if (a->p > b->p) return -1;
    if (a->p < b->p) return 1;
    return a->e < b->e ? -1 : (a->e > b->e);
}

void fro_moe_route(const float* logits, size_t T, size_t E, size_t topk,
                   int norm_topk, const float* pes, int32_t* sel, float* w,
                   float* probs) {
    float* p = (float*)malloc(nz(E) * sizeof(float));
    pe_t* v = (pe_t*)malloc(nz(E) * sizeof(pe_t));
    for (size_t t = 0; t < T; t++) {
        const float* row = logits + t * E;
        float m = -INFINITY;
        for (size_t e = 0; e < E; e++) m = fmaxf(m, row[e]);
        float s = 0.0f;
        for (size_t e = 0; e < E; e++) { p[e] = expf(row[e] - m); s = s + p[e]; }
        for (size_t e = 0; e < E; e++) p[e] = p[e] / s;
        if (probs) memcpy(probs + t * E, p, E * sizeof(float));
        for (size_t e = 0; e < E; e++) { v[e].p = p[e]; v[e].e = (int32_t)e; }
        qsort(v, E, sizeof(pe_t), pe_cmp); /* (p desc, e asc) == stable desc */
        float denom = 1.0f;
        if (norm_topk || pes) {
            denom = -0.0f;
            for (size_t i = 0; i < topk; i++) denom = denom + v[i].p;
        }
        for (size_t i = 0; i < topk; i++) {
            sel[t * topk + i] = v[i].e;
            float wi = v[i].p / denom;
            if (pes) wi = wi * pes[v[i].e];
            w[t * topk + i] = wi;
        }
    }
    free(p);
    free(v);
}

/* Routed expert layer: src/qwen3moe.rs:120-158 (act 0) and the expert part
 * of src/gemma4.rs:162-185 (act 1).  For each active expert the tokens routed
 * to it are gathered, gate/up (or packed gate_up) -> act -> down via
 * expert_mm, and out[t,:] += w * down (mul then add).  The reference visits
 * experts in HashMap order (random per process); here ascending expert id.
 * fro_moe_mt runs the experts' matmuls on nthreads threads (each expert's
 * rows are independent) and then combines on one thread in ascending expert
 * id, so its output is the same for any thread count. */
typedef struct {
    const float* x; size_t T, d, topk, mi, E; int act;
    const int32_t* sel; const float* w;
    const fro_expert_t* gate; const fro_expert_t* up; const fro_expert_t* down;
    float* dn;  /* (T*topk, d): the down output of (t, slot) */
    int w0, nw;
} moe_job;

static void* moe_worker(void* arg) {
    const moe_job* J = (const moe_job*)arg;
    const size_t T = J->T, d = J->d, topk = J->topk, mi = J->mi;
    const size_t gw = J->act == 1 ? 2 * mi : mi;
    float* rows = (float*)malloc(nz(T * d) * sizeof(float));
    float* g = (float*)malloc(nz(T * gw) * sizeof(float));
    float* u = (float*)malloc(nz(T * mi) * sizeof(float));
    float* h = (float*)malloc(nz(T * mi) * sizeof(float));
    float* dn = (float*)malloc(nz(T * d) * sizeof(float));
    size_t* tok = (size_t*)malloc(nz(T) * sizeof(size_t));
    for (size_t e = (size_t)J->w0; e < J->E; e += (size_t)J->nw) {
        size_t nt = 0;
        for (size_t t = 0; t < T; t++)
            for (size_t i = 0; i < topk; i++)
                if ((size_t)J->sel[t * topk + i] == e) tok[nt++] = t * topk + i;
        if (!nt) continue;
        for (size_t r = 0; r < nt; r++) memcpy(rows + r * d, J->x + tok[r] / topk * d, d * sizeof(float));
        fro_expert_mm(&J->gate[e], rows, nt, d, gw, g);
        if (J->act == 0) {
            fro_expert_mm(&J->up[e], rows, nt, d, mi, u);
            for (size_t i = 0; i < nt * mi; i++) h[i] = fro_silu(g[i]) * u[i];
        } else {
            for (size_t r = 0; r < nt; r++)
                for (size_t c = 0; c < mi; c++)
                    h[r * mi + c] = fro_gelu_tanh(g[r * gw + c]) * g[r * gw + c + mi];
        }
        fro_expert_mm(&J->down[e], h, nt, mi, d, dn);
        for (size_t r = 0; r < nt; r++) memcpy(J->dn + tok[r] * d, dn + r * d, d * sizeof(float));
    }
    free(rows); free(g); free(u); free(h); free(dn); free(tok);
    return NULL;
}

int fro_moe_ex_mt(const float* x, size_t T, size_t d, const float* logits, size_t E,
                  size_t topk, int norm_topk, const float* pes, size_t mi, int act,
                  const fro_expert_t* gate, const fro_expert_t* up, const fro_expert_t* down,
                  float* out, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    int32_t* sel = (int32_t*)malloc(nz(T * topk) * sizeof(int32_t));
    float* w = (float*)malloc(nz(T * topk) * sizeof(float));
    float* dn = (float*)malloc(nz(T * topk * d) * sizeof(float));
    fro_moe_route(logits, T, E, topk, norm_topk, pes, sel, w, NULL);
    moe_job jobs[64];
    pthread_t th[64];
    for (int i = 0; i < nthreads; i++) {
        moe_job J = {x, T, d, topk, mi, E, act, sel, w, gate, up, down, dn, i, nthreads};
        jobs[i] = J;
    }
    if (nthreads == 1) {
        moe_worker(&jobs[0]);
    } else {
        for (int i = 0; i < nthreads; i++) pthread_create(&th[i], NULL, moe_worker, &jobs[i]);
        for (int i = 0; i < nthreads; i++) pthread_join(th[i], NULL);
    }
    memset(out, 0, T * d * sizeof(float));
    for (size_t e = 0; e < E; e++)
        for (size_t t = 0; t < T; t++)
            for (size_t i = 0; i < topk; i++)
                if ((size_t)sel[t * topk + i] == e) {
                    const float tw = w[t * topk + i];
                    const float* r = dn + (t * topk + i) * d;
                    for (size_t c = 0; c < d; c++) out[t * d + c] = out[t * d + c] + tw * r[c];
                }
    free(sel); free(w); free(dn);
    return FRO_OK;
}

/* The int8 bank (every expert an i8 (in,out) array with f32 scales). */
int fro_moe_mt(const float* x, size_t T, size_t d, const float* logits, size_t E,
               size_t topk, int norm_topk, const float* pes, size_t mi, int act,
               const int8_t* const* gate, const float* const* gate_scale,
               const int8_t* const* up, const float* const* up_scale,
               const int8_t* const* down, const float* const* down_scale,
               float* out, int nthreads) {
    fro_expert_t* ex = (fro_expert_t*)calloc(nz(3 * E), sizeof(fro_expert_t));
    for (size_t e = 0; e < E; e++) {
        ex[e] = (fro_expert_t){FRO_DT_I8, gate[e], gate_scale[e], NULL, 0};
        if (act == 0) ex[E + e] = (fro_expert_t){FRO_DT_I8, up[e], up_scale[e], NULL, 0};
        ex[2 * E + e] = (fro_expert_t){FRO_DT_I8, down[e], down_scale[e], NULL, 0};
    }
    int rc = fro_moe_ex_mt(x, T, d, logits, E, topk, norm_topk, pes, mi, act, ex, ex + E, ex + 2 * E, out,
                           nthreads);
    free(ex);
    return rc;
}

int fro_moe(const float* x, size_t T, size_t d, const float* logits, size_t E,
            size_t topk, int norm_topk, const float* pes, size_t mi, int act,
            const int8_t* const* gate, const float* const* gate_scale,
            const int8_t* const* up, const float* const* up_scale,
            const int8_t* const* down, const float* const* down_scale,
            float* out) {
    return fro_moe_mt(x, T, d, logits, E, topk, norm_topk, pes, mi, act, gate, gate_scale, up,
                      up_scale, down, down_scale, out, 1);
}

/* ------------------------------------------------------------------------ */
/* The unembed row dot: Bundle::rowdot_f32 (src/bundle.rs:958-987) and       */
/* rowdot_f32_subset (995-1015).                                             */
/* ------------------------------------------------------------------------ */
/* One row.  f32 (dtype 3) / f16 (4): the iterator fold of w * x from -0.0
 * (Rust 1.89's f32 Sum; rust-version in the reference's Cargo.toml), a mul
 * then an add (967-968).  rowi8 (5), full: scale * rowi8_dot_avx2 (158-178),
 * the order the x86 build takes (975-978): 8 lane accumulators from +0.0,
 * lane q an FMA chain over k = 8i + q, hsum256 (146-153), then a mul + add
 * tail.  rowi8, subset (or a host without AVX2+FMA, 980): scale * the fold
 * from -0.0 (1011). */
FRO_FMA static float row_dot(int dtype, const void* data, const float* scale, size_t r,
                     size_t d, const float* x, int avx2) {
    if (dtype == 3) {
        const float* w = (const float*)data + r * d;
        float s = -0.0f;
        for (size_t k = 0; k < d; k++) s = s + w[k] * x[k];
        return s;
    }
    if (dtype == 4) {
        const uint16_t* w = (const uint16_t*)data + r * d;
        float s = -0.0f;
        for (size_t k = 0; k < d; k++) s = s + fro_f16_to_f32(w[k]) * x[k];
        return s;
    }
    const int8_t* w = (const int8_t*)data + r * d;
    if (!avx2) {
        float s = -0.0f;
        for (size_t k = 0; k < d; k++) s = s + (float)w[k] * x[k];
        return scale[r] * s;
    }
    float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t kk = 0;
    for (; kk + 8 <= d; kk += 8)
        for (int q = 0; q < 8; q++) l[q] = fmaf((float)w[kk + (size_t)q], x[kk + (size_t)q], l[q]);
    float q0 = l[0] + l[4], q1 = l[1] + l[5], q2 = l[2] + l[6], q3 = l[3] + l[7];
    float sum = (q0 + q2) + (q1 + q3);
    for (; kk < d; kk++) sum = sum + (float)w[kk] * x[kk];
    return scale[r] * sum;
}

void fro_rowdot_f32(int dtype, const void* data, const float* scale, size_t rows,
                    size_t d, const float* x, float* out) {
    for (size_t r = 0; r < rows; r++) out[r] = row_dot(dtype, data, scale, r, d, x, 1);
}

void fro_rowdot_f32_subset(int dtype, const void* data, const float* scale,
                           size_t rows, size_t d, const float* x,
                           const int64_t* cand, size_t ncand, float* out) {
    for (size_t i = 0; i < ncand; i++) {
        const int64_t c = cand[i];
        out[i] = (c < 0 || (uint64_t)c >= rows) ? -INFINITY
                                                : row_dot(dtype, data, scale, (size_t)c, d, x, 0);
    }
}

/* ------------------------------------------------------------------------ */
/* GPT-2 greedy decode with a KV cache: Gpt2::generate (src/composition.rs:  */
/* 317-341; int8 cache 251-270), forward_block (175-209), forward_block_q    */
/* (214-249), head_argmax (296-300), layernorm / gelu / softmax_rows (20-50).*/
/* ------------------------------------------------------------------------ */

/* ndarray 0.16.1 ArrayBase::sum over a contiguous row: numeric_util::
 * unrolled_fold (eight partial sums p0..p7 from 0, combined as acc += p0+p4,
 * p1+p5, p2+p6, p3+p7, then the < 8 tail in order).  layernorm's mean
 * (composition.rs:24) goes through it. */
float fro_nd_sum(const float* x, size_t n) {
    float p[8] = {0, 0, 0, 0, 0, 0, 0, 0}, acc = 0.0f;
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int q = 0; q < 8; q++) p[q] = p[q] + x[i + q];
    acc = acc + (p[0] + p[4]);
    acc = acc + (p[1] + p[5]);
    acc = acc + (p[2] + p[6]);
    acc = acc + (p[3] + p[7]);
    for (; i < n; i++) acc = acc + x[i];
    return acc;
}

/* layernorm (composition.rs:20-33): eps 1e-5, mean by nd_sum, variance a
 * fold from -0.0 (Iterator::sum), (v - mu) * inv * g + b with no FMA. */
void fro_layernorm(const float* x, size_t m, size_t d, const float* g, const float* b, float* out) {
    const float n = (float)d;
    for (size_t r = 0; r < m; r++) {
        const float* row = x + r * d;
        const float mu = fro_nd_sum(row, d) / n;
        float var = -0.0f;
        for (size_t i = 0; i < d; i++) var = var + (row[i] - mu) * (row[i] - mu);
        var = var / n;
        const float inv = 1.0f / sqrtf(var + 1e-5f);
        for (size_t i = 0; i < d; i++) out[r * d + i] = (row[i] - mu) * inv * g[i] + b[i];
    }
}

/* softmax_rows (composition.rs:40-50) on one row. */
static void softmax_row(float* v, size_t n) {
    float mx = -INFINITY;
    for (size_t j = 0; j < n; j++) mx = fmaxf(mx, v[j]);
    float s = 0.0f;
    for (size_t j = 0; j < n; j++) { v[j] = expf(v[j] - mx); s = s + v[j]; }
    for (size_t j = 0; j < n; j++) v[j] = v[j] / s;
}

typedef struct {
    const fro_gpt2_t* g;
    int nthreads;
    int kv8;
    size_t total;
    float** kc; float** vc;          /* f32 cache (total, d) per layer */
    int8_t** kq; int8_t** vq;        /* int8 cache (total, d) per layer */
    float** ks; float** vs;          /* int8 cache scales (total, n_head) */
} g2_run;

/* q8 of forward_block_q (composition.rs:220): (v / sc).round() clamped. */
static int8_t kv_q8(float v, float sc) {
    float q = roundf(v / sc);
    if (q != q) return 0; /* Rust's `as i8` saturates NaN to 0 */
    if (q < -127.0f) q = -127.0f;
    if (q > 127.0f) q = 127.0f;
    return (int8_t)q;
}

/* forward_block / forward_block_q: m rows at absolute positions cur..cur+m
 * through every layer; x (m, d) in, the pre-final-LN hidden states out (in
 * place).  The attention products are matrixmultiply sgemms in the
 * reference; each output element here is fro_mm_dot (their order). */
static int g2_block(g2_run* R, float* x, size_t m, size_t cur) {
    const fro_gpt2_t* g = R->g;
    const size_t d = g->d, H = g->n_head, hd = d / H, klen = cur + m;
    float* a = (float*)malloc(nz(m * d * 4));
    float* qkv = (float*)malloc(nz(m * 3 * d * 4));
    float* att = (float*)malloc(nz(m * d * 4));
    float* y = (float*)malloc(nz(m * 4 * d * 4));
    float* hm = (float*)malloc(nz(m * 4 * d * 4));
    float* sc = (float*)malloc(nz(m * klen * 4));
    float* kh = (float*)malloc(nz(klen * hd * 4));
    float* vh = (float*)malloc(nz(klen * hd * 4));
    const float rs = sqrtf((float)hd);
    int rc = FRO_OK;
    for (size_t l = 0; l < g->n_layer && !rc; l++) {
        const int8_t* const* W = g->wt + 4 * l;
        const float* const* S = g->scale + 4 * l;
        const float* const* B = g->bias + 4 * l;
        fro_layernorm(x, m, d, g->ln_g[2 * l], g->ln_b[2 * l], a);
        if ((rc = fro_mm_i8_mt(a, m, d, W[0], S[0], 3 * d, qkv, R->nthreads))) break;
        for (size_t i = 0; i < m; i++)
            for (size_t c = 0; c < 3 * d; c++) qkv[i * 3 * d + c] = qkv[i * 3 * d + c] + B[0][c];
        for (size_t i = 0; i < m; i++) {  /* append K/V (quantised per head for int8) */
            const size_t pos = cur + i;
            const float* kr = qkv + i * 3 * d + d;
            const float* vr = qkv + i * 3 * d + 2 * d;
            if (!R->kv8) {
                memcpy(R->kc[l] + pos * d, kr, d * 4);
                memcpy(R->vc[l] + pos * d, vr, d * 4);
            } else {
                for (size_t h = 0; h < H; h++) {
                    float mk = 0.0f, mv = 0.0f;
                    for (size_t c = 0; c < hd; c++) {
                        mk = fmaxf(mk, fabsf(kr[h * hd + c]));
                        mv = fmaxf(mv, fabsf(vr[h * hd + c]));
                    }
                    float sck = mk / 127.0f, scv = mv / 127.0f;
                    if (!(sck > 0.0f)) sck = 1.0f;
                    if (!(scv > 0.0f)) scv = 1.0f;
                    R->ks[l][pos * H + h] = sck;
                    R->vs[l][pos * H + h] = scv;
                    for (size_t c = 0; c < hd; c++) {
                        R->kq[l][pos * d + h * hd + c] = kv_q8(kr[h * hd + c], sck);
                        R->vq[l][pos * d + h * hd + c] = kv_q8(vr[h * hd + c], scv);
                    }
                }
            }
        }
        for (size_t h = 0; h < H; h++) {
            for (size_t j = 0; j < klen; j++)
                for (size_t c = 0; c < hd; c++) {
                    if (!R->kv8) {
                        kh[j * hd + c] = R->kc[l][j * d + h * hd + c];
                        vh[j * hd + c] = R->vc[l][j * d + h * hd + c];
                    } else {
                        kh[j * hd + c] = (float)R->kq[l][j * d + h * hd + c] * R->ks[l][j * H + h];
                        vh[j * hd + c] = (float)R->vq[l][j * d + h * hd + c] * R->vs[l][j * H + h];
                    }
                }
            for (size_t i = 0; i < m; i++) {
                const float* q = qkv + i * 3 * d + h * hd;
                float* s = sc + i * klen;
                for (size_t j = 0; j < klen; j++) {
                    s[j] = fro_mm_dot(q, 1, kh + j * hd, 1, hd) / rs;
                }
                for (size_t j = cur + i + 1; j < klen; j++) s[j] = -1e10f;  /* causal mask */
                softmax_row(s, klen);
                for (size_t c = 0; c < hd; c++) {
                    att[i * d + h * hd + c] = fro_mm_dot(s, 1, vh + c, hd, klen);
                }
            }
        }
        if ((rc = fro_mm_i8_mt(att, m, d, W[1], S[1], d, y, R->nthreads))) break;
        for (size_t i = 0; i < m * d; i++) x[i] = x[i] + (y[i] + B[1][i % d]);
        fro_layernorm(x, m, d, g->ln_g[2 * l + 1], g->ln_b[2 * l + 1], a);
        if ((rc = fro_mm_i8_mt(a, m, d, W[2], S[2], 4 * d, hm, R->nthreads))) break;
        for (size_t i = 0; i < m * 4 * d; i++) hm[i] = fro_gelu_tanh(hm[i] + B[2][i % (4 * d)]);
        if ((rc = fro_mm_i8_mt(hm, m, 4 * d, W[3], S[3], d, y, R->nthreads))) break;
        for (size_t i = 0; i < m * d; i++) x[i] = x[i] + (y[i] + B[3][i % d]);
    }
    free(a); free(qkv); free(att); free(y); free(hm); free(sc); free(kh); free(vh);
    return rc;
}

typedef struct { const fro_gpt2_t* g; const float* x; float* out; size_t lo, hi; } g2_head_job;
static void* g2_head_worker(void* p) {
    g2_head_job* J = (g2_head_job*)p;
    fro_rowdot_f32(FRO_DT_F16, J->g->wte + J->lo * J->g->d, NULL, J->hi - J->lo, J->g->d, J->x, J->out + J->lo);
    return NULL;
}

/* head_argmax (composition.rs:296-300): ln_f of the last row, the tied
 * unembed rowdot_f32("wte") over f16 rows, then Iterator::max_by with
 * partial_cmp (the last of equal maxima; a NaN panics -> FRO_ERR_NAN). */
static int g2_head(g2_run* R, const float* xlast, float* logits, int64_t* tok) {
    const fro_gpt2_t* g = R->g;
    float* xf = (float*)malloc(nz(g->d * 4));
    fro_layernorm(xlast, 1, g->d, g->ln_f_g, g->ln_f_b, xf);
    int nt = R->nthreads < 1 ? 1 : (R->nthreads > 64 ? 64 : R->nthreads);
    pthread_t th[64];
    g2_head_job jobs[64];
    for (int w = 0; w < nt; w++) {
        jobs[w] = (g2_head_job){g, xf, logits, g->vocab * (size_t)w / nt, g->vocab * (size_t)(w + 1) / nt};
        pthread_create(&th[w], NULL, g2_head_worker, &jobs[w]);
    }
    for (int w = 0; w < nt; w++) pthread_join(th[w], NULL);
    free(xf);
    size_t best = 0;
    for (size_t r = 0; r < g->vocab; r++) {
        if (isnan(logits[r])) return FRO_ERR_NAN;
        if (logits[r] >= logits[best]) best = r;
    }
    *tok = (int64_t)best;
    return FRO_OK;
}

/* rows_f32("wte", ids) + rows_f32("wpe", pos) (bundle.rs:936-955). */
static int g2_embed(const fro_gpt2_t* g, const int64_t* ids, size_t m, size_t pos0, float* x) {
    for (size_t t = 0; t < m; t++) {
        if (ids[t] < 0 || (size_t)ids[t] >= g->vocab || pos0 + t >= g->n_pos) return FRO_ERR_ARG;
        for (size_t c = 0; c < g->d; c++)
            x[t * g->d + c] = fro_f16_to_f32(g->wte[(size_t)ids[t] * g->d + c]) + g->wpe[(pos0 + t) * g->d + c];
    }
    return FRO_OK;
}

int fro_gpt2_generate(const fro_gpt2_t* g, const int64_t* prompt, size_t n_prompt, size_t n_new, int kv_int8,
                      int nthreads, int64_t* out, float* logits) {
    if (!n_prompt || !n_new) return FRO_ERR_ARG;
    const size_t d = g->d, L = g->n_layer, total = n_prompt + n_new;
    g2_run R = {g, nthreads, kv_int8, total, NULL, NULL, NULL, NULL, NULL, NULL};
    R.kc = (float**)calloc(L, sizeof(float*)); R.vc = (float**)calloc(L, sizeof(float*));
    R.kq = (int8_t**)calloc(L, sizeof(int8_t*)); R.vq = (int8_t**)calloc(L, sizeof(int8_t*));
    R.ks = (float**)calloc(L, sizeof(float*)); R.vs = (float**)calloc(L, sizeof(float*));
    for (size_t l = 0; l < L; l++) {
        if (!kv_int8) {
            R.kc[l] = (float*)calloc(total * d, 4); R.vc[l] = (float*)calloc(total * d, 4);
        } else {
            R.kq[l] = (int8_t*)calloc(total * d, 1); R.vq[l] = (int8_t*)calloc(total * d, 1);
            R.ks[l] = (float*)calloc(total * g->n_head, 4); R.vs[l] = (float*)calloc(total * g->n_head, 4);
        }
    }
    float* x = (float*)malloc(nz(n_prompt * d * 4));
    float* lg = (float*)malloc(nz(g->vocab * 4));
    int64_t next = 0;
    int rc = g2_embed(g, prompt, n_prompt, 0, x);
    if (!rc) rc = g2_block(&R, x, n_prompt, 0);
    if (!rc) rc = g2_head(&R, x + (n_prompt - 1) * d, lg, &next);
    size_t pos = n_prompt;
    for (size_t s = 0; !rc; s++) {
        out[s] = next;
        if (logits) memcpy(logits + s * g->vocab, lg, g->vocab * 4);
        if (s + 1 == n_new) break;
        rc = g2_embed(g, &next, 1, pos, x);
        if (!rc) rc = g2_block(&R, x, 1, pos);
        if (!rc) rc = g2_head(&R, x, lg, &next);
        pos++;
    }
    for (size_t l = 0; l < L; l++) {
        free(R.kc[l]); free(R.vc[l]); free(R.kq[l]); free(R.vq[l]); free(R.ks[l]); free(R.vs[l]);
    }
    free(R.kc); free(R.vc); free(R.kq); free(R.vq); free(R.ks); free(R.vs);
    free(x); free(lg);
    return rc;
}

/* Model::predict for Gpt2 (composition.rs:304-308): the whole sequence,
 * no cache, the last row's argmax.  hidden() (61-96) is forward_block at
 * cur = 0 over the full sequence (the cache it fills is unused). */
int fro_gpt2_predict(const fro_gpt2_t* g, const int64_t* ids, size_t n, int nthreads, int64_t* tok, float* logits) {
    if (!n) return FRO_ERR_ARG;
    int64_t t = 0;
    float* lg = logits ? logits : (float*)malloc(nz(g->vocab * 4));
    const size_t d = g->d, L = g->n_layer;
    g2_run R = {g, nthreads, 0, n, NULL, NULL, NULL, NULL, NULL, NULL};
    R.kc = (float**)calloc(L, sizeof(float*)); R.vc = (float**)calloc(L, sizeof(float*));
    for (size_t l = 0; l < L; l++) { R.kc[l] = (float*)calloc(n * d, 4); R.vc[l] = (float*)calloc(n * d, 4); }
    float* x = (float*)malloc(nz(n * d * 4));
    int rc = g2_embed(g, ids, n, 0, x);
    if (!rc) rc = g2_block(&R, x, n, 0);
    if (!rc) rc = g2_head(&R, x + (n - 1) * d, lg, &t);
    *tok = t;
    for (size_t l = 0; l < L; l++) { free(R.kc[l]); free(R.vc[l]); }
    free(R.kc); free(R.vc); free(x);
    if (!logits) free(lg);
    return rc;
}

/* The libm calls of the reference's f32 math: Rust's f32::exp reaches the
 * platform expf (llvm.exp.f32 lowers to the libcall), f32::tanh calls tanhf
 * (std's cmath binding), both from the system libm. */
void fro_libm_f32(int fn, const float* x, size_t n, float* out) {
    for (size_t i = 0; i < n; i++) out[i] = fn == 0 ? expf(x[i]) : (fn == 1 ? expm1f(x[i]) : tanhf(x[i]));
}

/* ------------------------------------------------------------------------ */
/* Affine int4 (q4a): w = scale*q + min, q an unsigned nibble                */
/* ------------------------------------------------------------------------ */
static unsigned nib_u4(const uint8_t* prow, size_t i) {
    uint8_t b = prow[i / 2];
    return (i % 2 == 0) ? (b & 0x0Fu) : (b >> 4);
}

/* put_q4a: src/convert.rs:223-260.  g = min(Q4A_GROUP = 32, in) (33-36);
 * per (out j, group): mn / mx folds from +-inf, scale = max((mx - mn) / 15,
 * 1e-8), min = mn; q = clamp(round_ties_even((v - min) / scale), 0, 15)
 * from the f32 scale / min; scale and min stored f16 (put_f16, RNE). */
size_t fro_put_q4a(const float* data, size_t rows, size_t cols, int transpose, uint8_t* packed,
                   uint16_t* scale_f16, uint16_t* min_f16) {
    size_t out = transpose ? rows : cols, inp = transpose ? cols : rows;
#define AT(i, j) (transpose ? data[(j) * inp + (i)] : data[(i) * out + (j)])
    size_t g = 32 < nz(inp) ? 32 : nz(inp);
    size_t ng = (inp + g - 1) / g, rb = (inp + 1) / 2;
    float* sc = (float*)malloc(nz(out * ng) * sizeof(float));
    float* mnv = (float*)malloc(nz(out * ng) * sizeof(float));
    for (size_t j = 0; j < out; j++)
        for (size_t gi = 0; gi < ng; gi++) {
            size_t lo = gi * g, hi = (gi + 1) * g < inp ? (gi + 1) * g : inp;
            float mn = INFINITY, mx = -INFINITY;
            for (size_t i = lo; i < hi; i++) { mn = fminf(mn, AT(i, j)); mx = fmaxf(mx, AT(i, j)); }
            float s = (mx - mn) / 15.0f;
            sc[j * ng + gi] = fmaxf(s, 1e-8f);
            mnv[j * ng + gi] = mn;
        }
    memset(packed, 0, out * rb);
    for (size_t j = 0; j < out; j++)
        for (size_t i = 0; i < inp; i++) {
            size_t gi = j * ng + i / g;
            uint8_t q = (uint8_t)clampf(round_ties_even((AT(i, j) - mnv[gi]) / sc[gi]), 0.0f, 15.0f);
            packed[j * rb + i / 2] |= (i % 2 == 0) ? q : (uint8_t)(q << 4);
        }
    for (size_t i = 0; i < out * ng; i++) {
        scale_f16[i] = fro_f32_to_f16(sc[i]);
        min_f16[i] = fro_f32_to_f16(mnv[i]);
    }
    free(sc);
    free(mnv);
    return g;
#undef AT
}

/* q4a_dot, the scalar form (src/bundle.rs:118-143): per group qsum += a*q,
 * asum += a; sum += scale*qsum + min*asum. */
float fro_q4a_dot(const uint8_t* prow, const float* a, const float* scale, const float* mins, size_t g, size_t k) {
    float sum = 0.0f;
    size_t gi = 0, kk = 0;
    while (kk < k) {
        size_t hi = kk + g < k ? kk + g : k;
        float qsum = 0.0f, asum = 0.0f;
        for (; kk < hi; kk++) {
            qsum = qsum + a[kk] * (float)nib_u4(prow, kk);
            asum = asum + a[kk];
        }
        sum = sum + (scale[gi] * qsum + mins[gi] * asum);
        gi++;
    }
    return sum;
}

/* q4a_dot_avx2 (src/bundle.rs:231-258), the x86 production order (dispatch
 * 121-124): per group two sets of 8 lane accumulators, q lanes an FMA chain
 * (q * a), a lanes an add chain, over the 8-nibble chunks read from byte
 * kk/2 (unpack8_nibbles); each set through hsum256; a mul+add tail; then
 * sum += scale*qsum + min*asum. */
FRO_FMA float fro_q4a_dot_avx2(const uint8_t* prow, const float* a, const float* scale, const float* mins, size_t g,
                       size_t k) {
    float sum = 0.0f;
    size_t gi = 0, kk = 0;
    while (kk < k) {
        size_t hi = kk + g < k ? kk + g : k;
        float l[8] = {0, 0, 0, 0, 0, 0, 0, 0}, m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        while (kk + 8 <= hi) {
            size_t base = (kk / 2) * 2;
            for (int q = 0; q < 8; q++) {
                l[q] = fmaf((float)nib_u4(prow, base + (size_t)q), a[kk + (size_t)q], l[q]);
                m[q] = m[q] + a[kk + (size_t)q];
            }
            kk += 8;
        }
        float qsum = ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7]));
        float asum = ((m[0] + m[4]) + (m[2] + m[6])) + ((m[1] + m[5]) + (m[3] + m[7]));
        for (; kk < hi; kk++) {
            qsum = qsum + a[kk] * (float)nib_u4(prow, kk);
            asum = asum + a[kk];
        }
        sum = sum + (scale[gi] * qsum + mins[gi] * asum);
        gi++;
    }
    return sum;
}

/* Bundle::mm Q4A arm: src/bundle.rs:802-845.  M==1 -> q4a_dot per output
 * column (AVX2 order); M>1 -> w[kk,col] = scale*q + min (f32, mul then
 * add, 826-829) then a.dot(w) (fro_mm_dot: matrixmultiply's order). */
int fro_mm_q4a(const float* a, size_t m, size_t k, const uint8_t* packed, const float* scale, const float* mins,
               size_t n, size_t g, float* out) {
    size_t ng = (k + g - 1) / g, rb = (k + 1) / 2;
    if (m == 1) {
        for (size_t j = 0; j < n; j++)
            out[j] = fro_q4a_dot_avx2(packed + j * rb, a, scale + j * ng, mins + j * ng, g, k);
        return FRO_OK;
    }
    float* wcol = (float*)malloc(nz(k) * sizeof(float));
    for (size_t j = 0; j < n; j++) {
        for (size_t kk = 0; kk < k; kk++) {
            size_t gi = j * ng + kk / g;
            wcol[kk] = scale[gi] * (float)nib_u4(packed + j * rb, kk) + mins[gi];
        }
        for (size_t i = 0; i < m; i++) {
            out[i * n + j] = fro_mm_dot(a + i * k, 1, wcol, 1, k);
        }
    }
    free(wcol);
    return FRO_OK;
}

/* expert_f32: src/bundle.rs:404-454, one arm per stored dtype, each value
 * as the reference forms it (f32 arithmetic, no contraction):
 *   i8  (410-420)  v[i,j] = (q[i,j] as f32) * scale[j]
 *   i4  (421-433)  v[i,j] = (s4(nib(j,i)) as f32) * scale[j*ng + i/g]
 *                  (stored (out,in), transposed while dequantising)
 *   q4a (434-448)  v[i,j] = scale[gi] * (u4(nib(j,i)) as f32) + mins[gi]
 *   f16 (449)      v = f16 -> f32;  f32 (450) as stored. */
int fro_expert_f32(const fro_expert_t* e, size_t inp, size_t out, float* v) {
    switch (e->dtype) {
        case FRO_DT_I8: {
            const int8_t* q = (const int8_t*)e->raw;
            for (size_t i = 0; i < inp; i++)
                for (size_t j = 0; j < out; j++) v[i * out + j] = (float)q[i * out + j] * e->scale[j];
            return FRO_OK;
        }
        case FRO_DT_I4:
        case FRO_DT_Q4A: {
            const uint8_t* p = (const uint8_t*)e->raw;
            const size_t g = e->g, ng = (inp + g - 1) / g, rb = (inp + 1) / 2;
            for (size_t j = 0; j < out; j++)
                for (size_t i = 0; i < inp; i++) {
                    const size_t gi = j * ng + i / g;
                    v[i * out + j] = e->dtype == FRO_DT_I4
                                         ? (float)nib_s4(p + j * rb, i) * e->scale[gi]
                                         : e->scale[gi] * (float)nib_u4(p + j * rb, i) + e->mins[gi];
                }
            return FRO_OK;
        }
        case FRO_DT_F16:
            fro_f16_to_f32_n((const uint16_t*)e->raw, v, inp * out);
            return FRO_OK;
        case FRO_DT_F32:
            memcpy(v, e->raw, inp * out * sizeof(float));
            return FRO_OK;
        default:
            return FRO_ERR_ARG;
    }
}

/* expert_mm: src/bundle.rs:457-461, x.dot(&expert_f32) (fro_sgemm). */
int fro_expert_mm(const fro_expert_t* e, const float* x, size_t m, size_t inp, size_t out, float* y) {
    float* v = (float*)malloc(nz(inp * out) * sizeof(float));
    int rc = fro_expert_f32(e, inp, out, v);
    if (rc == FRO_OK) fro_sgemm(x, m, inp, v, out, y);
    free(v);
    return rc;
}

/* fro_mm_i4 with the output columns split over nthreads threads (each
 * column's arithmetic as fro_mm_i4's: identical results). */
typedef struct { const float* a; size_t m, k; const uint8_t* packed; const float* scale; size_t n, g; float* out;
                 size_t lo, hi; } i4_job;
static void* i4_worker(void* p) {
    i4_job* J = (i4_job*)p;
    size_t ng = (J->k + J->g - 1) / J->g, rb = (J->k + 1) / 2;
    if (J->m == 1) {
        for (size_t j = J->lo; j < J->hi; j++)
            J->out[j] = fro_i4_dot_avx2(J->packed + j * rb, J->a, J->scale + j * ng, J->g, J->k);
        return NULL;
    }
    float* wcol = (float*)malloc(nz(J->k) * sizeof(float));
    for (size_t j = J->lo; j < J->hi; j++) {
        for (size_t kk = 0; kk < J->k; kk++)
            wcol[kk] = (float)nib_s4(J->packed + j * rb, kk) * J->scale[j * ng + kk / J->g];
        for (size_t i = 0; i < J->m; i++) {
            J->out[i * J->n + j] = fro_mm_dot(J->a + i * J->k, 1, wcol, 1, J->k);
        }
    }
    free(wcol);
    return NULL;
}
int fro_mm_i4_mt(const float* a, size_t m, size_t k, const uint8_t* packed, const float* scale, size_t n, size_t g,
                 float* out, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    i4_job jobs[256];
    for (int w = 0; w < nthreads; w++) {
        jobs[w] = (i4_job){a, m, k, packed, scale, n, g, out, n * (size_t)w / nthreads, n * (size_t)(w + 1) / nthreads};
        pthread_create(&th[w], NULL, i4_worker, &jobs[w]);
    }
    for (int w = 0; w < nthreads; w++) pthread_join(th[w], NULL);
    return FRO_OK;
}

static int lin_mm(const fro_lin_t* L, const float* a, size_t m, float* out, int nthreads) {
    if (L->dtype == 2) return fro_mm_i4_mt(a, m, L->k, L->packed, L->scale, L->n, L->g, out, nthreads);
    if (L->dtype == 3) return fro_mm_q4a(a, m, L->k, L->packed, L->scale, L->mins, L->n, L->g, out);
    return fro_mm_i8_mt(a, m, L->k, L->wt, L->scale, L->n, out, nthreads);
}

/* ------------------------------------------------------------------------ */
/* Gemma-2 greedy decode with a KV cache: Gemma (src/gemma.rs): norm 66-77,  */
/* rope 79-94, forward_block 242-291, forward_block_q 293-363, head_argmax   */
/* 386-390, generate 403-431 (kv_int8: generate_kv_int8 364-384).            */
/* ------------------------------------------------------------------------ */

/* RMSNorm with the +1 baked gain (gemma.rs:66-77): ms = the fold from -0.0
 * of v*v / n, inv = 1 / sqrt(ms + eps), v * inv * w. */
void fro_rmsnorm(const float* x, size_t m, size_t d, const float* w, float eps, float* out) {
    for (size_t r = 0; r < m; r++) {
        const float* row = x + r * d;
        float ms = -0.0f;
        for (size_t i = 0; i < d; i++) ms = ms + row[i] * row[i];
        ms = ms / (float)d;
        const float inv = 1.0f / sqrtf(ms + eps);
        for (size_t i = 0; i < d; i++) out[r * d + i] = row[i] * inv * w[i];
    }
}

typedef struct {
    const fro_gemma_t* g;
    int nthreads, kv8;
    float* inv;                       /* RoPE inverse frequencies (hd / 2) */
    float** kc; float** vc;           /* f32 cache (total, nkv*hd) per layer */
    int8_t** kq; int8_t** vq;
    float** ks; float** vs;           /* (total, nkv) */
} gm_run;

/* rope (gemma.rs:79-94) on n_heads heads of m rows at positions pos0.. */
static void gm_rope(const gm_run* R, float* x, size_t m, size_t n_heads, size_t pos0) {
    const size_t hd = R->g->hd, half = hd / 2;
    for (size_t i = 0; i < m; i++) {
        float* row = x + i * n_heads * hd;
        for (size_t h = 0; h < n_heads; h++)
            for (size_t j = 0; j < half; j++) {
                const float ang = (float)(pos0 + i) * R->inv[j];
                const float c = cosf(ang), s = sinf(ang);
                const float a = row[h * hd + j], b = row[h * hd + j + half];
                row[h * hd + j] = a * c - b * s;
                row[h * hd + j + half] = b * c + a * s;
            }
    }
}

/* Rope::head_norm (rope.rs:72-87): per head of hd, ms = the fold from -0.0
 * of v*v / hd, inv = 1 / sqrt(ms + eps), v * inv * w[c]. */
static void gm_head_norm(float* x, size_t m, size_t n_heads, size_t hd, const float* w, float eps) {
    for (size_t i = 0; i < m; i++)
        for (size_t h = 0; h < n_heads; h++) {
            float* v = x + (i * n_heads + h) * hd;
            float ms = -0.0f;
            for (size_t c = 0; c < hd; c++) ms = ms + v[c] * v[c];
            ms = ms / (float)hd;
            const float inv = 1.0f / sqrtf(ms + eps);
            for (size_t c = 0; c < hd; c++) v[c] = v[c] * inv * w[c];
        }
}

/* silu (rope.rs:39-41): x / (1 + exp(-x)). */
static float gm_silu(float x) { return x / (1.0f + expf(-x)); }

static int gm_block(gm_run* R, float* x, size_t m, size_t cur) {
    const fro_gemma_t* g = R->g;
    const size_t d = g->d, H = g->n_head, KV = g->n_kv, hd = g->hd, rep = H / KV, kvd = KV * hd, klen = cur + m;
    float* a = (float*)malloc(nz(m * d * 4));
    float* q = (float*)malloc(nz(m * H * hd * 4));
    float* k = (float*)malloc(nz(m * kvd * 4));
    float* v = (float*)malloc(nz(m * kvd * 4));
    float* att = (float*)malloc(nz(m * H * hd * 4));
    float* o = (float*)malloc(nz(m * d * 4));
    float* gate = (float*)malloc(nz(m * g->ffn * 4));
    float* up = (float*)malloc(nz(m * g->ffn * 4));
    float* sc = (float*)malloc(nz(klen * 4));
    float* kh = (float*)malloc(nz(klen * hd * 4));
    float* vh = (float*)malloc(nz(klen * hd * 4));
    int rc = FRO_OK;
    for (size_t l = 0; l < g->n_layer && !rc; l++) {
        const fro_lin_t* L = g->lin + 7 * l;
        const float* const* N = g->norms + 4 * l;
        fro_rmsnorm(x, m, d, N[0], g->eps, a);
        if ((rc = lin_mm(&L[0], a, m, q, R->nthreads)) || (rc = lin_mm(&L[1], a, m, k, R->nthreads)) ||
            (rc = lin_mm(&L[2], a, m, v, R->nthreads)))
            break;
        if (g->arch == 1) {  /* proj: + bias (rope.rs:110-117), then the QK-norm */
            const float* const* B = g->bias + 3 * l;
            float* outs[3] = {q, k, v};
            const size_t wid[3] = {H * hd, kvd, kvd};
            for (int t = 0; t < 3; t++)
                if (B[t])
                    for (size_t i = 0; i < m; i++)
                        for (size_t c = 0; c < wid[t]; c++) outs[t][i * wid[t] + c] = outs[t][i * wid[t] + c] + B[t][c];
            if (g->qk_norm[2 * l]) gm_head_norm(q, m, H, hd, g->qk_norm[2 * l], g->eps);
            if (g->qk_norm[2 * l + 1]) gm_head_norm(k, m, KV, hd, g->qk_norm[2 * l + 1], g->eps);
        }
        gm_rope(R, q, m, H, cur);
        gm_rope(R, k, m, KV, cur);
        for (size_t i = 0; i < m; i++) {  /* append K/V */
            const size_t pos = cur + i;
            if (!R->kv8) {
                memcpy(R->kc[l] + pos * kvd, k + i * kvd, kvd * 4);
                memcpy(R->vc[l] + pos * kvd, v + i * kvd, kvd * 4);
            } else {
                for (size_t kh_ = 0; kh_ < KV; kh_++) {
                    const float* kr = k + i * kvd + kh_ * hd;
                    const float* vr = v + i * kvd + kh_ * hd;
                    float mk = 0.0f, mv = 0.0f;
                    for (size_t c = 0; c < hd; c++) { mk = fmaxf(mk, fabsf(kr[c])); mv = fmaxf(mv, fabsf(vr[c])); }
                    const float sck = fmaxf(mk / 127.0f, 1e-8f), scv = fmaxf(mv / 127.0f, 1e-8f);
                    R->ks[l][pos * KV + kh_] = sck;
                    R->vs[l][pos * KV + kh_] = scv;
                    for (size_t c = 0; c < hd; c++) {
                        R->kq[l][pos * kvd + kh_ * hd + c] = kv_q8(kr[c], sck);
                        R->vq[l][pos * kvd + kh_ * hd + c] = kv_q8(vr[c], scv);
                    }
                }
            }
        }
        const int sliding = g->arch == 0 && l % 2 == 0;
        for (size_t h = 0; h < H; h++) {
            const size_t kv = h / rep;
            for (size_t j = 0; j < klen; j++)
                for (size_t c = 0; c < hd; c++) {
                    if (!R->kv8) {
                        kh[j * hd + c] = R->kc[l][j * kvd + kv * hd + c];
                        vh[j * hd + c] = R->vc[l][j * kvd + kv * hd + c];
                    } else {
                        kh[j * hd + c] = (float)R->kq[l][j * kvd + kv * hd + c] * R->ks[l][j * KV + kv];
                        vh[j * hd + c] = (float)R->vq[l][j * kvd + kv * hd + c] * R->vs[l][j * KV + kv];
                    }
                }
            for (size_t i = 0; i < m; i++) {
                const float* qr = q + i * H * hd + h * hd;
                const size_t abs_ = cur + i;
                for (size_t j = 0; j < klen; j++) {
                    const float acc = fro_mm_dot(qr, 1, kh + j * hd, 1, hd);
                    float s = g->arch == 1 ? acc / sqrtf((float)hd) : acc * g->qscale;
                    if (g->arch == 0 && g->attn_cap > 0.0f) s = g->attn_cap * tanhf(s / g->attn_cap);
                    if (j > abs_ || (sliding && abs_ >= g->window && j <= abs_ - g->window)) s = -1e30f;
                    sc[j] = s;
                }
                softmax_row(sc, klen);
                for (size_t c = 0; c < hd; c++) {
                    att[i * H * hd + h * hd + c] = fro_mm_dot(sc, 1, vh + c, hd, klen);
                }
            }
        }
        if ((rc = lin_mm(&L[3], att, m, o, R->nthreads))) break;
        if (N[1]) {  /* gemma: the post-norm before the residual; rope: x + o */
            fro_rmsnorm(o, m, d, N[1], g->eps, a);
            for (size_t i = 0; i < m * d; i++) x[i] = x[i] + a[i];
        } else {
            for (size_t i = 0; i < m * d; i++) x[i] = x[i] + o[i];
        }
        fro_rmsnorm(x, m, d, N[2], g->eps, a);
        if ((rc = lin_mm(&L[4], a, m, gate, R->nthreads)) || (rc = lin_mm(&L[5], a, m, up, R->nthreads))) break;
        for (size_t i = 0; i < m * g->ffn; i++)
            gate[i] = (g->arch == 1 ? gm_silu(gate[i]) : fro_gelu_tanh(gate[i])) * up[i];
        if ((rc = lin_mm(&L[6], gate, m, o, R->nthreads))) break;
        if (N[3]) {
            fro_rmsnorm(o, m, d, N[3], g->eps, a);
            for (size_t i = 0; i < m * d; i++) x[i] = x[i] + a[i];
        } else {
            for (size_t i = 0; i < m * d; i++) x[i] = x[i] + o[i];
        }
    }
    free(a); free(q); free(k); free(v); free(att); free(o); free(gate); free(up); free(sc); free(kh); free(vh);
    return rc;
}

typedef struct { const fro_gemma_t* g; const float* x; float* out; size_t lo, hi; } gm_head_job;
static void* gm_head_worker(void* p) {
    gm_head_job* J = (gm_head_job*)p;
    const fro_gemma_t* g = J->g;
    const size_t d = g->d, n = J->hi - J->lo;
    if (g->unembed) {
        fro_rowdot_f32(FRO_DT_F16, g->unembed + J->lo * d, NULL, n, d, J->x, J->out + J->lo);
    } else if (g->embed_dt == FRO_DT_F32) {
        fro_rowdot_f32(FRO_DT_F32, (const float*)(const void*)g->embed + J->lo * d, NULL, n, d, J->x, J->out + J->lo);
    } else if (g->embed_dt == FRO_DT_ROWI8) {
        fro_rowdot_f32(FRO_DT_ROWI8, (const int8_t*)(const void*)g->embed + J->lo * d, g->embed_scale + J->lo, n, d,
                       J->x, J->out + J->lo);
    } else {
        fro_rowdot_f32(FRO_DT_F16, g->embed + J->lo * d, NULL, n, d, J->x, J->out + J->lo);
    }
    return NULL;
}

/* the final norm of the last row, then head_argmax (gemma.rs:386-390) */
static int gm_head(gm_run* R, const float* xlast, float* logits, int64_t* tok) {
    const fro_gemma_t* g = R->g;
    float* xf = (float*)malloc(nz(g->d * 4));
    fro_rmsnorm(xlast, 1, g->d, g->norm, g->eps, xf);
    int nt = R->nthreads < 1 ? 1 : (R->nthreads > 64 ? 64 : R->nthreads);
    pthread_t th[64];
    gm_head_job jobs[64];
    for (int w = 0; w < nt; w++) {
        jobs[w] = (gm_head_job){g, xf, logits, g->vocab * (size_t)w / nt, g->vocab * (size_t)(w + 1) / nt};
        pthread_create(&th[w], NULL, gm_head_worker, &jobs[w]);
    }
    for (int w = 0; w < nt; w++) pthread_join(th[w], NULL);
    free(xf);
    size_t best = 0;
    for (size_t r = 0; r < g->vocab; r++) {
        if (isnan(logits[r])) return FRO_ERR_NAN;
        if (logits[r] >= logits[best]) best = r;
    }
    *tok = (int64_t)best;
    return FRO_OK;
}

/* rows_f32 (src/bundle.rs:936-955): the row in f32 (a rowi8 element q as
 * f32 times its row's scale), then times the embedding scale */
static int gm_embed(const fro_gemma_t* g, const int64_t* ids, size_t m, float* x) {
    const float* f = (const float*)(const void*)g->embed;
    const int8_t* q = (const int8_t*)(const void*)g->embed;
    for (size_t t = 0; t < m; t++) {
        if (ids[t] < 0 || (size_t)ids[t] >= g->vocab) return FRO_ERR_ARG;
        const size_t r = (size_t)ids[t], b = r * g->d;
        for (size_t c = 0; c < g->d; c++) {
            float e;
            if (g->embed_dt == FRO_DT_F32) e = f[b + c];
            else if (g->embed_dt == FRO_DT_ROWI8) e = (float)q[b + c] * g->embed_scale[r];
            else e = fro_f16_to_f32(g->embed[b + c]);
            x[t * g->d + c] = e * g->escale;
        }
    }
    return FRO_OK;
}

int fro_gemma_generate(const fro_gemma_t* g, const int64_t* prompt, size_t n_prompt, size_t n_new, int kv_int8,
                       int nthreads, int64_t* out, float* logits) {
    if (!n_prompt || !n_new) return FRO_ERR_ARG;
    const size_t d = g->d, L = g->n_layer, total = n_prompt + n_new, kvd = g->n_kv * g->hd;
    gm_run R;
    memset(&R, 0, sizeof R);
    R.g = g; R.nthreads = nthreads; R.kv8 = kv_int8;
    R.inv = (float*)malloc(nz(g->hd / 2 * 4));
    for (size_t j = 0; j < g->hd / 2; j++) R.inv[j] = 1.0f / powf(g->theta, 2.0f * (float)j / (float)g->hd);
    R.kc = (float**)calloc(L, sizeof(float*)); R.vc = (float**)calloc(L, sizeof(float*));
    R.kq = (int8_t**)calloc(L, sizeof(int8_t*)); R.vq = (int8_t**)calloc(L, sizeof(int8_t*));
    R.ks = (float**)calloc(L, sizeof(float*)); R.vs = (float**)calloc(L, sizeof(float*));
    for (size_t l = 0; l < L; l++) {
        if (!kv_int8) {
            R.kc[l] = (float*)calloc(total * kvd, 4); R.vc[l] = (float*)calloc(total * kvd, 4);
        } else {
            R.kq[l] = (int8_t*)calloc(total * kvd, 1); R.vq[l] = (int8_t*)calloc(total * kvd, 1);
            R.ks[l] = (float*)calloc(total * g->n_kv, 4); R.vs[l] = (float*)calloc(total * g->n_kv, 4);
        }
    }
    float* x = (float*)malloc(nz(n_prompt * d * 4));
    float* lg = (float*)malloc(nz(g->vocab * 4));
    int64_t next = 0;
    int rc = gm_embed(g, prompt, n_prompt, x);
    if (!rc) rc = gm_block(&R, x, n_prompt, 0);
    if (!rc) rc = gm_head(&R, x + (n_prompt - 1) * d, lg, &next);
    size_t pos = n_prompt;
    for (size_t s = 0; !rc; s++) {
        out[s] = next;
        if (logits) memcpy(logits + s * g->vocab, lg, g->vocab * 4);
        if (s + 1 == n_new) break;
        rc = gm_embed(g, &next, 1, x);
        if (!rc) rc = gm_block(&R, x, 1, pos);
        if (!rc) rc = gm_head(&R, x, lg, &next);
        pos++;
    }
    for (size_t l = 0; l < L; l++) {
        free(R.kc[l]); free(R.vc[l]); free(R.kq[l]); free(R.vq[l]); free(R.ks[l]); free(R.vs[l]);
    }
    free(R.kc); free(R.vc); free(R.kq); free(R.vq); free(R.ks); free(R.vs); free(R.inv);
    free(x); free(lg);
    return rc;
}
