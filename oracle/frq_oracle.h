/*
 * frq_oracle.h — CPU restatement of fieldrun's quantised-linear hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * kernels in fieldrun_amd/csrc and the CPU baseline timed by bench.py. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product library (libfrq.so) never links, loads or calls it.
 *
 * Every function restates one piece of /root/reference (Rust crate fieldrun
 * 0.1.0); the file:line each follows is cited at its definition in
 * frq_oracle.c.  Where the reference's own order is unspecified (the
 * permutation left by select_nth_unstable_by, HashMap iteration order,
 * matrixmultiply's internal k-blocking) the oracle fixes one deterministic
 * order and says so; the GPU kernels are checked against that order.
 *
 * Pinning status of each function (what checks it beyond this restatement):
 *   fro_f16_to_f32 / fro_f32_to_f16   exhaustive vs numpy float16 (IEEE)
 *   fro_put_i8 / fro_put_i4           reference KAT int8_quant_roundtrip +
 *                                     closed-form numpy quantiser
 *   fro_i8dot                         reference KATs i8dot_matches_manual,
 *                                     i8dot_simd_vs_scalar (xorshift vectors)
 *                                     + int64 brute force
 *   fro_quant_row / fro_mm_i8         closed-form invariants + brute-force
 *                                     sort + f64 epilogue bound
 *   fro_i4_dot / fro_i4_dot_avx2      reference KATs i4_q4a_dot_matches_manual
 *                                     (=1.0), i4_q4a_dot_simd_vs_reference,
 *                                     jit LCG vectors + f64 brute force
 *   fro_q4a_dot / _avx2 / fro_mm_q4a  reference KATs i4_q4a_dot_matches_manual
 *                                     (=12.5) and i4_q4a_dot_simd_vs_reference,
 *                                     f64 brute force, exact small-integer
 *                                     cases, hand-derived lane-order case;
 *                                     fro_put_q4a by closed forms (min/max
 *                                     nibbles, reconstruction bound)
 *   fro_mm_dot / fro_sgemm            a hand-derived case that separates the
 *                                     256-long blocks from one chain and from
 *                                     other block lengths, exact integers;
 *                                     that it is matrixmultiply 0.3.10's order
 *                                     (restated from that crate's published
 *                                     gemm loop) no reference test pins
 *   fro_mm_i4 (M>1), fro_expert_mm    f64 brute force and exact integers; the
 *                                     reference has no test for these
 *   fro_expert_f32                    closed forms per arm (i4 nibble order and
 *                                     group index, q4a mul then add, f16, f32,
 *                                     i8); fro_moe_ex_mt over f32 experts holding
 *                                     an int8 bank's q * s is that bank's layer
 *                                     bit for bit
 *   fro_moe_route / fro_moe           closed-form softmax + brute-force
 *                                     stable sort, f64 combine bound
 *   fro_nd_sum / fro_layernorm        hand-derived order case (the eight-lane
 *                                     fold vs a sequential sum), exact-integer
 *                                     rows vs f64, constant rows
 *   fro_gpt2_generate / _predict      an independent f64 numpy forward (tolerance),
 *                                     predict(prefix) == the cached decode step
 *                                     bit for bit (composition.rs:313-316 says the
 *                                     cache is exact); matrixmultiply's order for
 *                                     the attention products is parity unpinned
 *   fro_rowdot_f32 / _subset          exact small-integer dots (any order),
 *                                     f64 bound, and order-revealing cases
 *                                     whose f32 result follows by hand from
 *                                     the fold / the eight-lane AVX2 order;
 *                                     the reference has no test for these
 */
#ifndef FRQ_ORACLE_H
#define FRQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FRO_OUTLIER_T 32

#define FRO_OK 0
#define FRO_ERR_ARG 1 /* an index the reference would panic on          */
#define FRO_ERR_NAN 3 /* reference panics in partial_cmp().unwrap() */
#define FRO_DT_I8 1  /* expert / linear weight types (bundle.rs Arr) */
#define FRO_DT_I4 2
#define FRO_DT_Q4A 6
#define FRO_DT_F32 3 /* the row-dot table types (bundle.rs Arr) */
#define FRO_DT_F16 4
#define FRO_DT_ROWI8 5

/* IEEE binary16 <-> binary32 (half 2.7.1 semantics: RNE, exact upcast). */
float fro_f16_to_f32(uint16_t h);
uint16_t fro_f32_to_f16(float f);
void fro_f16_to_f32_n(const uint16_t* src, float* dst, size_t n);

/* BundleWriter quantisers. transpose=1: source is (out,in) nn.Linear. */
void fro_put_i8(const float* data, size_t rows, size_t cols, int transpose,
                int8_t* w_in_out, uint16_t* scale_f16);
size_t fro_put_i4(const float* data, size_t rows, size_t cols, int transpose,
                  uint8_t* packed, uint16_t* scale_f16);
void fro_put_embed_i8(const float* data, size_t vocab, size_t d, int8_t* q,
                      uint16_t* scale_f16);

/* Bundle::load's i8 arm: (in=K, out=N) row-major -> (N,K). */
void fro_i8_transpose(const int8_t* w_kn, size_t k, size_t n, int8_t* wt_nk);

/* i8dot: scalar i8 x i8 -> i32. */
int32_t fro_i8dot(const int8_t* a, const int8_t* w, size_t n);
/* i8dot_avx512bw (src/bundle.rs:1107-1126); needs a host with AVX-512BW. */
int32_t fro_i8dot_avx512bw(const int8_t* a, const int8_t* w, size_t n);
/* The dot of the int8 linears: 0 the scalar fallback (default), 1
 * i8dot_avx512bw.  Returns 0 (and changes nothing) when the host lacks
 * AVX-512BW.  Integer results are the same either way; only speed differs. */
int fro_set_i8dot(int variant);

/* Outlier-aware activation quant of ONE row.  Writes a8[k], *sa, the t
 * outliers (oidx, oval) in ascending channel order and *t = min(32,k).
 * Returns FRO_ERR_NAN when the reference would panic. */
int fro_quant_row(const float* a, size_t k, int8_t* a8, float* sa,
                  uint32_t* oidx, float* oval, size_t* t);

/* Bundle::mm I8 arm.  wt is (N,K), scale f32 [N].  acc (M,N) nullable. */
int fro_mm_i8(const float* a, size_t m, size_t k, const int8_t* wt,
              const float* scale, size_t n, float* out, int32_t* acc);
/* Same with the reference's rayon split over nthreads worker threads. */
int fro_mm_i8_mt(const float* a, size_t m, size_t k, const int8_t* wt,
                 const float* scale, size_t n, float* out, int nthreads);

/* i4_dot (scalar fold) and i4_dot_avx2 (the x86 production order). */
float fro_i4_dot(const uint8_t* prow, const float* a, const float* scale,
                 size_t g, size_t k);
float fro_i4_dot_avx2(const uint8_t* prow, const float* a, const float* scale,
                      size_t g, size_t k);
/* Bundle::mm I4 arm: M==1 uses the AVX2 order, M>1 dequant + f32 GEMM.
 * packed (N, ceil(K/2)), scale f32 (N, ceil(K/g)). */
int fro_mm_i4(const float* a, size_t m, size_t k, const uint8_t* packed,
              const float* scale, size_t n, size_t g, float* out);

/* Affine int4 (q4a): packed (N, ceil(K/2)) unsigned nibbles, scale and min
 * (N, ceil(K/g)).  put_q4a returns g (min(32, in)). */
size_t fro_put_q4a(const float* data, size_t rows, size_t cols, int transpose, uint8_t* packed,
                   uint16_t* scale_f16, uint16_t* min_f16);
float fro_q4a_dot(const uint8_t* prow, const float* a, const float* scale, const float* mins, size_t g, size_t k);
float fro_q4a_dot_avx2(const uint8_t* prow, const float* a, const float* scale, const float* mins, size_t g,
                       size_t k);
int fro_mm_q4a(const float* a, size_t m, size_t k, const uint8_t* packed, const float* scale, const float* mins,
               size_t n, size_t g, float* out);

/* expert_f32 (i8 arm) + expert_mm: raw (in,out) i8, scale f32 [out]. */
void fro_expert_mm_i8(const float* x, size_t m, const int8_t* raw,
                      const float* scale, size_t inp, size_t out, float* y);
/* One MoE expert weight as the bundle stores it (src/bundle.rs:288-294,
 * 404-454): dtype FRO_DT_I8 (raw (in,out) i8, scale [out]), FRO_DT_I4
 * (raw (out, ceil(in/2)) packed nibbles, even input index low, scale
 * (out, ceil(in/g))), FRO_DT_Q4A (as i4 with unsigned nibbles and mins
 * (out, ceil(in/g))), FRO_DT_F16 (raw (in,out) f16 bits) or FRO_DT_F32
 * (raw (in,out) f32).  Scales and mins are the f32 upcasts of the f16
 * __scale / __min siblings (arr1o). */
typedef struct {
    int dtype;
    const void* raw;
    const float* scale;
    const float* mins;
    size_t g;
} fro_expert_t;
/* expert_f32: the weight dequantised to f32 (in, out) row-major (v has
 * inp*out entries).  FRO_ERR_ARG for an unknown dtype (the reference
 * panics, :452). */
int fro_expert_f32(const fro_expert_t* e, size_t inp, size_t out, float* v);
/* expert_mm (src/bundle.rs:457-461): y (m,out) = x (m,inp) . expert_f32. */
int fro_expert_mm(const fro_expert_t* e, const float* x, size_t m, size_t inp, size_t out, float* y);
/* One element of a.dot (matrixmultiply 0.3.10 sgemm): k split into blocks
 * of FRO_MM_KC in order, each an FMA chain from +0, the block results added
 * in order (the first stored as is). */
#define FRO_MM_KC 256
float fro_mm_dot(const float* x, size_t xs, const float* w, size_t ws, size_t k);
/* f32 GEMM y(m,n) = x(m,k) . w(k,n), each element fro_mm_dot. */
void fro_sgemm(const float* x, size_t m, size_t k, const float* w, size_t n,
               float* y);

/* Nonlinearities used by the MoE branch. */
float fro_silu(float x);
float fro_gelu_tanh(float x);

/* qwen3moe softmax_rows + stable top-k + renorm; gemma4 variant multiplies
 * by per_expert_scale (nullable).  sel (T,topk) int32, w (T,topk) f32.
 * probs (T,E) nullable: the softmax output. */
void fro_moe_route(const float* logits, size_t T, size_t E, size_t topk,
                   int norm_topk, const float* per_expert_scale, int32_t* sel,
                   float* w, float* probs);

/* Full routed expert layer (qwen3moe moe_branch minus the router mm).
 * act 0: SwiGLU with separate gate/up (qwen3moe); act 1: gelu_tanh with a
 * packed gate_up expert (gemma4).  Expert e's arrays: gate[e]/up[e] (in=d,
 * out=mi) or gate[e] = gate_up (d, 2mi); down[e] (mi, d); i8 (in,out) with
 * f32 scales.  Experts are combined in ascending expert order. */
int fro_moe(const float* x, size_t T, size_t d, const float* logits, size_t E,
            size_t topk, int norm_topk, const float* per_expert_scale,
            size_t mi, int act, const int8_t* const* gate,
            const float* const* gate_scale, const int8_t* const* up,
            const float* const* up_scale, const int8_t* const* down,
            const float* const* down_scale, float* out);
int fro_moe_mt(const float* x, size_t T, size_t d, const float* logits, size_t E,
            size_t topk, int norm_topk, const float* per_expert_scale,
            size_t mi, int act, const int8_t* const* gate,
            const float* const* gate_scale, const int8_t* const* up,
            const float* const* up_scale, const int8_t* const* down,
            const float* const* down_scale, float* out, int nthreads);
/* The same layer over experts of any stored dtype (fro_expert_t, arrays of
 * E each; up is ignored for act 1), on nthreads threads. */
int fro_moe_ex_mt(const float* x, size_t T, size_t d, const float* logits, size_t E,
                  size_t topk, int norm_topk, const float* per_expert_scale,
                  size_t mi, int act, const fro_expert_t* gate, const fro_expert_t* up,
                  const fro_expert_t* down, float* out, int nthreads);

/* Bundle::rowdot_f32 / rowdot_f32_subset over a row-major (rows, d) table:
 * dtype 3 f32 (float data), 4 f16 (uint16 bits), 5 rowi8 (int8 data +
 * scale[rows]). Subset ids < 0 or >= rows give -inf. */
void fro_rowdot_f32(int dtype, const void* data, const float* scale, size_t rows,
                    size_t d, const float* x, float* out);
void fro_rowdot_f32_subset(int dtype, const void* data, const float* scale,
                           size_t rows, size_t d, const float* x,
                           const int64_t* cand, size_t ncand, float* out);

/* GPT-2 with a KV cache (src/composition.rs).  Weights as the bundle holds
 * them after Bundle::load: wte f16 bits (vocab, d), wpe f32 (n_pos, d); per
 * layer l: ln_g/ln_b[2l] = ln_1, [2l+1] = ln_2 (f32 [d]); wt/scale/bias
 * [4l + 0..3] = attn.c_attn, attn.c_proj, mlp.c_fc, mlp.c_proj with wt the
 * (N, K) transposed int8 store, scale and bias f32 [N]. */
typedef struct {
    size_t n_layer, n_head, d, n_pos, vocab;
    const uint16_t* wte;
    const float* wpe;
    const float* ln_f_g;
    const float* ln_f_b;
    const float* const* ln_g;
    const float* const* ln_b;
    const int8_t* const* wt;
    const float* const* scale;
    const float* const* bias;
} fro_gpt2_t;

/* The system libm's expf (fn 0), expm1f (1), tanhf (2) over n values. */
void fro_libm_f32(int fn, const float* x, size_t n, float* out);
/* ndarray 0.16.1 ArrayBase::sum of a contiguous f32 row (unrolled_fold). */
float fro_nd_sum(const float* x, size_t n);
/* layernorm (composition.rs:20-33) over m rows of d. */
void fro_layernorm(const float* x, size_t m, size_t d, const float* g, const float* b, float* out);
/* Gpt2::generate (composition.rs:317-341; kv_int8: 251-270): n_new greedy
 * tokens after the prompt; logits (n_new, vocab) nullable: the logits each
 * token was chosen from.  FRO_ERR_ARG for a token / position beyond the
 * tables (the reference's index panic), FRO_ERR_NAN for NaN activations or
 * logits. */
int fro_gpt2_generate(const fro_gpt2_t* g, const int64_t* prompt, size_t n_prompt, size_t n_new, int kv_int8,
                      int nthreads, int64_t* out, float* logits);
/* Model::predict (composition.rs:304-308). */
int fro_gpt2_predict(const fro_gpt2_t* g, const int64_t* ids, size_t n, int nthreads, int64_t* tok, float* logits);

/* fro_mm_i4 over nthreads threads (columns split; identical results). */
int fro_mm_i4_mt(const float* a, size_t m, size_t k, const uint8_t* packed, const float* scale, size_t n, size_t g,
                 float* out, int nthreads);

/* A linear as Bundle::load keeps it: dtype 1 int8 (wt (N,K) transposed,
 * scale f32 [N]), 2 int4 (packed (N, ceil(K/2)), scale f32 (N, ng), g) or
 * 3 q4a (as int4 plus mins f32 (N, ng)). */
typedef struct {
    int dtype;
    size_t n, k, g;
    const uint8_t* packed;
    const int8_t* wt;
    const float* scale;
    const float* mins;
} fro_lin_t;

/* Gemma-2 (src/gemma.rs).  norms[4l + 0..3]: input, post_attention,
 * pre_feedforward, post_feedforward (f32, the +1 baked); lin[7l + 0..6]:
 * q, k, v, o, gate, up, down. qscale = query_pre_attn_scalar^-0.5. */
typedef struct {
    size_t n_layer, n_head, n_kv, hd, d, ffn, vocab, window;
    float theta, eps, attn_cap, qscale, escale;
    const uint16_t* embed;      /* (vocab, d) f16 bits: embedding and tied unembed */
    const float* norm;          /* final norm */
    const float* const* norms;
    const fro_lin_t* lin;
    /* the Llama / Qwen family (src/rope.rs) when arch == 1: no embedding
     * scale, norms[4l + 0] = in_ln and [4l + 2] = post_ln (1 and 3 NULL: a
     * plain residual), scores / sqrt(hd) (qscale unused), no soft-cap or
     * window, SiLU; bias[3l + 0..2] q / k / v biases (NULL when absent),
     * qk_norm[2l + 0..1] per-head q / k norms (NULL when absent); unembed
     * the lm_head (NULL: embed). */
    int arch;
    const float* const* bias;
    const float* const* qk_norm;
    const uint16_t* unembed;
    /* the embed table's type (Bundle::rows_f32 / rowdot_f32 take f32, f16
     * and rowi8, src/bundle.rs:936-987): FRO_DT_F32, FRO_DT_F16 (or 0) or
     * FRO_DT_ROWI8 with embed_scale its per-row f32 scales */
    int embed_dt;
    const float* embed_scale;
} fro_gemma_t;

/* RMSNorm with the baked (1 + w) gain (gemma.rs:66-77) over m rows. */
void fro_rmsnorm(const float* x, size_t m, size_t d, const float* w, float eps, float* out);
/* Gemma::generate (gemma.rs:403-431; kv_int8: 364-384) or, arch 1,
 * Rope::generate (src/rope.rs:1147-1170, forward_block 391-437): n_new
 * greedy tokens, logits (n_new, vocab) nullable. */
int fro_gemma_generate(const fro_gemma_t* g, const int64_t* prompt, size_t n_prompt, size_t n_new, int kv_int8,
                       int nthreads, int64_t* out, float* logits);

#ifdef __cplusplus
}
#endif
#endif
