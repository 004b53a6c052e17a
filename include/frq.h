/*
 * frq.h — C ABI of the MI355X (gfx950) quantised-linear library (libfrq.so).
 *
 * This is the drop-in boundary for fieldrun's quantised-linear hot path.  A
 * host (the reference's Rust Bundle through a thin FFI crate, or Python
 * ctypes as in fieldrun_amd/__init__.py) uploads each weight once into HBM
 * and then calls the linear / expert entry points with plain pointers and
 * sizes.  No torch or HIP types appear in the signatures: streams and device
 * buffers are passed as void* / typed device pointers.
 *
 * Citations are to the reference crate (/root/reference, fieldrun 0.1.0).
 *
 * Conventions
 *  - Every entry point returns an int status (FRQ_OK = 0) or a NULL handle;
 *    frq_last_error() then returns a one-line message (thread-local).  The
 *    reference panics in the same situations (src/bundle.rs:370, 378-380,
 *    703, 737, 917); nothing unwinds across this ABI.
 *  - A frq_ctx owns one HIP stream and a workspace on one device.  Calls on
 *    one ctx must not overlap (one ctx per host thread, as the reference's
 *    Bundle is shared `&self` across rayon workers, src/model.rs:258).
 *    Weight handles (frq_w, frq_moe_w) are immutable after upload and may be
 *    used from any ctx on the same device.
 *  - "Host" entry points take host pointers, copy in, compute and copy out,
 *    and return after the result is on the host.  "_dev" entry points take
 *    device pointers, enqueue on the ctx stream and return immediately;
 *    their data-dependent errors (NaN activations) are reported by the next
 *    frq_sync().
 */
#ifndef FRQ_H
#define FRQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    FRQ_OK = 0,
    FRQ_ERR_ARG = 1,     /* bad argument / shape mismatch                  */
    FRQ_ERR_HIP = 2,     /* HIP runtime error (allocation, launch, copy)   */
    FRQ_ERR_NAN = 3,     /* NaN activation: bundle.rs:703/737 unwrap panic */
    FRQ_ERR_DTYPE = 4,   /* weight dtype not valid for this call (:370,917) */
    FRQ_ERR_FORMAT = 5,  /* bad bundle manifest (bundle.rs:316-321)        */
    FRQ_ERR_MISSING = 6, /* missing array (bundle.rs:378-380)              */
    FRQ_ERR_NODEV = 7    /* no HIP device / library built without GPU      */
};

enum {
    FRQ_DT_I8 = 1,    /* int8 linear weight (W8A8)                        */
    FRQ_DT_I4 = 2,    /* group-wise int4 linear weight (W4A32)            */
    FRQ_DT_F32 = 3,   /* row-major f32 rows (embed / unembed)             */
    FRQ_DT_F16 = 4,   /* row-major f16 rows                               */
    FRQ_DT_ROWI8 = 5, /* row-major int8 rows + f32 scale per row          */
    FRQ_DT_Q4A = 6    /* group-wise affine int4 linear (W4A32, scale+min) */
};
enum { FRQ_ACT_SILU = 0, FRQ_ACT_GELU_TANH = 1 };

typedef struct frq_ctx frq_ctx;
typedef struct frq_w frq_w;
typedef struct frq_moe_w frq_moe_w;
typedef struct frq_bundle frq_bundle;
typedef struct frq_gpt2 frq_gpt2;
typedef struct frq_gemma frq_gemma;

/* Last error message of the calling thread ("" when none). */
const char* frq_last_error(void);
/* Library version string. */
const char* frq_version(void);
/* Number of visible HIP devices (0 when none). */
int frq_device_count(void);

/* Context: device selection plus a stream and workspace.  Stands in for the
 * `--device gpu` arm of device::select (src/device.rs:40-87). */
frq_ctx* frq_init(int device);
void frq_free(frq_ctx* ctx);
/* Enqueue on a caller stream (e.g. torch.cuda.current_stream().cuda_stream)
 * instead of the ctx's own; NULL restores the ctx stream. */
int frq_set_stream(frq_ctx* ctx, void* hip_stream);
void* frq_get_stream(frq_ctx* ctx);
/* Wait for the ctx stream; returns FRQ_ERR_NAN if a _dev call since the last
 * sync saw a NaN activation, else FRQ_OK / FRQ_ERR_HIP. */
int frq_sync(frq_ctx* ctx);

/* ---- weight upload (one-time, into persistent HBM) ---------------------- */

/* int8 weight from the loader's transposed store: wt (N,K) row-major
 * (wt[j*K+kk] = W[kk,j]) and f32 per-output scale[N].  Replaces
 * Bundle::i8_for_gpu (src/bundle.rs:521-526) as the upload hook. */
frq_w* frq_upload_i8(frq_ctx* ctx, const int8_t* wt_nk, const float* scale,
                     size_t n, size_t k);
/* int8 weight straight from the bundle blob: w (in=K, out=N) row-major as
 * written by put_i8 (src/convert.rs:344-360) and its f16 `__scale` [N].  The
 * (K,N)->(N,K) transpose of Bundle::load (src/bundle.rs:345-355) and the
 * f16->f32 upcast of arr1o (921-933) run on the device. */
frq_w* frq_upload_i8_bundle(frq_ctx* ctx, const int8_t* w_kn,
                            const uint16_t* scale_f16, size_t k, size_t n);
/* Group-wise int4 weight as stored: packed (N, ceil(K/2)) bytes, even input
 * index in the low nibble, and f16 scales (N, ceil(K/g)) (src/bundle.rs:
 * 50-56, 356-360; src/convert.rs:189-216). */
frq_w* frq_upload_i4(frq_ctx* ctx, const uint8_t* packed,
                     const uint16_t* scale_f16, size_t n, size_t k, size_t g);
/* Group-wise affine int4 (q4a) weight as stored: packed (N, ceil(K/2))
 * unsigned nibbles (even input index low) and f16 scale and min, each
 * (N, ceil(K/g)); w = scale*q + min (src/bundle.rs:68-77, 361-364;
 * src/convert.rs:223-260).  frq_mm runs the Q4A arm of Bundle::mm
 * (802-845): M == 1 in q4a_dot_avx2's order, M > 1 dequantise + GEMM. */
frq_w* frq_upload_q4a(frq_ctx* ctx, const uint8_t* packed, const uint16_t* scale_f16,
                      const uint16_t* min_f16, size_t n, size_t k, size_t g);
/* Row-major (rows, d) embedding/unembedding table as stored: FRQ_DT_F32
 * (float data), FRQ_DT_F16 (uint16_t f16 bits) or FRQ_DT_ROWI8 (int8 data
 * plus scale[rows], the f32 upcast of the `__scale` sibling that
 * Bundle::rowdot_f32 reads with arr1o).  Replaces the F32 / F16 / RowI8
 * arrays of Bundle::load (src/bundle.rs:366-369) for rowdot_f32. */
frq_w* frq_upload_rows(frq_ctx* ctx, int dtype, const void* data,
                       const float* scale, size_t rows, size_t d);
void frq_w_free(frq_w* w);
/* dtype (FRQ_DT_*), N (out; rows), K (in; d), g (int4 group, else 0). */
int frq_w_info(const frq_w* w, int* dtype, size_t* n, size_t* k, size_t* g);

/* ---- the linear: Bundle::mm (src/bundle.rs:644-919) ----------------------
 * out (M,N) = a (M,K) @ W for an int8 weight (W8A8 with outlier-aware
 * per-token activation quant, src/bundle.rs:688-756) or an int4 weight
 * (W4A32, src/bundle.rs:760-799).  a and out are row-major f32. */
int frq_mm(frq_ctx* ctx, const frq_w* w, const float* a, size_t m,
           float* out);
int frq_mm_dev(frq_ctx* ctx, const frq_w* w, const float* d_a, size_t m,
               float* d_out);
/* Bundle::mm (src/bundle.rs:644-919) with every output in one fixed f32
 * order at any M (the order the CPU oracle restates, bit for bit), on device
 * pointers: int8 at M <= 16 as frq_mm_dev; at M > 16 the MFMA GEMM's exact
 * int32 sums, then the M > 1 arm's f32 outlier correction and epilogue
 * (732-756), the correction summed over the outliers in ascending channel
 * (the reference sums them in select_nth_unstable_by's permutation, which
 * its source does not fix); int4 in i4_dot_avx2's order at M = 1 and a.dot's
 * (matrixmultiply 0.3.10's blocked sgemm) at M > 1 (760-799); q4a likewise
 * (802-845).  frq_mm_dev's int8 results at M > 16 are within 1e-6
 * sum|terms| instead (the correction on the f16 MFMA).  The decode engines
 * run this linear. */
int frq_mm_exact_dev(frq_ctx* ctx, const frq_w* w, const float* d_a, size_t m,
                     float* d_out);
/* m independent rows, each Bundle::mm at M == 1 (src/bundle.rs:644-919):
 * row i of d_out is bit-identical to frq_mm_dev(ctx, w, d_a + i*K, 1, ...)
 * (int8: 688-756 at M == 1; int4: i4_dot_avx2's order, 767-776; q4a:
 * 802-845 at M == 1).  The reference reaches this when each of m sequences
 * runs its own decode step (Gemma::generate, src/gemma.rs:416, once per
 * sequence); the batched decode engine runs its linears through it. */
int frq_mm_rows_dev(frq_ctx* ctx, const frq_w* w, const float* d_a, size_t m,
                    float* d_out);
/* No counterpart in the reference.  frq_mm_dev that allocates nothing, for
 * callers that cannot call hipMalloc (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  The per-call scratch
 * (quantised rows, outliers, the GEMM pre-pass, int4 digit rows) lives in
 * one static device array of FRQ_NOALLOC_SCRATCH_BYTES per GPU, which the
 * library holds until the process ends; a call that needs more is refused
 * with FRQ_ERR_ARG (every int8 batch up to 16 rows fits, and larger batches
 * whose GEMM pre-pass and split-K tiles fit).  The array keeps the last
 * call's contents, and every call on one GPU shares it: calls that overlap
 * on one GPU (two streams, two contexts or two threads) race.  Results are
 * frq_mm_dev's. */
#define FRQ_NOALLOC_SCRATCH_BYTES (32u << 20)
int frq_mm_dev_noalloc(frq_ctx* ctx, const frq_w* w, const float* d_a, size_t m,
                       float* d_out);
/* int8 only, host pointers: also returns the internals the reference keeps
 * in locals — acc (M,N) i32 (the i8dot sums), a8 (M,K) i8, sa[M], and the
 * min(32,K) outliers per row (oidx, oval; (M,32), ascending channel).  Any
 * of the extra outputs may be NULL. */
int frq_mm_i8_debug(frq_ctx* ctx, const frq_w* w, const float* a, size_t m,
                    float* out, int32_t* acc, int8_t* a8, float* sa,
                    uint32_t* oidx, float* oval);

/* The int8 linear in its two reference steps, on device pointers (ctx
 * stream).  frq_quant_i8_dev is the activation quant of the I8 arm
 * (src/bundle.rs:699-708 == 732-743): a (M,K) f32 -> a8 (M, kp) i8 with row
 * pitch kp = frq_quant_pitch(K) (padding zero), sa[M], and the min(32,K)
 * outliers per row (oidx, oval; (M,32), ascending channel).
 * frq_mm_i8_q_dev is the dot + epilogue (709-715 / 744-752) on such a
 * quantised batch; frq_mm_dev == frq_quant_i8_dev + frq_mm_i8_q_dev. */
size_t frq_quant_pitch(size_t k);
int frq_quant_i8_dev(frq_ctx* ctx, const float* d_a, size_t m, size_t k,
                     int8_t* d_a8, float* d_sa, uint32_t* d_oidx,
                     float* d_oval);
int frq_mm_i8_q_dev(frq_ctx* ctx, const frq_w* w, const int8_t* d_a8,
                    const float* d_sa, const uint32_t* d_oidx,
                    const float* d_oval, size_t m, float* d_out);
/* The dot alone on such a quantised batch: acc (M,N) i32 = i8dot(a8[i],
 * wt[j]) for every row and column (src/bundle.rs:710 / 745, the exact sums
 * the epilogue scales), on device pointers.  M > 16 runs the MFMA GEMM whose
 * int32 sums frq_mm_exact_dev's epilogue takes (the engines' prefill GEMM);
 * M <= 16 the skinny / GEMV dot. */
int frq_mm_i8_acc_dev(frq_ctx* ctx, const frq_w* w, const int8_t* d_a8, size_t m,
                      int32_t* d_acc);

/* ---- the unembed: Bundle::rowdot_f32 (src/bundle.rs:958-987) -----------
 * out[r] = dot(W[r], x) for every row of a frq_upload_rows table (out has
 * rows entries, x has d), bit-identical to the reference's order (f32/f16:
 * a fold from -0.0; rowi8: scale * rowi8_dot_avx2, 158-178).  Other weight
 * dtypes are FRQ_ERR_DTYPE (the reference panics, 983). */
int frq_rowdot_f32(frq_ctx* ctx, const frq_w* w, const float* x, float* out);
int frq_rowdot_f32_dev(frq_ctx* ctx, const frq_w* w, const float* d_x,
                       float* d_out);
/* Bundle::rowdot_f32_subset (src/bundle.rs:995-1015): out[i] =
 * dot(W[cand[i]], x) for ncand candidate ids (rowi8: scale * the fold from
 * -0.0, 1011); an id < 0 or >= rows gives -inf. */
int frq_rowdot_f32_subset(frq_ctx* ctx, const frq_w* w, const float* x,
                          const int64_t* cand, size_t ncand, float* out);
int frq_rowdot_f32_subset_dev(frq_ctx* ctx, const frq_w* w, const float* d_x,
                              const int64_t* d_cand, size_t ncand,
                              float* d_out);

/* ---- MoE experts: expert_f32 + expert_mm (src/bundle.rs:404-461) and the
 * routed branch of src/qwen3moe.rs:120-158 / src/gemma4.rs:131-187 -------- */

/* Upload all experts of one layer.  act FRQ_ACT_SILU: gate[e], up[e] are
 * (in=d, out=mi) and down[e] (in=mi, out=d), i8 (in,out) row-major as the
 * bundle stores them, scales f32 [out].  act FRQ_ACT_GELU_TANH: gate[e] is
 * the packed gate_up (d, 2*mi) and up/up_scale are ignored. */
frq_moe_w* frq_moe_upload_i8(frq_ctx* ctx, size_t n_exp, size_t d, size_t mi,
                             int act, const int8_t* const* gate,
                             const float* const* gate_scale,
                             const int8_t* const* up,
                             const float* const* up_scale,
                             const int8_t* const* down,
                             const float* const* down_scale);
/* The expert bank of one layer in the dtype its bundle stores (the arms of
 * expert_f32, src/bundle.rs:404-454; written by put_lin,
 * src/convert.rs:174-260): dtype FRQ_DT_I8 (gate[e] etc. int8 (in, out),
 * *_scale f16 [out]), FRQ_DT_I4 (packed (out, ceil(in/2)) nibbles, even
 * input index low, *_scale f16 (out, ceil(in/g))), FRQ_DT_Q4A (as i4 with
 * unsigned nibbles and *_min f16 (out, ceil(in/g))), FRQ_DT_F16 (f16 bits,
 * (in, out)) or FRQ_DT_F32 ((in, out)); *_min only for q4a, g only for
 * i4 / q4a (the loader's defaults are 32 and 64).  Shapes and act as
 * frq_moe_upload_i8 (gate = the packed gate_up for FRQ_ACT_GELU_TANH).  The
 * weights stay in their stored precision in HBM and are dequantised in
 * registers, each value as expert_f32 forms it; i4 banks with g % 32 == 0
 * also keep an MFMA operand copy of the nibbles.  FRQ_ERR_DTYPE for another
 * dtype (the reference panics, :452). */
frq_moe_w* frq_moe_upload(frq_ctx* ctx, int dtype, size_t n_exp, size_t d, size_t mi, int act, size_t g,
                          const void* const* gate, const uint16_t* const* gate_scale,
                          const uint16_t* const* gate_min, const void* const* up,
                          const uint16_t* const* up_scale, const uint16_t* const* up_min,
                          const void* const* down, const uint16_t* const* down_scale,
                          const uint16_t* const* down_min);
void frq_moe_free(frq_moe_w* m);
/* dtype (FRQ_DT_*), n_exp, d, mi and the int4 group (0 for other dtypes). */
int frq_moe_info(const frq_moe_w* m, int* dtype, size_t* n_exp, size_t* d, size_t* mi, size_t* g);

/* Routed expert layer: softmax over the router logits (T,E), stable top-k,
 * renormalise (norm_topk; per_expert_scale non-NULL selects the gemma4
 * weighting p/sum*pes[e]), per-expert W8A32 matmuls with SwiGLU or
 * gelu_tanh gating, weighted combine into out (T,d).  x, logits, out f32.
 * topk in [1, min(n_exp, 256)] (FRQ_ERR_ARG otherwise); a NaN logit, or a
 * row whose max is +-inf, is FRQ_ERR_NAN (the reference's sort panics). */
int frq_moe(frq_ctx* ctx, const frq_moe_w* m, const float* x, size_t T,
            const float* logits, size_t topk, int norm_topk,
            const float* per_expert_scale, float* out);
int frq_moe_dev(frq_ctx* ctx, const frq_moe_w* m, const float* d_x, size_t T,
                const float* d_logits, size_t topk, int norm_topk,
                const float* d_per_expert_scale, float* d_out);
/* Routing only (host pointers): sel (T,topk) expert ids in descending-p
 * order, w (T,topk) combine weights. */
int frq_moe_route(frq_ctx* ctx, const float* logits, size_t T, size_t E,
                  size_t topk, int norm_topk, const float* per_expert_scale,
                  int32_t* sel, float* w);
/* One expert matmul, expert_mm (src/bundle.rs:457-461): y (M,out) =
 * x (M,in) @ expert_f32 for expert `e` of bank `which` (0 gate/gate_up,
 * 1 up, 2 down), any bank dtype, in a.dot's order (matrixmultiply 0.3.10's
 * sgemm: 256-long k blocks, each an FMA chain from +0, added in order). */
int frq_expert_mm(frq_ctx* ctx, const frq_moe_w* m, int which, size_t e,
                  const float* x, size_t mrows, float* y);

/* ---- the bundle: Bundle::load (src/bundle.rs:314-376, FORMAT.md) --------
 * frq_bundle_open reads <stem>.fieldrun.json and maps <stem>.fieldrun.bin
 * read-only (host only, no device): FRQ_ERR_FORMAT for a manifest the
 * reference refuses (format != "fieldrun-bundle", version != 1, an array
 * beyond the blob), FRQ_ERR_ARG for I/O errors; *out is the bundle or NULL. */
int frq_bundle_open(const char* stem, frq_bundle** out);
void frq_bundle_close(frq_bundle* b);
/* arch (NUL-terminated, truncated to arch_cap), config / config_f: up to
 * *n entries copied, *n set to the manifest's count. */
int frq_bundle_header(const frq_bundle* b, char* arch, size_t arch_cap,
                      int64_t* config, size_t* n_config, double* config_f,
                      size_t* n_config_f);
/* One array as stored (expert arrays included): dtype string, shape (up
 * to *ndim dims copied, *ndim set), int4 group (0 when absent), a pointer
 * into the mapped blob (valid until frq_bundle_close) and its byte count.
 * FRQ_ERR_MISSING when absent (src/bundle.rs:378-380). */
int frq_bundle_array(const frq_bundle* b, const char* name, char* dtype,
                     size_t dtype_cap, size_t* shape, size_t* ndim,
                     size_t* group, const void** data, size_t* bytes);
/* Upload one array onto ctx's device in its stored precision: an i8 linear
 * (with its f16 __scale, as frq_upload_i8_bundle), an i4 linear (with its
 * f16 (out, ceil(in/g)) __scale and group, default 32), a rowi8 table (f16
 * row scales) or a 2-D f16 / f32 table (as frq_upload_rows).  The caller
 * owns *out (frq_w_free).  FRQ_ERR_MISSING for an absent array or scale,
 * FRQ_ERR_FORMAT when a size does not match its shape, FRQ_ERR_DTYPE for a
 * dtype with no device form here. */
int frq_bundle_weight(frq_ctx* ctx, const frq_bundle* b, const char* name,
                      frq_w** out);
/* The routed expert bank of one MoE layer: n_exp experts named
 * {prefix}experts.{e}.gate / .up / .down (FRQ_ACT_SILU, qwen3moe) or
 * .gate_up / .down (FRQ_ACT_GELU_TANH, gemma4) (src/qwen3moe.rs:148-152,
 * src/gemma4.rs:174-181), in any dtype expert_f32 reads (i8 / i4 / q4a
 * with their f16 __scale (and __min) siblings, f16, f32; the first
 * expert's dtype, every expert alike), uploaded as frq_moe_upload. */
int frq_bundle_moe(frq_ctx* ctx, const frq_bundle* b, const char* prefix,
                   size_t n_exp, int act, frq_moe_w** out);

/* ---- GPT-2 decode: Gpt2 (src/composition.rs) on the device --------------
 * frq_gpt2_load is Gpt2::new (52-56) over an arch "gpt2" bundle (config
 * [n_layer, n_head, n_embd, n_positions, vocab]; arrays as convert_gpt2
 * writes them, src/convert.rs:505-545): the int8 / int4 linears, the f16
 * wte table (embedding rows and the tied unembed), wpe, the layernorms and
 * biases go to ctx's device with a KV cache of n_positions rows per layer
 * (kv_int8: int8 with an f32 scale per position and head, as
 * forward_block_q, 214-249).  FRQ_ERR_FORMAT / FRQ_ERR_MISSING /
 * FRQ_ERR_DTYPE for a bundle that does not match. */
int frq_gpt2_load(frq_ctx* ctx, const frq_bundle* b, int kv_int8, frq_gpt2** out);
void frq_gpt2_free(frq_gpt2* g);
int frq_gpt2_info(const frq_gpt2* g, size_t* n_layer, size_t* n_head, size_t* d, size_t* n_pos,
                  size_t* vocab);
/* Model::generate for Gpt2 (317-341 / 251-270): n_new greedy tokens after
 * the prompt (prefill, then one cached decode step per token) into out;
 * logits (n_new, vocab), nullable, receives the logits each token was
 * chosen from.  FRQ_ERR_ARG for an id outside the vocabulary or a position
 * past n_positions (the reference panics on those rows), FRQ_ERR_NAN for
 * NaN activations or logits.  Calls on one model must not overlap. */
int frq_gpt2_generate(frq_ctx* ctx, frq_gpt2* g, const int64_t* prompt, size_t n_prompt, size_t n_new,
                      int64_t* out, float* logits);
/* Model::predict (304-308): the next token after ids (logits nullable). */
int frq_gpt2_predict(frq_ctx* ctx, frq_gpt2* g, const int64_t* ids, size_t n, int64_t* token,
                     float* logits);
/* Decode steps run as one captured HIP graph per generate call (replayed
 * per token) unless switched off here; the results are the same. */
int frq_gpt2_set_graphs(frq_gpt2* g, int on);
/* ---- Gemma-2 decode: Gemma (src/gemma.rs) on the device -----------------
 * frq_gemma_load is Gemma::new (52-60) over an arch "gemma" bundle (config
 * [n_layer, H, nkv, hd, d, ffn, vocab, tied], config_f [theta, eps,
 * attn_cap, final_cap, query_pre_attn_scalar, escale]; arrays as
 * convert_gemma writes them, src/convert.rs:636-657): int4 / int8 / q4a
 * linears (q|k|v and gate|up uploaded side by side), the embed (rows and
 * the tied unembed) as an f32, f16 or rowi8 table (Bundle::rows_f32 /
 * rowdot_f32, src/bundle.rs:936-987), the RMSNorm gains; kv_int8: the int8 cache of
 * forward_block_q (293-363).  generate / predict as Model::generate
 * (403-431) / predict (436-441): tokens and logits as the reference's.
 * The cache and the RoPE table grow to the longest call. */
int frq_gemma_load(frq_ctx* ctx, const frq_bundle* b, int kv_int8, frq_gemma** out);
void frq_gemma_free(frq_gemma* g);
int frq_gemma_info(const frq_gemma* g, size_t* n_layer, size_t* d, size_t* vocab);
int frq_gemma_generate(frq_ctx* ctx, frq_gemma* g, const int64_t* prompt, size_t n_prompt, size_t n_new,
                       int64_t* out, float* logits);
int frq_gemma_predict(frq_ctx* ctx, frq_gemma* g, const int64_t* ids, size_t n, int64_t* token,
                      float* logits);
int frq_gemma_set_graphs(frq_gemma* g, int on);
/* nb sequences at once (configs[2]'s batch 16): prompts (nb, n_prompt),
 * each sequence its own Model::generate (src/gemma.rs:403-431; the reference
 * has no batched generate, a batch is nb independent calls): out (nb, n_new)
 * and logits (nb, n_new, vocab), nullable, are what nb calls of
 * frq_gemma_generate give, bit for bit.  Each sequence has its own KV cache;
 * the decode steps of all nb run together (the weights stream once a step,
 * every row of an int4 linear in the M == 1 order of i4_dot_avx2). */
int frq_gemma_generate_batch(frq_ctx* ctx, frq_gemma* g, const int64_t* prompts, size_t nb, size_t n_prompt,
                             size_t n_new, int64_t* out, float* logits);
/* Rope::new (src/rope.rs:56-64) over an arch "rope" bundle (Llama / Qwen2.5
 * / Qwen3 / Mistral: config [n_layer, H, nkv, hd, d, ffn, vocab, tied],
 * config_f [theta, eps]; arrays as convert_rope writes them,
 * src/convert.rs:619-634: in_ln / post_ln, optional q/k/v biases and q/k
 * norms, lm_head unless tied) into the same engine: generate, predict,
 * free and set_graphs are the frq_gemma_* calls (Model::generate,
 * rope.rs:1147-1170; predict 730-734). */
int frq_rope_load(frq_ctx* ctx, const frq_bundle* b, int kv_int8, frq_gemma** out);
/* The f32 libm functions the decode kernels use (fn 0 expf, 1 expm1f, 2
 * tanhf, 3 expf in the branch-free form the attention kernels use),
 * bit-identical to the libm behind Rust's f32::exp / f32::tanh
 * (glibc's expf and fdlibm's expm1f / tanhf): out[i] = f(x[i]) for n host
 * values, on ctx's device, or on the host when ctx is NULL. */
int frq_libm_f32(frq_ctx* ctx, int fn, const float* x, size_t n, float* out);
/* Checking hook of the decode kernels' sequential fold (RMSNorm mean
 * squares, softmax sums; the Rust iterator sum, a fold in index order):
 * out[r] = init + x[r][0] + ... + x[r][n-1] in f32, computed on ctx's
 * device by the speculative segmented fold the kernels use.  x is (rows, n)
 * row-major on the host. */
int frq_seq_fold_f32(frq_ctx* ctx, const float* x, size_t rows, size_t n, float init, float* out);

#ifdef __cplusplus
}
#endif
#endif
