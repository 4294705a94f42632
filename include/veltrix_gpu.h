/*
 * veltrix_gpu.h -- entry points this engine adds to the reference's API.
 *
 * The reference has no batched verify (src/speculative.c:186-207 runs one
 * single-token forward per draft) and no M-row GEMM; these are the additive
 * entry points for them, plus the AVX2-lane GEMV variants of
 * src/simd/simd.h:23-27 (declared there in the reference, internal header),
 * model options, synthetic models and seeded speculative sampling.
 */
#ifndef VELTRIX_GPU_H
#define VELTRIX_GPU_H

#include "veltrix.h"
#include "speculative.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- GEMV / GEMM ----------------------------------------------------------- */

/* AVX2-lane GEMV (reference src/simd/avx2.c:311-370, declared at
 * src/simd/simd.h:23): same arithmetic pattern as the x86 build, including
 * the read of x[cols..cols+3]. */
void vx_gemv_q4_0_avx2(const void *A, const float *x, float *y, int rows, int cols);
/* (reference src/simd/avx2.c:224-279, src/simd/simd.h:25) */
void vx_gemv_q4_0_avx2_sparse_rows(const void *A, const float *x, float *y, int rows, int cols,
                                   const float *gate, float threshold);

/* Y[M][rows] = X[M][cols] . A^T, A in GGUF Q4_0 / Q8_0 blocks, host memory.
 * Equivalent to M calls of the reference's GEMV (vx_gemv_q4_0, or
 * vx_dequantize_row_q8_0 + vx_gemv_f32) but one pass over A on the GPU.
 * flags: VX_GEMM_AVX2_LANES selects the lane pattern for Q4_0 (X rows must
 * then have ldx >= cols + 4; the 4 floats after each row are read).  Returns
 * VX_OK or a negative vx_error. */
#define VX_GEMM_AVX2_LANES 1
vx_error vx_gemm_q4_0(const void *A, const float *X, int ldx, float *Y, int M, int rows, int cols,
                      int flags);
vx_error vx_gemm_q8_0(const void *A, const float *X, int ldx, float *Y, int M, int rows, int cols);

/* ---- model ---------------------------------------------------------------- */

#define VX_Q4_EXACT 0        /* d*(s-8)*x: the reference's portable build        */
#define VX_Q4_AVX2_LANES 1   /* the reference's x86 build (vx_gemv_q4_0_avx2)    */

typedef struct {
    int q4_kernel;             /* VX_Q4_EXACT (default) or VX_Q4_AVX2_LANES             */
    int attn_cap;              /* attend to at most the first attn_cap positions;
                                  4096 as the reference (src/model.c:304-305), 0 = none */
    float ffn_gate_threshold;  /* up rows with |silu(gate)| below it are zero; 0.01    */
    int fused;                 /* VX_FUSED_*: how the row work between GEMMs runs
                                  (AVX2-lane mode always uses separate kernels)       */
    int pro_max_rows;          /* VX_FUSED_PROLOGUE: forwards of more rows use the
                                  separate row kernels                                 */
    int kv_half;               /* 1: IEEE fp16 KV cache (flagged mode; the reference
                                  keeps fp32); needs VX_FUSED_PROLOGUE, VX_Q4_EXACT,
                                  pro_max_rows >= 16 and head_dim 64 or 128.  Changing
                                  it drops the cache (cache_len 0); k_cache/v_cache
                                  then hold halves                                    */
    int prefill_min_rows;      /* prompt chunks of at least this many rows whose
                                  positions fit the context run as one large-M
                                  batch (up to 512 rows; exact Q4_0 kernel, fp32
                                  cache); 0 = never.  Default 48               */
} vx_model_options;

#define VX_FUSED_NONE 0        /* separate row kernels (11 launches per layer)          */
#define VX_FUSED_PROLOGUE 2    /* in the consuming GEMM, which builds its own input
                                  panel slice; RMSNorm applied to the product (7).
                                  Value 1 (row work in the producing GEMM's last
                                  workgroups) was removed and is refused            */

void vx_model_get_options(const vx_model *model, vx_model_options *opt);
vx_error vx_model_set_options(vx_model *model, const vx_model_options *opt);

/* Batched verify: runs tokens[0..n) at positions cache_len.. like n calls of
 * vx_model_forward with one token each, but in batches of up to 16 rows, and
 * writes every token's logits to logits_all[n][n_vocab]. */
vx_error vx_model_verify(vx_model *model, const int *tokens, int n_tokens, float *logits_all);

/* The configuration vx_model_create would derive from a GGUF file (the
 * reference loader's rules, src/gguf.c:523-551 and src/format.c:185-322),
 * without touching the GPU. */
vx_error vx_model_read_config(const char *path, vx_model_config *cfg);

/* A random-init model built directly in HBM: weights N(0, std^2) quantised
 * with the reference's Q4_0 writer (Q8_0: amax/127), norms F32 ones.
 * cfg supplies n_layers, n_heads, n_kv_heads, n_embd, n_ff, n_vocab, n_ctx,
 * rope_theta; the rest is Llama defaults. */
typedef struct {
    uint64_t seed;
    float std;
    int matrix_type;           /* VX_TYPE_Q4_0 or VX_TYPE_Q8_0 (attention + FFN) */
    int embd_type;             /* token embedding                               */
    int output_type;           /* output projection                             */
} vx_synth_spec;
vx_error vx_model_create_synthetic(const vx_model_config *cfg, const vx_synth_spec *spec,
                                   vx_model **model);

/* Read one weight matrix back as GGUF blocks (host memory, rows*cols/32
 * blocks).  name uses GGUF tensor names ("blk.3.ffn_up.weight", ...). */
vx_error vx_model_read_tensor(const vx_model *model, const char *name, void *dst, size_t bytes);
/* Copy the device KV cache of one layer (positions [0, n)) to the host. */
vx_error vx_model_read_kv(const vx_model *model, int layer, int n, float *k, float *v);

/* ---- speculative decoding ---------------------------------------------------- */

/* vx_speculative_generate = prefill + decode.  prefill runs prompt[0..n-1)
 * through both models and stages prompt[n-1] as the first token to verify;
 * decode generates up to max_tokens from that state.  Each decode call
 * restarts from the state prefill left (KV caches are rolled back by
 * cache_len, uniforms restart), so repeated calls repeat the same work. */
int vx_speculative_prefill(vx_speculative_state *state, const int *prompt, int prompt_len);
int vx_speculative_decode(vx_speculative_state *state, int *output, int max_tokens);

/* Uniform draws come from splitmix64 streams keyed by this seed: draft token
 * i of round r uses u(seed, 1, r*k + i), verify position j uses
 * u(seed, 2, r*(k+1) + j); u = (splitmix64(...) >> 40) / 2^24. */
void vx_speculative_set_seed(vx_speculative_state *state, uint64_t seed);
float vx_uniform(uint64_t seed, uint64_t stream, uint64_t index);

typedef struct {
    int rounds;                /* verify steps run                                */
    int drafted;               /* draft tokens proposed                           */
    int accepted;              /* draft tokens accepted                           */
    int emitted;               /* tokens written to output                        */
    double verify_ms;          /* wall time in the batched target verify + accept */
    double draft_ms;           /* wall time in draft decoding                     */
    double prefill_ms;
} vx_speculative_stats;
void vx_speculative_get_stats(const vx_speculative_state *state, vx_speculative_stats *st);

/* Per-round trace (tests): for round r, the draft tokens, the emitted tokens
 * and the accepted count are appended to caller arrays when set. */
void vx_speculative_set_trace(vx_speculative_state *state, int *drafts, int *emitted,
                              int *accepted, int max_rounds);

/* ---- GEMM profiling ------------------------------------------------------------
 * vx_model_set_profiling(model, n), n >= 1: every n-th GEMM launch of each
 * matrix class is bracketed by two HIP events that the dispatch records
 * around the kernel on the model's stream (n = 1: every launch; 0: off);
 * vx_model_get_profile folds the elapsed times per class.  bytes are
 * algorithmic: weight blocks + fp32 activations in + fp32 results out.
 * VX_PROF_SWIGLU times the verify batches' SwiGLU panel launch that feeds
 * the down projection (bytes: the fp64 gate/up sums read and the fp16
 * hi/lo panel written; no flops). */
enum { VX_PROF_QKV = 0, VX_PROF_O, VX_PROF_GATEUP, VX_PROF_DOWN, VX_PROF_OUTPUT, VX_PROF_SWIGLU, VX_PROF_N };
typedef struct {
    int launches;
    double ms;
    double bytes;
    double flops;
} vx_gemm_profile;
void vx_model_set_profiling(vx_model *model, int on);
vx_error vx_model_get_profile(vx_model *model, vx_gemm_profile prof[VX_PROF_N]);

/* ---- library ------------------------------------------------------------------ */
const char *vx_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
