/*
 * oracle.h -- CPU oracle for the speculative-decoding verify path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a from-scratch C restatement of the
 * arithmetic of the reference CPU engine (spear34000/veltrix-engine), used by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker.  The product library never links, loads or calls it.
 *
 * Every function names the reference file:line it restates.  Pins (the
 * checks that make this oracle trustworthy) live in tests/test_oracle_*.py:
 * each function is compared against the reference built from its own sources
 * (oracle/_ref, see oracle/Makefile) and/or against closed forms.
 *
 * Two Q4_0 arithmetic modes mirror the two builds of the reference:
 *   OR_Q4_EXACT      -- portable build: d*(s-8)*x (src/quantize.c:728-750,
 *                       src/model.c:216-220)
 *   OR_Q4_AVX2LANES  -- x86 build: the lane pattern of vx_gemv_q4_0_avx2
 *                       (src/simd/avx2.c:311-370), which weights elements
 *                       t%8>=4 twice, offsets by 8*(sum x[0..31]+sum x[4..35])
 *                       and reads 4 floats past the row.
 */
#ifndef VX_ORACLE_H
#define VX_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#define OR_TYPE_F32  0
#define OR_TYPE_Q4_0 2
#define OR_TYPE_Q8_0 8

#define OR_Q4_EXACT     0
#define OR_Q4_AVX2LANES 1

/* ---- fp16 / blocks -------------------------------------------------- */
float    or_fp16_to_fp32(uint16_t h);
uint16_t or_fp32_to_fp16(float f);
void     or_quantize_row_q4_0(const float *x, void *y, int n);
void     or_dequantize_row_q4_0(const void *x, float *y, int n, float scale);
void     or_dequantize_row_q8_0(const void *x, float *y, int n, float scale);

/* ---- matrix-vector -------------------------------------------------- */
void or_gemv_q4_0(const void *A, const float *x, float *y, int rows, int cols);
void or_gemv_q4_0_sparse_rows(const void *A, const float *x, float *y, int rows, int cols,
                              const float *gate, float thr);
void or_gemv_f32(float *y, const float *A, const float *x, int rows, int cols);
void or_gemv_f32_sparse_rows(float *y, const float *A, const float *x, int rows, int cols,
                             const float *gate, float thr);
/* x must hold cols+4 readable floats (the lane pattern reads x[cols..cols+3]). */
void or_gemv_q4_0_avx2lanes(const void *A, const float *x, float *y, int rows, int cols);
void or_gemv_q4_0_avx2lanes_sparse_rows(const void *A, const float *x, float *y, int rows,
                                        int cols, const float *gate, float thr);
void or_gemv_f32_avx2lanes(float *y, const float *A, const float *x, int rows, int cols);

/* ---- elementwise ---------------------------------------------------- */
void  or_rms_norm(float *o, const float *x, const float *w, int n);
void  or_softmax(float *x, int n);
void  or_silu(float *x, int n);
void  or_rope(float *q, float *k, int pos, int n_heads, int n_kv_heads, int head_dim,
              int rope_dims, float theta);

/* ---- model ---------------------------------------------------------- */
typedef struct {
    int type;          /* OR_TYPE_*                      */
    const void *data;  /* NULL = tensor absent           */
    int rows, cols;    /* rows = ne[1], cols = ne[0]     */
} or_mat;

#define OR_MAX_FLIPS 4

typedef struct {
    int n_layers, n_heads, n_kv_heads, n_embd, n_head_dim, n_ff, n_vocab, n_ctx;
    float rope_theta;
    int   q4_mode;           /* OR_Q4_EXACT / OR_Q4_AVX2LANES                    */
    int   attn_cap;          /* attend to the first min(pos+1, attn_cap) positions;
                                4096 in the reference, 0 = no cap                  */
    int   attn_o_inplace;    /* 1: reproduce the portable build's in-place attn_o  */
    float gate_thr;          /* FFN up-row skip threshold, 0.01 in the reference  */
    float wscale;            /* synthetic weight scale (dequantize paths)         */
    or_mat tok_embd, output;
    const float *out_norm;   /* F32 or NULL                                       */
    int has_out_norm;        /* tensor present (weight may still be non-F32)      */
    const or_mat *wq, *wk, *wv, *wo, *wg, *wu, *wd;   /* [n_layers]               */
    const float *const *attn_norm;                    /* [n_layers], F32 or NULL  */
    const float *const *ffn_norm;
    const float *const *bq, *const *bk, *const *bv;   /* optional F32 biases      */
    float *k_cache, *v_cache;   /* [n_layers][n_ctx][kv_dim], caller-owned        */
    int cache_len;
    int kv_half;                /* 1: rows rounded to IEEE fp16 (nearest even) as
                                   they are stored -- the GPU engine's flagged fp16
                                   KV mode; 0 (the reference): fp32                 */
    /* Test hooks of the FFN gate-skip |silu(g_i)| < gate_thr (src/model.c:582-585;
     * the reference has no such hooks).  They let a test prove that a logit
     * difference comes from one skip decision that sits at the threshold. */
    float *gate_near;           /* optional [n][n_layers] (n = tokens of the call):
                                   min over FFN columns i of ||silu(g_i)| - gate_thr| */
    int *gate_near_idx;         /* optional [n][n_layers]: the column i of that minimum */
    int flip;                   /* number of inverted skip decisions (0..OR_MAX_FLIPS), */
    int flip_tok[OR_MAX_FLIPS];   /* each at token index within the call, layer, column */
    int flip_layer[OR_MAX_FLIPS];
    int flip_col[OR_MAX_FLIPS];
    /* Test hook of the cache store (the reference has no such hook).  With
     * kv_keep set, attention() leaves cache row pos as the caller placed it
     * (another engine's own stored row) and writes the row it computed, in
     * the cache's format, to kv_own_k / kv_own_v [n_layers][kv_dim] when they
     * are set.  Two engines then attend over identical cache contents, which
     * separates a difference in the arithmetic from binary16 rounding of two
     * fp32 values a few ulps apart landing on neighbouring binary16 values. */
    int kv_keep;
    float *kv_own_k, *kv_own_v;
} or_model;

/* x rounded to the nearest IEEE binary16 value (ties to even), as fp32:
 * overflow gives +-inf, NaN stays NaN. */
float or_round_half(float x);

/* Sequential single-token forwards over tokens[0..n); writes the last token's
 * logits (src/model.c:391-628).  Returns 0 or a negative error.  In the
 * OR_Q4_EXACT mode the tokens run layer-major in chunks (each matrix
 * dequantised once per chunk, tokens in vector lanes) with results
 * bit-identical to the token-major or_forward_tokenwise. */
int or_forward(or_model *m, const int *tokens, int n, float *logits);
/* Teacher-forced: logits for EVERY token (row i = logits after token i), i.e.
 * n calls of the reference forward with n_tokens = 1. */
int or_forward_all(or_model *m, const int *tokens, int n, float *logits_all);
/* The token-major restatement (one token through every layer, then the
 * next): all = 0 is or_forward, all = 1 or_forward_all. */
int or_forward_tokenwise(or_model *m, const int *tokens, int n, float *logits, int all);

/* ---- acceptance: textbook speculative sampling on softmax probabilities
 * (the reference compares raw logits, src/speculative.c:167, :205) ------ */
int  or_argmax(const float *x, int n);
/* p = softmax(l / T) with the reference's sample_top_p arithmetic
 * (src/speculative.c:44-53).  T must be > 0. */
void or_softmax_temp(const float *l, int n, float T, float *p);
/* Draft sampling distribution: nucleus of softmax(l/T) renormalised; returns
 * the sampled token for uniform u (src/speculative.c:35-91, ties -> lower index). */
int  or_sample_top_p(const float *l, int n, float T, float top_p, float u, float *q_out);
/* 2^32 fixed-point inverse CDF over w[0..n): first v with C_v >= max(1,
 * ceil(U*S/2^24)), U = u*2^24, W_v = round(w_v*2^32), C_v = W_0+..+W_v.  Returns -1 when the total mass is zero. */
int  or_inverse_cdf_fixed(const float *w, int n, float u);
int  or_accept_greedy(const float *L, int V, const int *draft, int k, int *out);
int  or_accept_sampled(const float *L, int V, const float *Q, int Vd, const int *draft, int k,
                       float T, const float *u, int *out, int *n_accepted);

#endif
