/*
 * vx_host.h -- internal declarations shared by the engine's C host files.
 * Not installed; the public surface is the headers in ../../include.
 */
#ifndef VX_HOST_H
#define VX_HOST_H

#include <stdint.h>
#include <stdio.h>

#include "quantize.h"
#include "veltrix.h"
#include "veltrix_gpu.h"
#include "vxh.h"

#define VX_MAX_BATCH 16
#define VX_PF_ROWS 512             /* rows of one large-M prefill chunk */

/* ---- errors ----------------------------------------------------------------- */
void vx_set_error(const char *fmt, ...);
vx_error vx_from_vxh(int rc);          /* maps VXH_ERR_* -> vx_error, keeps the message */
int vx_gpu_ready(void);                /* vxh_init() once; 0 or VXH_ERR_*            */

/* ---- GGUF loading (host/gguf.c) ------------------------------------------------- */
typedef struct {
    char name[VX_MAX_NAME];
    int type;                          /* ggml type id                          */
    int n_dims;
    int64_t ne[4];
    const uint8_t *data;               /* points into the file buffer            */
    size_t nbytes;                     /* bytes available for this tensor        */
} vx_gguf_tensor;

typedef struct {
    uint8_t *buf;
    size_t size;
    int n_tensors;
    vx_gguf_tensor *tensors;
    vx_model_config cfg;
} vx_gguf;

vx_error vx_gguf_open(const char *path, vx_gguf *g);
void vx_gguf_close(vx_gguf *g);
const vx_gguf_tensor *vx_gguf_find(const vx_gguf *g, const char *name);
/* The arch table / weight-name patterns of the reference (src/format.c:84-203). */
void vx_apply_arch(vx_model_config *cfg, const char *arch);
const vx_gguf_tensor *vx_gguf_find_role(const vx_gguf *g, const char *role, int layer);

/* ---- device model state (host/model.c) -------------------------------------------- */
typedef struct {
    vxh_qmat wqkv;                     /* rows [q | k | v], d + 2*kvd              */
    vxh_qmat wo;                       /* d x d, may be absent                     */
    vxh_qmat wgu;                      /* gate/up, 16-row interleaved tiles        */
    vxh_qmat wd;                       /* d x F                                    */
    int has_o;
    float *attn_norm, *ffn_norm;       /* device F32 or NULL (ones)                */
    float *bq, *bk, *bv;               /* device F32 biases or NULL                */
} vx_dev_layer;

typedef struct vx_dev {
    vxh_stream stream;
    int n_layers, d, n_heads, n_kv, hd, kvd, F, V;
    vx_dev_layer *layers;
    vxh_qmat embd;
    int has_embd;
    vxh_qmat out;
    int has_out, out_rows;
    float *out_norm;
    int has_out_norm;
    int has_f32;                       /* an F32 layer or output matrix: the plain-panel forward only */
    /* KV cache and RoPE tables, allocated on first use */
    int n_ctx_alloc;
    unsigned kv_gen;                   /* bumped whenever the cache is allocated or dropped */
    float *rope_cos, *rope_sin;
    int n_pos;
    /* activations, VX_MAX_BATCH rows */
    int *tok;                          /* [16]                                      */
    float *x, *xn, *xtail, *q, *att, *logits;
    /* fp64 GEMM accumulators (zero between uses; each consumer clears what
     * it reads): q|k|v rows, residual-stream updates, gate/up, logits */
    double *acc_qkv, *acc_x, *acc_gu, *acc_lg;
    int ld_qkv, ld_gu, ld_lg;
    int acc_dirty;                     /* a forward failed part-way: re-zero first */
    int acc_x_rows;                    /* rows of acc_x still holding a down projection
                                        * (the prologue forward's output GEMM reads it
                                        * in place); the next prologue forward clears
                                        * them with its embedding gather, others re-zero */
    vxh_panel pan_d, pan_f;
    vxh_workspace ws;
    /* sampling buffers */
    float *stats;                      /* [16][3]                                   */
    int *acc_out;                      /* [2 + 16]                                  */
    /* options */
    vx_model_options opt;
    /* per-layer RMSNorm sums of squares ss[(l * 2 + j) * 16 + m] (j = 0
     * attention norm, 1 FFN norm; l = L is the output norm), added by the
     * prologue GEMMs and applied to their products */
    double *ss;                        /* [(L+1)][2][16]; acc_x follows it in one allocation */
    /* decode forwards (at most two rows): every layer's own accumulators,
     * [row][layer][q|k|v, attention output, gate/up, down], after acc_x in
     * the same allocation, so the embedding gather's launch clears them all
     * and no GEMM of the forward clears an accumulator */
    double *acc_dec;
    int ld_dec_rec;                    /* doubles of one layer's record */
    /* prologue path: the second residual buffer (the residual alternates
     * between x and x2 inside a layer) and the attention projection's
     * accumulator (acc_x holds the down projection's) */
    float *x2;
    double *acc_y;
    /* large-M prompt prefill (allocated on first use): token ids, the
     * residual rows, normed rows, q|k|v rows, rotated q, attention rows,
     * gate/up rows, SwiGLU rows, each [VX_PF_ROWS][...] fp32, and the
     * attention workspace for that many rows */
    int pf_ready;
    int pf_ws_ctx, pf_ws_cap;          /* n_ctx_alloc and attn_cap pf_ws was sized for */
    int *pf_tok;
    float *pf_x, *pf_xn, *pf_qkv, *pf_q, *pf_att, *pf_gu, *pf_h;
    void *pf_px;                       /* rows panel of the GEMM input (vxh_rows_panel) */
    vxh_workspace pf_ws;
    /* GEMM profiling (vx_model_set_profiling) */
    int prof_on;                       /* 0: off; n: every n-th launch per class   */
    int prof_tick[VX_PROF_N];
    int prof_n, prof_cap;
    vxh_event *prof_ev;                /* [2 * prof_cap]                            */
    int *prof_cls;
    double *prof_bytes, *prof_flops;
    vx_gemm_profile prof[VX_PROF_N];
} vx_dev;

#define VX_LOGITS_NONE 0
#define VX_LOGITS_LAST 1
#define VX_LOGITS_ALL 2

/* Runs M <= 16 tokens (device ids in dev->tok) at positions n_past..;
 * logits land in dev->logits ([M][V] for ALL, row 0 for LAST).  Does not
 * touch cache_len. */
vx_error vx_dev_forward(vx_model *m, int M, int n_past, int logits_mode);
/* vx_dev_forward over M token ids already in device memory (ids[0..M)),
 * instead of the model's own token buffer: no copy launch. */
vx_error vx_dev_forward_ids(vx_model *m, const int *ids, int M, int n_past, int logits_mode);
/* Host-token convenience: uploads tokens, runs all batches, advances
 * cache_len with the reference's clamp rule. */
vx_error vx_dev_run_tokens(vx_model *m, const int *tokens, int n, int logits_mode,
                           float *logits_host);
vx_error vx_dev_ensure_kv(vx_model *m);
/* Exposed to speculative.c */
vx_dev *vx_dev_of(const vx_model *m);
double vx_now_ms(void);

/* ---- splitmix64 uniforms ---------------------------------------------------------- */
uint64_t vx_splitmix64(uint64_t x);

#endif
