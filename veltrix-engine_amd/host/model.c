/*
 * model.c -- vx_model on the GPU: creation (GGUF file or synthetic), weight
 * upload into tiled HBM matrices, and the batched forward that every entry
 * point (vx_model_forward, vx_model_verify, speculative decoding) runs.
 *
 * The forward restates the data flow of the reference's vx_model_forward
 * (src/model.c:391-628) for M tokens at once:
 *
 *   x = embed(tokens)                                      (:454-500)
 *   per layer:  q,k,v = W{q,k,v} . rmsnorm(x)               (:514-536)
 *               rope(q,k); write k,v at the rows' positions (:540, :291-296)
 *               a = attention(q)                            (:541, :275-341)
 *               x = x + Wo . a        (no Wo: x = x + a)    (:543-547)
 *               h = silu(Wg.n) * Wu.n, n = rmsnorm(x), up rows with
 *                   |silu(g)| < 0.01 zero                    (:551-585)
 *               x = x + Wd . h                              (:587-589)
 *   logits = Wout . rmsnorm(x)                              (:598-612)
 *
 * with Wq/Wk/Wv fused into one matrix and Wgate/Wup interleaved so the
 * SwiGLU product is formed in the GEMM epilogue.  Row m of a batch sits at
 * position n_past + m; causal attention inside the batch reproduces the
 * reference's one-token-at-a-time KV growth.
 */
#include <math.h>
#include <stdarg.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "model.h"
#include "vx_host.h"

/* --------------------------------------------------------------------------- */
/* errors / globals                                                             */
/* --------------------------------------------------------------------------- */
static __thread char g_err[512];
static vx_compute_level g_level = VX_COMPUTE_EXACT;
static int g_timing = 0;
static double g_timing_ms = 0.0;
static long g_timing_tokens = 0;

void vx_set_error(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

const char *vx_last_error(void) { return g_err; }

vx_error vx_from_vxh(int rc)
{
    if (rc == VXH_OK) return VX_OK;
    vx_set_error("%s", vxh_last_error());
    switch (rc) {
    case VXH_ERR_ALLOC: return VX_ERR_MEMORY;
    case VXH_ERR_PARAM: return VX_ERR_PARAM;
    default: return VX_ERR_UNSUPPORTED;
    }
}

int vx_gpu_ready(void) { return vxh_init(); }

double vx_now_ms(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

uint64_t vx_splitmix64(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

void vx_set_compute_level(vx_compute_level level) { g_level = level; }
void vx_enable_metalearn(bool enable) { (void)enable; }   /* accepted, ignored */
void vx_set_n_threads(int n) { (void)n; }   /* host threads do not matter here */

void vx_set_forward_timing_enabled(int enabled)
{
    g_timing = enabled ? 1 : 0;
    g_timing_ms = 0.0;
    g_timing_tokens = 0;
}

void vx_print_forward_timing(void)
{
    if (!g_timing) return;
    fprintf(stderr, "[timing] forward=%.1fms tokens=%ld\n", g_timing_ms, g_timing_tokens);
}

vx_dev *vx_dev_of(const vx_model *m) { return m ? (vx_dev *)m->dev : NULL; }

#define TRY(expr)                                                          \
    do {                                                                   \
        int rc_ = (expr);                                                  \
        if (rc_ != VXH_OK) return vx_from_vxh(rc_);                        \
    } while (0)

/* --------------------------------------------------------------------------- */
/* host-side model skeleton                                                     */
/* --------------------------------------------------------------------------- */
static vx_tensor **alloc_roles(int n) { return (vx_tensor **)calloc((size_t)(n > 0 ? n : 1), sizeof(vx_tensor *)); }

static void free_host(vx_model *m)
{
    if (!m) return;
    if (m->tensors) {
        for (int i = 0; i < m->n_tensors; i++) free(m->tensors[i]);
        free(m->tensors);
    }
    free(m->attn_q); free(m->attn_k); free(m->attn_v); free(m->attn_o);
    free(m->attn_q_bias); free(m->attn_k_bias); free(m->attn_v_bias);
    free(m->ffn_gate); free(m->ffn_up); free(m->ffn_down);
    free(m->ffn_gate_bias); free(m->ffn_up_bias); free(m->ffn_down_bias);
    free(m->attn_norm); free(m->ffn_norm); free(m->attn_norm_bias); free(m->ffn_norm_bias);
}

static int alloc_host_roles(vx_model *m, int L)
{
    m->attn_q = alloc_roles(L); m->attn_k = alloc_roles(L); m->attn_v = alloc_roles(L);
    m->attn_o = alloc_roles(L); m->attn_q_bias = alloc_roles(L); m->attn_k_bias = alloc_roles(L);
    m->attn_v_bias = alloc_roles(L); m->ffn_gate = alloc_roles(L); m->ffn_up = alloc_roles(L);
    m->ffn_down = alloc_roles(L); m->ffn_gate_bias = alloc_roles(L); m->ffn_up_bias = alloc_roles(L);
    m->ffn_down_bias = alloc_roles(L); m->attn_norm = alloc_roles(L); m->ffn_norm = alloc_roles(L);
    m->attn_norm_bias = alloc_roles(L); m->ffn_norm_bias = alloc_roles(L);
    return m->attn_q && m->attn_k && m->attn_v && m->attn_o && m->attn_q_bias && m->attn_k_bias &&
           m->attn_v_bias && m->ffn_gate && m->ffn_up && m->ffn_down && m->ffn_gate_bias &&
           m->ffn_up_bias && m->ffn_down_bias && m->attn_norm && m->ffn_norm && m->attn_norm_bias &&
           m->ffn_norm_bias;
}

static vx_tensor *add_tensor(vx_model *m, int cap, const char *name, int type, int64_t ne0,
                             int64_t ne1, size_t nbytes)
{
    if (m->n_tensors >= cap) return NULL;
    vx_tensor *t = (vx_tensor *)calloc(1, sizeof(vx_tensor));
    if (!t) return NULL;
    snprintf(t->name, VX_MAX_NAME, "%s", name);
    t->type = (vx_type)type;
    t->ne[0] = (int32_t)ne0;
    t->ne[1] = (int32_t)ne1;
    t->nbytes = nbytes;
    t->data = NULL;   /* bytes live on the device */
    m->tensors[m->n_tensors++] = t;
    return t;
}

/* --------------------------------------------------------------------------- */
/* device state                                                                 */
/* --------------------------------------------------------------------------- */
static int gu_rows(int F) { return (F + 15) / 16 * 32; }
static int round32(int n) { return (n + 31) / 32 * 32; }
static void prof_free(vx_dev *d);

static void dev_free(vx_dev *d)
{
    if (!d) return;
    if (d->layers) {
        for (int l = 0; l < d->n_layers; l++) {
            vx_dev_layer *L = &d->layers[l];
            vxh_qmat_free(&L->wqkv); vxh_qmat_free(&L->wo); vxh_qmat_free(&L->wgu); vxh_qmat_free(&L->wd);
            vxh_free(L->attn_norm); vxh_free(L->ffn_norm);
            vxh_free(L->bq); vxh_free(L->bk); vxh_free(L->bv);
        }
        free(d->layers);
    }
    vxh_qmat_free(&d->embd);
    vxh_qmat_free(&d->out);
    vxh_free(d->out_norm);
    vxh_free(d->rope_cos); vxh_free(d->rope_sin);
    vxh_free(d->tok); vxh_free(d->x); vxh_free(d->xn); vxh_free(d->xtail);
    vxh_free(d->q); vxh_free(d->att); vxh_free(d->logits);
    vxh_free(d->acc_qkv); vxh_free(d->acc_gu); vxh_free(d->acc_lg);
    vxh_free(d->stats); vxh_free(d->acc_out);
    vxh_free(d->ss);
    vxh_free(d->x2); vxh_free(d->acc_y);
    vxh_free(d->pf_tok); vxh_free(d->pf_x); vxh_free(d->pf_xn); vxh_free(d->pf_qkv);
    vxh_free(d->pf_q); vxh_free(d->pf_att); vxh_free(d->pf_gu); vxh_free(d->pf_h); vxh_free(d->pf_px);
    vxh_workspace_free(&d->pf_ws);
    vxh_panel_free(&d->pan_d);
    vxh_panel_free(&d->pan_f);
    vxh_workspace_free(&d->ws);
    prof_free(d);
    if (d->stream) vxh_stream_destroy(d->stream);
    free(d);
}

static vx_error dev_alloc_common(vx_model *m)
{
    const vx_model_config *c = &m->config;
    int rc = vx_gpu_ready();
    if (rc) return vx_from_vxh(rc);
    vx_dev *d = (vx_dev *)calloc(1, sizeof(vx_dev));
    if (!d) return VX_ERR_MEMORY;
    m->dev = d;
    d->n_layers = c->n_layers;
    d->d = c->n_embd;
    d->n_heads = c->n_heads;
    d->n_kv = c->n_kv_heads;
    d->hd = c->n_head_dim;
    d->kvd = c->n_kv_heads * c->n_head_dim;
    d->F = c->n_ff;
    d->V = c->n_vocab;
    d->opt.q4_kernel = VX_Q4_EXACT;
    d->opt.attn_cap = 4096;
    d->opt.ffn_gate_threshold = 0.01f;
    d->opt.fused = VX_FUSED_PROLOGUE;
    d->opt.pro_max_rows = VX_MAX_BATCH;
    d->opt.prefill_min_rows = 48;
    if (d->d % 32 || d->F % 32 || d->F <= 0 || d->d <= 0 || d->n_heads * d->hd != d->d ||
        d->hd % 2 || d->n_kv <= 0 || d->n_heads % d->n_kv) {
        vx_set_error("unsupported shape: n_embd %d n_ff %d heads %d/%d head_dim %d", d->d, d->F,
                     d->n_heads, d->n_kv, d->hd);
        return VX_ERR_UNSUPPORTED;
    }
    TRY(vxh_stream_create(&d->stream));
    d->layers = (vx_dev_layer *)calloc((size_t)(d->n_layers > 0 ? d->n_layers : 1), sizeof(vx_dev_layer));
    if (!d->layers) return VX_ERR_MEMORY;
    const int B = VX_MAX_BATCH;
    TRY(vxh_malloc((void **)&d->tok, sizeof(int) * B));
    TRY(vxh_malloc((void **)&d->x, sizeof(float) * B * d->d));
    TRY(vxh_malloc((void **)&d->xn, sizeof(float) * B * d->d));
    TRY(vxh_malloc((void **)&d->xtail, sizeof(float) * B * 4));
    TRY(vxh_fill_f32(d->xtail, 0.0f, B * 4, d->stream));
    TRY(vxh_malloc((void **)&d->q, sizeof(float) * B * d->d));
    TRY(vxh_malloc((void **)&d->att, sizeof(float) * B * d->d));
    TRY(vxh_malloc((void **)&d->logits, sizeof(float) * B * (size_t)d->V));
    d->ld_qkv = round32(d->d + 2 * d->kvd);
    d->ld_gu = gu_rows(d->F);
    d->ld_lg = round32(d->V);
    TRY(vxh_malloc((void **)&d->acc_qkv, sizeof(double) * B * (size_t)d->ld_qkv));
    /* ss then acc_x in one allocation, so the prologue forward clears both
     * (the sums of squares, the rows it starts from) with one range */
    const size_t n_ss = (size_t)(d->n_layers + 1) * 2 * B;
    d->ld_dec_rec = d->ld_qkv + d->d + d->ld_gu + d->d;
    const size_t n_dec = (size_t)B * (d->n_layers > 0 ? d->n_layers : 1) * d->ld_dec_rec;
    TRY(vxh_malloc((void **)&d->ss, sizeof(double) * (n_ss + (size_t)B * d->d + n_dec)));
    d->acc_x = d->ss + n_ss;
    d->acc_dec = d->acc_x + (size_t)B * d->d;
    TRY(vxh_fill_f32((float *)d->acc_dec, 0.0f, 2 * n_dec, d->stream));
    TRY(vxh_malloc((void **)&d->acc_gu, sizeof(double) * B * (size_t)d->ld_gu));
    TRY(vxh_malloc((void **)&d->acc_lg, sizeof(double) * B * (size_t)d->ld_lg));
    d->acc_dirty = 1;                  /* zeroed before the first forward */
    TRY(vxh_malloc((void **)&d->stats, sizeof(float) * (B + 1) * 3));
    TRY(vxh_malloc((void **)&d->acc_out, sizeof(int) * (B + 4)));
    TRY(vxh_panel_alloc(&d->pan_d, B, d->d));
    TRY(vxh_panel_alloc(&d->pan_f, B, d->F));
    TRY(vxh_malloc((void **)&d->x2, sizeof(float) * B * d->d));
    TRY(vxh_malloc((void **)&d->acc_y, sizeof(double) * B * (size_t)d->d));
    return VX_OK;
}

/* Upload n_rows GGUF rows (host or device) into a tiled matrix. */
static vx_error put_rows(vx_dev *d, vxh_qmat *q, const void *src, int on_dev, int n_rows, int group,
                         int stride, int offset)
{
    TRY(vxh_qmat_set_rows(q, src, on_dev, n_rows, group, stride, offset, d->stream));
    return VX_OK;
}

static vx_error upload_f32(vx_dev *d, float **dst, const void *src, int n)
{
    TRY(vxh_malloc((void **)dst, sizeof(float) * (size_t)n));
    TRY(vxh_upload(*dst, src, sizeof(float) * (size_t)n, d->stream));
    return VX_OK;
}

/* Workspace of the attention partials at n_ctx (the model's GEMMs use its
 * own accumulators, so the workspace accumulator is a token). */
static vx_error dev_alloc_workspace(vx_dev *d, int n_ctx, int cap)
{
    const int B = VX_MAX_BATCH;
    size_t an = vxh_attention_workspace_floats(B, n_ctx, cap, d->n_heads, d->n_kv, d->hd);
    if (d->ws.part && d->ws.part_floats >= an) return VX_OK;
    vxh_workspace_free(&d->ws);
    TRY(vxh_workspace_alloc(&d->ws, 32, an));
    return VX_OK;
}

vx_error vx_dev_ensure_kv(vx_model *m)
{
    vx_dev *d = vx_dev_of(m);
    int n_ctx = m->config.n_ctx > 0 ? m->config.n_ctx : 4096;
    if (m->k_cache && d->n_ctx_alloc == n_ctx) return VX_OK;
    if (m->k_cache) {
        /* n_ctx changed after the first forward: the reference keeps its
         * first allocation; so does this engine */
        return VX_OK;
    }
    size_t per = (size_t)(d->n_layers > 0 ? d->n_layers : 1) * n_ctx * d->kvd;
    const size_t esz = d->opt.kv_half ? 2 : sizeof(float);   /* kvd is even: whole floats */
    if ((size_t)n_ctx * d->kvd * esz > 0xFFFFFFFFull) {
        /* the attention kernels address a layer's rows with 32-bit offsets */
        vx_set_error("KV cache of %d positions x %d exceeds 4 GiB per layer", n_ctx, d->kvd);
        return VX_ERR_UNSUPPORTED;
    }
    TRY(vxh_malloc((void **)&m->k_cache, per * esz));
    TRY(vxh_malloc((void **)&m->v_cache, per * esz));
    TRY(vxh_fill_f32(m->k_cache, 0.0f, per * esz / sizeof(float), d->stream));
    TRY(vxh_fill_f32(m->v_cache, 0.0f, per * esz / sizeof(float), d->stream));
    d->n_ctx_alloc = n_ctx;
    d->kv_gen++;
    /* RoPE angle table for positions 0..n_ctx, computed like the reference
     * (src/tensor.c:182-187) */
    int half = d->hd / 2;
    d->n_pos = n_ctx + 1;
    float *cs = (float *)malloc(sizeof(float) * (size_t)d->n_pos * half);
    float *sn = (float *)malloc(sizeof(float) * (size_t)d->n_pos * half);
    if (!cs || !sn) { free(cs); free(sn); return VX_ERR_MEMORY; }
    float theta = m->config.rope_theta;
    for (int i = 0; i < half; i++) {
        float freq = 1.0f / powf(theta, (float)(i * 2) / (float)d->hd);
        for (int p = 0; p < d->n_pos; p++) {
            float ang = (float)p * freq;
            cs[(size_t)p * half + i] = cosf(ang);
            sn[(size_t)p * half + i] = sinf(ang);
        }
    }
    /* a cache dropped by vx_model_set_options kept its tables */
    if (d->rope_cos) { vxh_free(d->rope_cos); d->rope_cos = NULL; }
    if (d->rope_sin) { vxh_free(d->rope_sin); d->rope_sin = NULL; }
    vx_error e = upload_f32(d, &d->rope_cos, cs, d->n_pos * half);
    if (e == VX_OK) e = upload_f32(d, &d->rope_sin, sn, d->n_pos * half);
    free(cs);
    free(sn);
    if (e != VX_OK) return e;
    e = dev_alloc_workspace(d, n_ctx, d->opt.attn_cap);
    if (e != VX_OK) return e;
    TRY(vxh_stream_sync(d->stream));
    return VX_OK;
}

/* --------------------------------------------------------------------------- */
/* creation from GGUF                                                           */
/* --------------------------------------------------------------------------- */
static int is_quant_type(int t) { return t == VX_TYPE_Q4_0 || t == VX_TYPE_Q8_0; }
/* matrix types a GGUF may carry: the quantised ones and F32 (src/model.c:174-179, 206-211) */
static int is_mat_type(int t) { return is_quant_type(t) || t == VX_TYPE_F32; }

static vx_error check_mat(const vx_gguf_tensor *t, int rows, int cols, int *type)
{
    if (!t) return VX_OK;
    if (!is_mat_type(t->type)) {
        vx_set_error("%s: type %d not supported (Q4_0, Q8_0 and F32 only)", t->name, t->type);
        return VX_ERR_UNSUPPORTED;
    }
    if (t->type == VX_TYPE_F32 && cols % 32) {
        vx_set_error("%s: F32 rows of %d columns (a multiple of 32 needed)", t->name, cols);
        return VX_ERR_UNSUPPORTED;
    }
    if (t->ne[0] != cols || t->ne[1] != rows) {
        vx_set_error("%s: shape %lldx%lld, expected %dx%d", t->name, (long long)t->ne[1],
                     (long long)t->ne[0], rows, cols);
        return VX_ERR_FORMAT;
    }
    size_t need = t->type == VX_TYPE_F32 ? (size_t)rows * cols * sizeof(float)
                                         : (size_t)rows * (cols / 32) * (t->type == VX_TYPE_Q4_0 ? 18 : 34);
    if (t->nbytes < need) {
        vx_set_error("%s: truncated (%zu of %zu bytes)", t->name, t->nbytes, need);
        return VX_ERR_FORMAT;
    }
    if (*type < 0) *type = t->type;
    else if (*type != t->type) {
        vx_set_error("%s: fused matrices need one type (%d vs %d)", t->name, t->type, *type);
        return VX_ERR_UNSUPPORTED;
    }
    return VX_OK;
}

static const float *f32_or_null(const vx_gguf_tensor *t, int n)
{
    if (!t || t->type != VX_TYPE_F32 || t->nbytes < sizeof(float) * (size_t)n) return NULL;
    return (const float *)t->data;
}

static vx_tensor *meta_of(vx_model *m, int cap, const vx_gguf_tensor *t)
{
    if (!t) return NULL;
    return add_tensor(m, cap, t->name, t->type, t->ne[0], t->ne[1], t->nbytes);
}

static vx_error create_from_gguf(vx_gguf *g, vx_model *m)
{
    m->config = g->cfg;
    const vx_model_config *c = &m->config;
    if (c->n_layers <= 0) return VX_ERR_PARAM;
    if (c->n_embd <= 0 || c->n_embd > 8192) return VX_ERR_PARAM;
    if (c->mlp_type != VX_MLP_SWIGLU || c->norm_type != VX_NORM_RMS) {
        vx_set_error("architecture %d (mlp %d, norm %d) not supported: Llama-family SwiGLU + RMSNorm only",
                     c->arch, c->mlp_type, c->norm_type);
        return VX_ERR_UNSUPPORTED;
    }
    if (c->rope_partial_dims > 0 && c->rope_partial_dims < c->n_head_dim) return VX_ERR_UNSUPPORTED;
    int L = c->n_layers;
    int cap = g->n_tensors + 4;
    m->tensors = (vx_tensor **)calloc((size_t)cap, sizeof(vx_tensor *));
    if (!m->tensors || !alloc_host_roles(m, L)) return VX_ERR_MEMORY;
    vx_error e = dev_alloc_common(m);
    if (e != VX_OK) return e;
    vx_dev *d = vx_dev_of(m);
    const int dd = d->d, kvd = d->kvd, F = d->F, V = d->V;

    /* embedding / output / final norm */
    const vx_gguf_tensor *te = vx_gguf_find_role(g, "tok_embd", -1);
    const vx_gguf_tensor *to = vx_gguf_find_role(g, "output", -1);
    const vx_gguf_tensor *tn = vx_gguf_find_role(g, "output_norm", -1);
    m->tok_embd = meta_of(m, cap, te);
    m->output_w = to ? meta_of(m, cap, to) : m->tok_embd;   /* src/format.c:237-238 */
    m->norm_w = meta_of(m, cap, tn);
    if (!to) to = te;
    if (te) {
        int et = -1;
        if ((e = check_mat(te, (int)te->ne[1], dd, &et)) != VX_OK) return e;
        TRY(vxh_qmat_alloc(&d->embd, te->type, (int)te->ne[1], dd));
        if ((e = put_rows(d, &d->embd, te->data, 0, (int)te->ne[1], (int)te->ne[1], 0, 0)) != VX_OK) return e;
        d->has_embd = 1;
    }
    if (to) {
        int ot = -1;
        int rows = (int)to->ne[1];
        if ((e = check_mat(to, rows, dd, &ot)) != VX_OK) return e;
        if (rows > 0 && rows <= V) {
            TRY(vxh_qmat_alloc(&d->out, to->type, rows, dd));
            if ((e = put_rows(d, &d->out, to->data, 0, rows, rows, 0, 0)) != VX_OK) return e;
            d->has_out = 1;
            d->out_rows = rows;
            if (to->type == VX_TYPE_F32) d->has_f32 = 1;
        }
    }
    if (tn) {
        d->has_out_norm = 1;
        const float *w = f32_or_null(tn, dd);
        if (w && (e = upload_f32(d, &d->out_norm, w, dd)) != VX_OK) return e;
    }

    for (int l = 0; l < L; l++) {
        vx_dev_layer *Ld = &d->layers[l];
        const vx_gguf_tensor *tq = vx_gguf_find_role(g, "attn_q", l), *tk = vx_gguf_find_role(g, "attn_k", l),
                             *tv = vx_gguf_find_role(g, "attn_v", l), *tO = vx_gguf_find_role(g, "attn_o", l),
                             *tg = vx_gguf_find_role(g, "ffn_gate", l), *tu = vx_gguf_find_role(g, "ffn_up", l),
                             *tdn = vx_gguf_find_role(g, "ffn_down", l),
                             *tan = vx_gguf_find_role(g, "attn_norm", l), *tfn = vx_gguf_find_role(g, "ffn_norm", l),
                             *tbq = vx_gguf_find_role(g, "attn_q_bias", l),
                             *tbk = vx_gguf_find_role(g, "attn_k_bias", l),
                             *tbv = vx_gguf_find_role(g, "attn_v_bias", l);
        m->attn_q[l] = meta_of(m, cap, tq); m->attn_k[l] = meta_of(m, cap, tk);
        m->attn_v[l] = meta_of(m, cap, tv); m->attn_o[l] = meta_of(m, cap, tO);
        m->ffn_gate[l] = meta_of(m, cap, tg); m->ffn_up[l] = meta_of(m, cap, tu);
        m->ffn_down[l] = meta_of(m, cap, tdn); m->attn_norm[l] = meta_of(m, cap, tan);
        m->ffn_norm[l] = meta_of(m, cap, tfn); m->attn_q_bias[l] = meta_of(m, cap, tbq);
        m->attn_k_bias[l] = meta_of(m, cap, tbk); m->attn_v_bias[l] = meta_of(m, cap, tbv);

        int tqkv = -1, tgu = -1, to1 = -1, td1 = -1;
        if ((e = check_mat(tq, dd, dd, &tqkv)) || (e = check_mat(tk, kvd, dd, &tqkv)) ||
            (e = check_mat(tv, kvd, dd, &tqkv)) || (e = check_mat(tO, dd, dd, &to1)) ||
            (e = check_mat(tg, F, dd, &tgu)) || (e = check_mat(tu, F, dd, &tgu)) ||
            (e = check_mat(tdn, dd, F, &td1)))
            return e;
        if (tqkv < 0) tqkv = VX_TYPE_Q4_0;
        if (tgu < 0) tgu = VX_TYPE_Q4_0;
        if (td1 < 0) td1 = VX_TYPE_Q4_0;
        if (tqkv == VX_TYPE_F32 || tgu == VX_TYPE_F32 || td1 == VX_TYPE_F32 || to1 == VX_TYPE_F32) d->has_f32 = 1;
        TRY(vxh_qmat_alloc(&Ld->wqkv, tqkv, dd + 2 * kvd, dd));
        if (tq && (e = put_rows(d, &Ld->wqkv, tq->data, 0, dd, dd, 0, 0))) return e;
        if (tk && (e = put_rows(d, &Ld->wqkv, tk->data, 0, kvd, kvd, 0, dd))) return e;
        if (tv && (e = put_rows(d, &Ld->wqkv, tv->data, 0, kvd, kvd, 0, dd + kvd))) return e;
        if (tO) {
            TRY(vxh_qmat_alloc(&Ld->wo, to1, dd, dd));
            if ((e = put_rows(d, &Ld->wo, tO->data, 0, dd, dd, 0, 0))) return e;
            Ld->has_o = 1;
        }
        TRY(vxh_qmat_alloc(&Ld->wgu, tgu, gu_rows(F), dd));
        if (tg && (e = put_rows(d, &Ld->wgu, tg->data, 0, F, 16, 32, 0))) return e;
        if (tu && (e = put_rows(d, &Ld->wgu, tu->data, 0, F, 16, 32, 16))) return e;
        TRY(vxh_qmat_alloc(&Ld->wd, td1, dd, F));
        if (tdn && (e = put_rows(d, &Ld->wd, tdn->data, 0, dd, dd, 0, 0))) return e;
        const float *w;
        if ((w = f32_or_null(tan, dd)) && (e = upload_f32(d, &Ld->attn_norm, w, dd))) return e;
        if ((w = f32_or_null(tfn, dd)) && (e = upload_f32(d, &Ld->ffn_norm, w, dd))) return e;
        if ((w = f32_or_null(tbq, dd)) && (e = upload_f32(d, &Ld->bq, w, dd))) return e;
        if ((w = f32_or_null(tbk, kvd)) && (e = upload_f32(d, &Ld->bk, w, kvd))) return e;
        if ((w = f32_or_null(tbv, kvd)) && (e = upload_f32(d, &Ld->bv, w, kvd))) return e;
    }
    TRY(vxh_stream_sync(d->stream));
    return VX_OK;
}

vx_error vx_model_read_config(const char *path, vx_model_config *cfg)
{
    if (!path || !cfg) return VX_ERR_PARAM;
    vx_gguf g;
    vx_error e = vx_gguf_open(path, &g);
    if (e != VX_OK) return e;
    *cfg = g.cfg;
    vx_gguf_close(&g);
    return VX_OK;
}

vx_error vx_model_create(const char *path, vx_model **out)
{
    if (!path || !out) return VX_ERR_PARAM;
    *out = NULL;
    vx_gguf g;
    vx_error e = vx_gguf_open(path, &g);
    if (e != VX_OK) return e;
    vx_model *m = (vx_model *)calloc(1, sizeof(vx_model));
    if (!m) { vx_gguf_close(&g); return VX_ERR_MEMORY; }
    e = create_from_gguf(&g, m);
    vx_gguf_close(&g);
    if (e != VX_OK) { vx_model_destroy(m); return e; }
    *out = m;
    return VX_OK;
}

/* --------------------------------------------------------------------------- */
/* synthetic models                                                             */
/* --------------------------------------------------------------------------- */
static vx_error synth_into(vx_dev *d, void *stage, vxh_qmat *q, int type, int rows, int cols,
                           uint64_t seed, float std, int group, int stride, int offset)
{
    TRY(vxh_synth_blocks(stage, type, rows, cols, seed, std, d->stream));
    return put_rows(d, q, stage, 1, rows, group, stride, offset);
}

vx_error vx_model_create_synthetic(const vx_model_config *cfg, const vx_synth_spec *spec,
                                   vx_model **out)
{
    if (!cfg || !spec || !out) return VX_ERR_PARAM;
    *out = NULL;
    int mt = spec->matrix_type, et = spec->embd_type, ot = spec->output_type;
    if (!is_quant_type(mt) || !is_quant_type(et) || !is_quant_type(ot)) return VX_ERR_UNSUPPORTED;
    vx_model *m = (vx_model *)calloc(1, sizeof(vx_model));
    if (!m) return VX_ERR_MEMORY;
    vx_model_config *c = &m->config;
    c->n_layers = cfg->n_layers;
    c->n_heads = cfg->n_heads;
    c->n_kv_heads = cfg->n_kv_heads > 0 ? cfg->n_kv_heads : cfg->n_heads;
    c->n_embd = cfg->n_embd;
    c->n_head_dim = cfg->n_embd / (cfg->n_heads > 0 ? cfg->n_heads : 1);
    c->n_ff = cfg->n_ff;
    c->n_vocab = cfg->n_vocab;
    c->n_ctx = cfg->n_ctx > 0 ? cfg->n_ctx : 4096;
    c->rope_theta = cfg->rope_theta > 0 ? cfg->rope_theta : 10000.0f;
    c->n_threads = 1;
    vx_apply_arch(c, "llama");
    int L = c->n_layers;
    int cap = 9 * L + 4;
    m->tensors = (vx_tensor **)calloc((size_t)cap, sizeof(vx_tensor *));
    vx_error e = VX_OK;
    if (!m->tensors || !alloc_host_roles(m, L)) { e = VX_ERR_MEMORY; goto fail; }
    if ((e = dev_alloc_common(m)) != VX_OK) goto fail;
    {
        vx_dev *d = vx_dev_of(m);
        const int dd = d->d, kvd = d->kvd, F = d->F, V = d->V;
        /* the staging buffer holds the largest matrix synthesised through it:
         * rows V, d, kvd or F (embedding/output, q and attn_o, k/v, gate/up)
         * of d columns, or d rows of F columns (down) */
        int rmax = V > dd ? V : dd;
        if (kvd > rmax) rmax = kvd;
        if (F > rmax) rmax = F;
        size_t big = (size_t)rmax * dd;
        void *stage = NULL;
        int rc = vxh_malloc(&stage, big / 32 * 34);
        if (rc) { e = vx_from_vxh(rc); goto fail; }
        uint64_t s0 = spec->seed;
        float sd = spec->std;
#define SEED(i) vx_splitmix64(s0 + (uint64_t)(i) * 0x9E3779B97F4A7C15ull)
        char nm[VX_MAX_NAME];
        if ((rc = vxh_qmat_alloc(&d->embd, et, V, dd))) { e = vx_from_vxh(rc); goto fail_stage; }
        if ((e = synth_into(d, stage, &d->embd, et, V, dd, SEED(1), sd, V, 0, 0))) goto fail_stage;
        d->has_embd = 1;
        if ((rc = vxh_qmat_alloc(&d->out, ot, V, dd))) { e = vx_from_vxh(rc); goto fail_stage; }
        if ((e = synth_into(d, stage, &d->out, ot, V, dd, SEED(2), sd, V, 0, 0))) goto fail_stage;
        d->has_out = 1;
        d->out_rows = V;
        d->has_out_norm = 1;
        m->tok_embd = add_tensor(m, cap, "token_embd.weight", et, dd, V, (size_t)V * dd / 32 * (et == 2 ? 18 : 34));
        m->output_w = add_tensor(m, cap, "output.weight", ot, dd, V, (size_t)V * dd / 32 * (ot == 2 ? 18 : 34));
        m->norm_w = add_tensor(m, cap, "output_norm.weight", VX_TYPE_F32, dd, 1, sizeof(float) * dd);
        size_t bq = (size_t)(mt == 2 ? 18 : 34);
        for (int l = 0; l < L; l++) {
            vx_dev_layer *Ld = &d->layers[l];
            uint64_t b = 16 + (uint64_t)l * 8;
            if ((rc = vxh_qmat_alloc(&Ld->wqkv, mt, dd + 2 * kvd, dd))) { e = vx_from_vxh(rc); goto fail_stage; }
            if ((e = synth_into(d, stage, &Ld->wqkv, mt, dd, dd, SEED(b + 0), sd, dd, 0, 0))) goto fail_stage;
            if ((e = synth_into(d, stage, &Ld->wqkv, mt, kvd, dd, SEED(b + 1), sd, kvd, 0, dd))) goto fail_stage;
            if ((e = synth_into(d, stage, &Ld->wqkv, mt, kvd, dd, SEED(b + 2), sd, kvd, 0, dd + kvd))) goto fail_stage;
            if ((rc = vxh_qmat_alloc(&Ld->wo, mt, dd, dd))) { e = vx_from_vxh(rc); goto fail_stage; }
            if ((e = synth_into(d, stage, &Ld->wo, mt, dd, dd, SEED(b + 3), sd, dd, 0, 0))) goto fail_stage;
            Ld->has_o = 1;
            if ((rc = vxh_qmat_alloc(&Ld->wgu, mt, gu_rows(F), dd))) { e = vx_from_vxh(rc); goto fail_stage; }
            if ((e = synth_into(d, stage, &Ld->wgu, mt, F, dd, SEED(b + 4), sd, 16, 32, 0))) goto fail_stage;
            if ((e = synth_into(d, stage, &Ld->wgu, mt, F, dd, SEED(b + 5), sd, 16, 32, 16))) goto fail_stage;
            if ((rc = vxh_qmat_alloc(&Ld->wd, mt, dd, F))) { e = vx_from_vxh(rc); goto fail_stage; }
            if ((e = synth_into(d, stage, &Ld->wd, mt, dd, F, SEED(b + 6), sd, dd, 0, 0))) goto fail_stage;
            snprintf(nm, sizeof nm, "blk.%d.attn_norm.weight", l);
            m->attn_norm[l] = add_tensor(m, cap, nm, VX_TYPE_F32, dd, 1, sizeof(float) * dd);
            snprintf(nm, sizeof nm, "blk.%d.attn_q.weight", l);
            m->attn_q[l] = add_tensor(m, cap, nm, mt, dd, dd, (size_t)dd * dd / 32 * bq);
            snprintf(nm, sizeof nm, "blk.%d.attn_k.weight", l);
            m->attn_k[l] = add_tensor(m, cap, nm, mt, dd, kvd, (size_t)kvd * dd / 32 * bq);
            snprintf(nm, sizeof nm, "blk.%d.attn_v.weight", l);
            m->attn_v[l] = add_tensor(m, cap, nm, mt, dd, kvd, (size_t)kvd * dd / 32 * bq);
            snprintf(nm, sizeof nm, "blk.%d.attn_output.weight", l);
            m->attn_o[l] = add_tensor(m, cap, nm, mt, dd, dd, (size_t)dd * dd / 32 * bq);
            snprintf(nm, sizeof nm, "blk.%d.ffn_norm.weight", l);
            m->ffn_norm[l] = add_tensor(m, cap, nm, VX_TYPE_F32, dd, 1, sizeof(float) * dd);
            snprintf(nm, sizeof nm, "blk.%d.ffn_gate.weight", l);
            m->ffn_gate[l] = add_tensor(m, cap, nm, mt, dd, F, (size_t)F * dd / 32 * bq);
            snprintf(nm, sizeof nm, "blk.%d.ffn_up.weight", l);
            m->ffn_up[l] = add_tensor(m, cap, nm, mt, dd, F, (size_t)F * dd / 32 * bq);
            snprintf(nm, sizeof nm, "blk.%d.ffn_down.weight", l);
            m->ffn_down[l] = add_tensor(m, cap, nm, mt, F, dd, (size_t)F * dd / 32 * bq);
        }
#undef SEED
        rc = vxh_stream_sync(d->stream);
        vxh_free(stage);
        if (rc) { e = vx_from_vxh(rc); goto fail; }
    }
    *out = m;
    return VX_OK;
fail_stage:
fail:
    vx_model_destroy(m);
    return e;
}

void vx_model_destroy(vx_model *m)
{
    if (!m) return;
    vx_dev *d = vx_dev_of(m);
    if (d) {
        vxh_stream_sync(d->stream);
        vxh_free(m->k_cache);
        vxh_free(m->v_cache);
        dev_free(d);
    }
    free_host(m);
    free(m);
}

void vx_model_kv_truncate(vx_model *m, int length)
{
    if (!m) return;
    if (length < 0) length = 0;
    if (length <= m->cache_len) m->cache_len = length;
}

void vx_model_get_options(const vx_model *m, vx_model_options *opt)
{
    vx_dev *d = vx_dev_of(m);
    if (d && opt) *opt = d->opt;
}

vx_error vx_model_set_options(vx_model *m, const vx_model_options *opt)
{
    vx_dev *d = vx_dev_of(m);
    if (!d || !opt) return VX_ERR_PARAM;
    if (opt->q4_kernel != VX_Q4_EXACT && opt->q4_kernel != VX_Q4_AVX2_LANES) return VX_ERR_PARAM;
    if (opt->attn_cap < 0) return VX_ERR_PARAM;
    if ((opt->fused != VX_FUSED_NONE && opt->fused != VX_FUSED_PROLOGUE) || opt->pro_max_rows < 0)
        return VX_ERR_PARAM;
    if (opt->kv_half != 0 && opt->kv_half != 1) return VX_ERR_PARAM;
    if (opt->prefill_min_rows < 0) return VX_ERR_PARAM;
    if (opt->kv_half) {
        /* every forward must take the q|k|v attention kernel, the only one
         * with an fp16 cache */
        int has_o = 1;
        for (int l = 0; l < d->n_layers; l++) has_o &= d->layers[l].has_o;
        if (opt->fused != VX_FUSED_PROLOGUE || opt->q4_kernel != VX_Q4_EXACT || opt->pro_max_rows < VX_MAX_BATCH ||
            (d->hd != 64 && d->hd != 128) || !has_o || d->has_f32) {
            vx_set_error("fp16 KV cache: needs the prologue path, exact Q4_0, pro_max_rows >= %d, "
                         "head_dim 64 or 128 and no F32 matrices", VX_MAX_BATCH);
            return VX_ERR_UNSUPPORTED;
        }
    }
    int cap_changed = opt->attn_cap != d->opt.attn_cap;
    int kv_changed = opt->kv_half != d->opt.kv_half;
    if (kv_changed && m->k_cache) {
        /* a cache of the other element type: dropped, allocated again by the next forward */
        TRY(vxh_stream_sync(d->stream));
        vxh_free(m->k_cache);
        vxh_free(m->v_cache);
        m->k_cache = m->v_cache = NULL;
        m->cache_len = 0;
        d->kv_gen++;
    }
    d->opt = *opt;   /* the prefill workspace follows the cap on its next use (pf_alloc) */
    if (cap_changed && m->k_cache) return dev_alloc_workspace(d, d->n_ctx_alloc, d->opt.attn_cap);
    return VX_OK;
}

/* --------------------------------------------------------------------------- */
/* the batched forward                                                          */
/* --------------------------------------------------------------------------- */
static float scale_for(const vx_dev *d, int type)
{
    /* the synthetic weight scale reaches every dequantize path of the
     * reference; the x86 Q4_0 kernel bypasses it (src/model.c:212-244) */
    float s = vx_get_synthetic_weight_scale();
    if (type == VX_TYPE_Q4_0 && d->opt.q4_kernel == VX_Q4_AVX2_LANES) return 1.0f;
    if (type == VX_TYPE_F32) return 1.0f;   /* F32 GEMVs read the weights as they are */
    return s;
}

/* Folds the recorded event pairs into d->prof (synchronises the stream). */
static vx_error prof_fold(vx_dev *d)
{
    if (d->prof_n == 0) return VX_OK;
    TRY(vxh_stream_sync(d->stream));
    for (int i = 0; i < d->prof_n; i++) {
        float ms = 0.0f;
        TRY(vxh_event_elapsed_ms(d->prof_ev[2 * i], d->prof_ev[2 * i + 1], &ms));
        vx_gemm_profile *p = &d->prof[d->prof_cls[i]];
        p->launches++;
        p->ms += ms;
        p->bytes += d->prof_bytes[i];
        p->flops += d->prof_flops[i];
    }
    d->prof_n = 0;
    return VX_OK;
}

static void prof_free(vx_dev *d)
{
    for (int i = 0; i < 2 * d->prof_cap; i++) vxh_event_destroy(d->prof_ev[i]);
    free(d->prof_ev);
    free(d->prof_cls);
    free(d->prof_bytes);
    free(d->prof_flops);
    d->prof_ev = NULL;
    d->prof_cls = NULL;
    d->prof_bytes = d->prof_flops = NULL;
    d->prof_cap = d->prof_n = 0;
}

void vx_model_set_profiling(vx_model *m, int on)
{
    vx_dev *d = vx_dev_of(m);
    if (!d) return;
    prof_fold(d);
    memset(d->prof, 0, sizeof(d->prof));
    d->prof_on = on > 0 ? on : 0;
    memset(d->prof_tick, 0, sizeof(d->prof_tick));
    if (d->prof_on && !d->prof_cap) {
        int cap = 4096;
        d->prof_ev = (vxh_event *)calloc((size_t)cap * 2, sizeof(vxh_event));
        d->prof_cls = (int *)calloc((size_t)cap, sizeof(int));
        d->prof_bytes = (double *)calloc((size_t)cap, sizeof(double));
        d->prof_flops = (double *)calloc((size_t)cap, sizeof(double));
        if (!d->prof_ev || !d->prof_cls || !d->prof_bytes || !d->prof_flops) { prof_free(d); d->prof_on = 0; return; }
        for (int i = 0; i < 2 * cap; i++)
            if (vxh_event_create(&d->prof_ev[i]) != VXH_OK) { d->prof_cap = i / 2; prof_free(d); d->prof_on = 0; return; }
        d->prof_cap = cap;
    }
}

vx_error vx_model_get_profile(vx_model *m, vx_gemm_profile prof[VX_PROF_N])
{
    vx_dev *d = vx_dev_of(m);
    if (!d || !prof) return VX_ERR_PARAM;
    vx_error e = prof_fold(d);
    memcpy(prof, d->prof, sizeof(d->prof));
    return e;
}

/* Profiling slot for one GEMM launch (NULL events when profiling is off). */
static vx_error prof_slot(vx_dev *d, const vxh_qmat *W, int M, int n_out, int cls, int rows_logical,
                          vxh_event *e0, vxh_event *e1)
{
    *e0 = *e1 = NULL;
    if (!d->prof_on) return VX_OK;
    if (d->prof_tick[cls]++ % d->prof_on) return VX_OK;   /* every prof_on-th launch of the class */
    if (d->prof_n == d->prof_cap) {
        vx_error e = prof_fold(d);
        if (e != VX_OK) return e;
    }
    int slot = d->prof_n++;
    d->prof_cls[slot] = cls;
    double wb = (double)rows_logical * W->n_cols / 32.0 * (W->type == VX_TYPE_Q4_0 ? 18.0 : 34.0);
    d->prof_bytes[slot] = wb + 4.0 * M * W->n_cols + 4.0 * M * n_out;
    d->prof_flops[slot] = 2.0 * M * (double)rows_logical * W->n_cols;
    *e0 = d->prof_ev[2 * slot];
    *e1 = d->prof_ev[2 * slot + 1];
    return VX_OK;
}

/* Profiling slot of a SwiGLU panel launch of M rows of F columns. */
static vx_error prof_slot_panel(vx_dev *d, int M, int F, vxh_event *e0, vxh_event *e1)
{
    *e0 = *e1 = NULL;
    if (!d->prof_on) return VX_OK;
    if (d->prof_tick[VX_PROF_SWIGLU]++ % d->prof_on) return VX_OK;
    if (d->prof_n == d->prof_cap) {
        vx_error e = prof_fold(d);
        if (e != VX_OK) return e;
    }
    int slot = d->prof_n++;
    d->prof_cls[slot] = VX_PROF_SWIGLU;
    d->prof_bytes[slot] = 16.0 * M * F + 4.0 * M * F;
    d->prof_flops[slot] = 0.0;
    *e0 = d->prof_ev[2 * slot];
    *e1 = d->prof_ev[2 * slot + 1];
    return VX_OK;
}

/* acc[m][n] += scale * (W x_m)[n] for n < n_out (fp64 accumulator). */
static vx_error gemm(vx_dev *d, const vxh_qmat *W, vxh_panel *P, int M, double *acc, int ld_acc,
                     int n_out, int cls, int rows_logical)
{
    vxh_event e0, e1;
    vx_error e = prof_slot(d, W, M, n_out, cls, rows_logical, &e0, &e1);
    if (e != VX_OK) return e;
    TRY(vxh_gemm_acc_timed(W, P, M, acc, ld_acc, n_out, scale_for(d, W->type), NULL, 0, 0.0f,
                           VXH_PATH_AUTO, e0, e1, d->stream));
    return VX_OK;
}

static vx_error zero_acc(vx_dev *d)
{
    const int B = VX_MAX_BATCH;
    vxh_stream s = d->stream;
    TRY(vxh_fill_f32((float *)d->acc_qkv, 0.0f, 2 * (size_t)B * d->ld_qkv, s));
    TRY(vxh_fill_f32((float *)d->acc_x, 0.0f, 2 * (size_t)B * d->d, s));
    d->acc_x_rows = 0;
    TRY(vxh_fill_f32((float *)d->acc_gu, 0.0f, 2 * (size_t)B * d->ld_gu, s));
    TRY(vxh_fill_f32((float *)d->acc_lg, 0.0f, 2 * (size_t)B * d->ld_lg, s));
    TRY(vxh_fill_f32((float *)d->acc_y, 0.0f, 2 * (size_t)B * d->d, s));
    d->acc_dirty = 0;
    return VX_OK;
}

/* The prologue path needs the exact Q4_0 kernel (the AVX2-lane corrections
 * come with the separate panels) and an output projection in every layer;
 * it runs batches of at most pro_max_rows rows. */
static int pro_ok(const vx_dev *d, int M)
{
    if (d->opt.fused != VX_FUSED_PROLOGUE || M > d->opt.pro_max_rows) return 0;
    if (d->opt.q4_kernel != VX_Q4_EXACT || d->has_f32) return 0;
    for (int l = 0; l < d->n_layers; l++)
        if (!d->layers[l].has_o) return 0;
    return 1;
}

static vx_error pgemm(vx_dev *d, const vxh_qmat *W, const vxh_pro *p, int M, double *acc, int ld_acc,
                      int n_out, int cls, int rows_logical)
{
    vxh_event e0, e1;
    vx_error e = prof_slot(d, W, M, n_out, cls, rows_logical, &e0, &e1);
    if (e != VX_OK) return e;
    TRY(vxh_gemm_pro(W, M, p, acc, ld_acc, n_out, scale_for(d, W->type), e0, e1, d->stream));
    return VX_OK;
}

/* Prologue forward: each GEMM builds its own input panel slice.
 *   QKV     t = x + acc_x (previous down projection) -> x2, panel attn_norm .* t
 *   RoPE    q|k|v = RoPE(acc_qkv / rms(t)), new k/v rows into the cache
 *   attn    partials per chunk, combined
 *   O       panel att -> acc_y
 *   gate/up t = x2 + acc_y -> x, panel ffn_norm .* t -> acc_gu
 *   down    panel SwiGLU(acc_gu / rms(t)) -> acc_x
 * 7 launches per layer; for one or two rows the attention's first launch
 * does the RoPE and the output projection the combine, 5 launches.
 * An accumulator is cleared by a later launch that no longer races with its
 * readers: acc_gu by the next QKV (or the output GEMM), acc_x by gate/up,
 * acc_y by down; acc_qkv by RoPE (or the output projection). */
static vx_error forward_pro(vx_model *m, int M, int n_past, int logits_mode)
{
    vx_dev *d = vx_dev_of(m);
    const int dd = d->d, kvd = d->kvd, V = d->V, L = d->n_layers, n_ctx = d->n_ctx_alloc;
    const int B = VX_MAX_BATCH;
    vxh_stream s = d->stream;
    vx_error e;
#define SS(l, j) (d->ss + ((size_t)(l) * 2 + (j)) * B)
    if (d->acc_dirty && (e = zero_acc(d)) != VX_OK) return e;
    d->acc_dirty = 1;
    /* one- and two-row forwards (draft decode): the output projection
     * combines the attention partials itself.  These and the verify batches
     * that take the q|k|v attention give every layer its own accumulators
     * (acc_dec), cleared here with the rest, so no launch of the forward
     * clears one */
    const int attn_in_o = M <= VXH_PRO_ATTN_MAX_ROWS && d->hd % 4 == 0;
    const int qkv_fast = M <= VXH_ATTN_QKV_FAST_ROWS && (d->hd == 64 || d->hd == 128);
    const int dec = attn_in_o || (qkv_fast && !d->opt.kv_half);
    /* the sums of squares and acc_x's rows (the previous prologue forward's
     * output GEMM may have left its last down projection in acc_x_rows of
     * them) -- and, decoding, all of acc_x and rows 0..M-1 of every layer's
     * accumulators -- are cleared by the embedding gather's launch */
    const long n_clr = dec ? (long)(L + 1) * 2 * B + (long)B * dd + (long)M * L * d->ld_dec_rec
                           : (long)(L + 1) * 2 * B + (long)(M > d->acc_x_rows ? M : d->acc_x_rows) * dd;
    if (d->has_embd)
        TRY(vxh_qmat_gather_rows_clear(&d->embd, d->tok, M, vx_get_synthetic_weight_scale(), d->x, dd, d->ss,
                                       n_clr, s));
    else {
        TRY(vxh_fill_f32(d->x, 0.0f, (size_t)M * dd, s));
        TRY(vxh_fill_f32((float *)d->ss, 0.0f, 2 * (size_t)n_clr, s));
    }
    d->acc_x_rows = 0;

    /* accumulators of layer l: q|k|v, attention output (y), gate/up, down (x) */
    const int ld_dec = L * d->ld_dec_rec;
#define ACC_Q(l) (dec ? d->acc_dec + (size_t)(l) * d->ld_dec_rec : d->acc_qkv)
#define ACC_Y(l) (dec ? d->acc_dec + (size_t)(l) * d->ld_dec_rec + d->ld_qkv : d->acc_y)
#define ACC_G(l) (dec ? d->acc_dec + (size_t)(l) * d->ld_dec_rec + d->ld_qkv + dd : d->acc_gu)
#define ACC_X(l) (dec ? d->acc_dec + (size_t)(l) * d->ld_dec_rec + d->ld_qkv + dd + d->ld_gu : d->acc_x)
    const int ldq = dec ? ld_dec : d->ld_qkv, ldy = dec ? ld_dec : dd, ldg = dec ? ld_dec : d->ld_gu,
              ldx = dec ? ld_dec : dd;
    vxh_pro p;
    for (int l = 0; l < L; l++) {
        vx_dev_layer *Ld = &d->layers[l];
        const int kvh = d->opt.kv_half;
        const size_t kv_off = (size_t)l * n_ctx * kvd;
        float *kc = m->k_cache + kv_off, *vc = m->v_cache + kv_off;
        uint16_t *kh = (uint16_t *)m->k_cache + kv_off, *vh = (uint16_t *)m->v_cache + kv_off;
        memset(&p, 0, sizeof(p));
        p.kind = VXH_PRO_RESID;
        p.x = d->x; p.ldx = dd;
        if (dec && l > 0) { p.src = ACC_X(l - 1); p.ld_src = ldx; }
        else { p.src = d->acc_x; p.ld_src = dd; }
        p.w = Ld->attn_norm;
        p.x_out = d->x2; p.ld_xout = dd;
        p.ss = SS(l, 0);
        if (!dec) { p.clear = d->acc_gu; p.n_clear = (size_t)M * d->ld_gu; }
        if ((e = pgemm(d, &Ld->wqkv, &p, M, ACC_Q(l), ldq, dd + 2 * kvd, VX_PROF_QKV, dd + 2 * kvd)))
            return e;
        memset(&p, 0, sizeof(p));
        if (attn_in_o) {
            /* partials of the attention, combined by the output projection */
            int n_chunks = 0;
            if (kvh)
                TRY(vxh_attention_parts_qkv_f16(ACC_Q(l), ldq, SS(l, 0), dd, Ld->bq, Ld->bk, Ld->bv,
                                                d->rope_cos, d->rope_sin, d->n_pos, M, n_past, n_ctx,
                                                d->n_heads, d->n_kv, d->hd, d->opt.attn_cap, kh, vh, &d->ws,
                                                &n_chunks, s));
            else
                TRY(vxh_attention_parts_qkv(ACC_Q(l), ldq, SS(l, 0), dd, Ld->bq, Ld->bk, Ld->bv,
                                            d->rope_cos, d->rope_sin, d->n_pos, M, n_past, n_ctx, d->n_heads,
                                            d->n_kv, d->hd, d->opt.attn_cap, kc, vc, &d->ws, &n_chunks, s));
            p.kind = VXH_PRO_ATTN;
            p.part = d->ws.part; p.n_chunks = n_chunks;
            p.n_heads = d->n_heads; p.n_kv_heads = d->n_kv; p.head_dim = d->hd;
        } else if (qkv_fast) {
            /* RoPE and the new k/v rows inside the attention's first launch */
            if (kvh)
                TRY(vxh_attention_qkv_f16(d->acc_qkv, d->ld_qkv, SS(l, 0), dd, Ld->bq, Ld->bk, Ld->bv,
                                          d->rope_cos, d->rope_sin, d->n_pos, M, n_past, n_ctx, d->n_heads,
                                          d->n_kv, d->hd, d->opt.attn_cap, kh, vh, d->att, dd, &d->ws, s));
            else if (dec)
                TRY(vxh_attention_qkv_keep(ACC_Q(l), ldq, SS(l, 0), dd, Ld->bq, Ld->bk, Ld->bv,
                                           d->rope_cos, d->rope_sin, d->n_pos, M, n_past, n_ctx, d->n_heads,
                                           d->n_kv, d->hd, d->opt.attn_cap, kc, vc, d->att, dd, &d->ws, s));
            else
                TRY(vxh_attention_qkv(d->acc_qkv, d->ld_qkv, SS(l, 0), dd, Ld->bq, Ld->bk, Ld->bv,
                                      d->rope_cos, d->rope_sin, d->n_pos, M, n_past, n_ctx, d->n_heads,
                                      d->n_kv, d->hd, d->opt.attn_cap, kc, vc, d->att, dd, &d->ws, s));
            p.kind = VXH_PRO_ROWS;
            p.x = d->att; p.ldx = dd;
        } else {
            if (kvh) return VX_ERR_UNSUPPORTED;   /* excluded by vx_model_set_options */
            TRY(vxh_rope_kv_norm(d->acc_qkv, d->ld_qkv, M, n_past, n_ctx, d->n_heads, d->n_kv, d->hd,
                                 Ld->bq, Ld->bk, Ld->bv, d->rope_cos, d->rope_sin, d->n_pos, SS(l, 0), dd,
                                 d->q, kc, vc, s));
            TRY(vxh_attention(d->q, M, n_past, n_ctx, d->n_heads, d->n_kv, d->hd, d->opt.attn_cap, kc, vc,
                              d->att, dd, &d->ws, s));
            p.kind = VXH_PRO_ROWS;
            p.x = d->att; p.ldx = dd;
        }
        if ((e = pgemm(d, &Ld->wo, &p, M, ACC_Y(l), ldy, dd, VX_PROF_O, dd))) return e;
        memset(&p, 0, sizeof(p));
        p.kind = VXH_PRO_RESID;
        p.x = d->x2; p.ldx = dd;
        p.src = ACC_Y(l); p.ld_src = ldy;
        p.w = Ld->ffn_norm;
        p.x_out = d->x; p.ld_xout = dd;
        p.ss = SS(l, 1);
        if (!dec) { p.clear = d->acc_x; p.n_clear = (size_t)M * dd; }
        if ((e = pgemm(d, &Ld->wgu, &p, M, ACC_G(l), ldg, d->ld_gu, VX_PROF_GATEUP, 2 * d->F)))
            return e;
        if (M > VXH_PRO_ATTN_MAX_ROWS) {
            /* verify batches: the SwiGLU panel once per forward (each of the
             * down GEMM's tile groups would rebuild its slice from the fp64
             * gate/up sums); the panel launch clears acc_gu and acc_y */
            vxh_event pe0, pe1;
            if ((e = prof_slot_panel(d, M, d->F, &pe0, &pe1))) return e;
            TRY(vxh_swiglu_panel_norm_timed(ACC_G(l), ldg, M, d->F, d->opt.ffn_gate_threshold, SS(l, 1), dd,
                                            dec ? NULL : d->acc_y, dec ? 0 : (size_t)M * dd, &d->pan_f, pe0, pe1,
                                            s));
            if ((e = gemm(d, &Ld->wd, &d->pan_f, M, ACC_X(l), ldx, dd, VX_PROF_DOWN, dd))) return e;
        } else {
            memset(&p, 0, sizeof(p));
            p.kind = VXH_PRO_SWIGLU;
            p.src = ACC_G(l); p.ld_src = ldg;
            p.ss_in = SS(l, 1); p.ss_K = dd;
            p.thr = d->opt.ffn_gate_threshold;
            if (!dec) { p.clear = d->acc_y; p.n_clear = (size_t)M * dd; }
            if ((e = pgemm(d, &Ld->wd, &p, M, ACC_X(l), ldx, dd, VX_PROF_DOWN, dd))) return e;
        }
    }
    int gu_cleared = 0;
    if (logits_mode != VX_LOGITS_NONE && d->has_out) {
        /* the output GEMM adds the last down projection to the residual in
         * its prologue (t = x + acc_x, as the residual kinds do) and leaves
         * acc_x to the next forward's clear */
        const int rows = logits_mode == VX_LOGITS_LAST ? 1 : M;
        const int r0 = logits_mode == VX_LOGITS_LAST ? M - 1 : 0;
        const int orows = d->out_rows;
        if (orows < V) TRY(vxh_fill_rows(d->logits, V, rows, orows, V - orows, -1e30f, s));
        {
            memset(&p, 0, sizeof(p));
            p.kind = VXH_PRO_RESID;
            p.x = d->x + (size_t)r0 * dd; p.ldx = dd;
            p.src = L > 0 ? ACC_X(L - 1) + (size_t)r0 * ldx : d->acc_x + (size_t)r0 * dd;
            p.ld_src = L > 0 ? ldx : dd;
            p.w = d->has_out_norm ? d->out_norm : NULL;
            p.ss = d->has_out_norm ? SS(L, 0) : NULL;
            if (!dec) { p.clear = d->acc_gu; p.n_clear = (size_t)M * d->ld_gu; }
            if ((e = pgemm(d, &d->out, &p, rows, d->acc_lg, d->ld_lg, orows, VX_PROF_OUTPUT, orows)))
                return e;
            gu_cleared = 1;
            if (d->has_out_norm)
                TRY(vxh_acc_store_norm(d->acc_lg, d->ld_lg, rows, orows, d->logits, V, SS(L, 0), dd, s));
            else
                TRY(vxh_acc_store(d->acc_lg, d->ld_lg, rows, orows, d->logits, V, NULL, 0, s));
        }
    } else {
        /* x += last down projection (clears its accumulator) */
        if (L > 0) TRY(vxh_acc_store(ACC_X(L - 1), ldx, M, dd, d->x, dd, d->x, dd, s));
        if (logits_mode != VX_LOGITS_NONE) {   /* no output matrix: every logit -1e30 */
            const int rows = logits_mode == VX_LOGITS_LAST ? 1 : M;
            TRY(vxh_fill_rows(d->logits, V, rows, 0, V, -1e30f, s));
        }
    }
    if (!dec && !gu_cleared && L > 0) TRY(vxh_fill_f32((float *)d->acc_gu, 0.0f, 2 * (size_t)M * d->ld_gu, s));
#undef SS
#undef ACC_Q
#undef ACC_Y
#undef ACC_G
#undef ACC_X
    /* rows of acc_x the output GEMM read and left (decoding reads the last
     * layer's own accumulator instead) */
    d->acc_x_rows = (gu_cleared && !dec) ? M : 0;
    d->acc_dirty = 0;
    return VX_OK;
}

/* One batched forward.  Every GEMM adds into an fp64 accumulator that the
 * next kernel consumes (and clears): q|k|v -> RoPE/KV write, attention
 * output projection and down projection -> the residual + RMSNorm panel of
 * the next block, gate/up -> the SwiGLU panel, logits -> a store. */
vx_error vx_dev_forward_ids(vx_model *m, const int *ids, int M, int n_past, int logits_mode)
{
    vx_dev *d = vx_dev_of(m);
    if (!d || !ids) return VX_ERR_PARAM;
    int *own = d->tok;
    d->tok = (int *)ids;   /* read by the embedding gather only */
    vx_error e = vx_dev_forward(m, M, n_past, logits_mode);
    d->tok = own;
    return e;
}

vx_error vx_dev_forward(vx_model *m, int M, int n_past, int logits_mode)
{
    vx_dev *d = vx_dev_of(m);
    if (M < 1 || M > VX_MAX_BATCH) return VX_ERR_PARAM;
    if (!m->k_cache || !m->v_cache) {
        /* nothing to attend to or store into: fail before any launch */
        vx_set_error("forward without a KV cache (dropped by an option change?)");
        return VX_ERR_PARAM;
    }
    if (pro_ok(d, M)) return forward_pro(m, M, n_past, logits_mode);
    if (d->opt.kv_half) return VX_ERR_UNSUPPORTED;   /* fp16 caches: prologue path only */
    const int dd = d->d, kvd = d->kvd, F = d->F, V = d->V, n_ctx = d->n_ctx_alloc;
    const int avx2 = d->opt.q4_kernel == VX_Q4_AVX2_LANES;
    const float thr = d->opt.ffn_gate_threshold;
    vxh_stream s = d->stream;
    vx_error e;

    if ((d->acc_dirty || d->acc_x_rows) && (e = zero_acc(d)) != VX_OK) return e;
    d->acc_dirty = 1;
    if (d->has_embd) TRY(vxh_qmat_gather_rows(&d->embd, d->tok, M, vx_get_synthetic_weight_scale(), d->x, dd, s));
    else TRY(vxh_fill_f32(d->x, 0.0f, (size_t)M * dd, s));

    for (int l = 0; l < d->n_layers; l++) {
        vx_dev_layer *Ld = &d->layers[l];
        float *kc = m->k_cache + (size_t)l * n_ctx * kvd;
        float *vc = m->v_cache + (size_t)l * n_ctx * kvd;
        /* x += previous down projection; attention RMSNorm; QKV tail = x[0..3] */
        TRY(vxh_resid_rmsnorm_panel(d->x, dd, d->acc_x, dd, M, dd, Ld->attn_norm, avx2, 1, &d->pan_d,
                                    (avx2 && Ld->has_o) ? d->xn : NULL, dd, s));
        if ((e = gemm(d, &Ld->wqkv, &d->pan_d, M, d->acc_qkv, d->ld_qkv, dd + 2 * kvd, VX_PROF_QKV,
                      dd + 2 * kvd)))
            return e;
        TRY(vxh_rope_kv(d->acc_qkv, d->ld_qkv, M, n_past, n_ctx, d->n_heads, d->n_kv, d->hd, Ld->bq,
                        Ld->bk, Ld->bv, d->rope_cos, d->rope_sin, d->n_pos, d->q, kc, vc, s));
        TRY(vxh_attention(d->q, M, n_past, n_ctx, d->n_heads, d->n_kv, d->hd, d->opt.attn_cap, kc, vc,
                          d->att, dd, &d->ws, s));
        if (Ld->has_o) {
            /* attn_o's x86-build tail is the normed x (src/model.c:426, :544) */
            TRY(vxh_prep_panel(&d->pan_d, d->att, dd, M, dd, avx2, d->xn, dd, s));
            if ((e = gemm(d, &Ld->wo, &d->pan_d, M, d->acc_x, dd, dd, VX_PROF_O, dd))) return e;
        } else {
            TRY(vxh_add_rows(d->x, dd, d->att, dd, M, dd, s));
        }
        /* x += attention output; FFN RMSNorm; gate/up tail = x[0..3] */
        TRY(vxh_resid_rmsnorm_panel(d->x, dd, d->acc_x, dd, M, dd, Ld->ffn_norm, avx2, 1, &d->pan_d,
                                    NULL, 0, s));
        /* the logits' x86-build tail reads the last layer's post-attention
         * residual (src/model.c:426, :547) */
        if (avx2 && l == d->n_layers - 1) TRY(vxh_copy_rows(d->xtail, 4, d->x, dd, M, 4, s));
        if ((e = gemm(d, &Ld->wgu, &d->pan_d, M, d->acc_gu, d->ld_gu, d->ld_gu, VX_PROF_GATEUP, 2 * F)))
            return e;
        TRY(vxh_swiglu_panel(d->acc_gu, d->ld_gu, M, F, thr, avx2, &d->pan_f, NULL, 0, s));
        if ((e = gemm(d, &Ld->wd, &d->pan_f, M, d->acc_x, dd, dd, VX_PROF_DOWN, dd))) return e;
    }
    /* x += last down projection (clears the residual accumulator) */
    TRY(vxh_acc_store(d->acc_x, dd, M, dd, d->x, dd, d->x, dd, s));

    if (logits_mode != VX_LOGITS_NONE) {
        int rows = logits_mode == VX_LOGITS_LAST ? 1 : M;
        int r0 = logits_mode == VX_LOGITS_LAST ? M - 1 : 0;
        const float *src = d->x + (size_t)r0 * dd;
        const float *tail = d->xtail + (size_t)r0 * 4;
        if (d->has_out_norm)
            TRY(vxh_rmsnorm_panel(src, dd, rows, dd, d->out_norm, avx2, tail, 4, &d->pan_d, NULL, 0, s));
        else
            TRY(vxh_prep_panel(&d->pan_d, src, dd, rows, dd, avx2, tail, 4, s));
        int orows = d->has_out ? d->out_rows : 0;
        if (orows < V) TRY(vxh_fill_rows(d->logits, V, rows, orows, V - orows, -1e30f, s));
        if (d->has_out) {
            if ((e = gemm(d, &d->out, &d->pan_d, rows, d->acc_lg, d->ld_lg, orows, VX_PROF_OUTPUT, orows)))
                return e;
            TRY(vxh_acc_store(d->acc_lg, d->ld_lg, rows, orows, d->logits, V, NULL, 0, s));
        }
    }
    d->acc_dirty = 0;
    return VX_OK;
}

/* --------------------------------------------------------------------------- */
/* large-M prompt prefill                                                        */
/* --------------------------------------------------------------------------- */
/* The large-M path covers the exact Q4_0/Q8_0 arithmetic with an fp32 cache;
 * the AVX2-lane mode and the fp16 cache stay on the batched forward. */
static int pf_ok(const vx_dev *d)
{
    return d->opt.prefill_min_rows > 0 && d->opt.q4_kernel == VX_Q4_EXACT && !d->opt.kv_half &&
           !d->has_f32 && d->hd % 4 == 0 && d->hd <= 128;
}

static vx_error pf_alloc(vx_dev *d)
{
    if (d->pf_ready && (d->pf_ws_ctx != d->n_ctx_alloc || d->pf_ws_cap != d->opt.attn_cap)) {
        /* a cache allocated again for another n_ctx, or another cap: the
         * attention workspace is sized for both */
        TRY(vxh_stream_sync(d->stream));
        vxh_workspace_free(&d->pf_ws);
        size_t an = vxh_attention_workspace_floats(VX_PF_ROWS, d->n_ctx_alloc, d->opt.attn_cap, d->n_heads,
                                                   d->n_kv, d->hd);
        TRY(vxh_workspace_alloc(&d->pf_ws, 32, an));
        d->pf_ws_ctx = d->n_ctx_alloc;
        d->pf_ws_cap = d->opt.attn_cap;
    }
    if (d->pf_ready) return VX_OK;
    const size_t R = VX_PF_ROWS;
    TRY(vxh_malloc((void **)&d->pf_tok, sizeof(int) * R));
    TRY(vxh_malloc((void **)&d->pf_x, sizeof(float) * R * d->d));
    TRY(vxh_malloc((void **)&d->pf_xn, sizeof(float) * R * d->d));
    TRY(vxh_malloc((void **)&d->pf_qkv, sizeof(float) * R * d->ld_qkv));
    TRY(vxh_malloc((void **)&d->pf_q, sizeof(float) * R * d->d));
    TRY(vxh_malloc((void **)&d->pf_att, sizeof(float) * R * d->d));
    TRY(vxh_malloc((void **)&d->pf_gu, sizeof(float) * R * d->ld_gu));
    TRY(vxh_malloc((void **)&d->pf_h, sizeof(float) * R * d->F));
    TRY(vxh_malloc((void **)&d->pf_px, vxh_rows_panel_bytes(VX_PF_ROWS, d->F > d->d ? d->F : d->d)));
    size_t an = vxh_attention_workspace_floats(VX_PF_ROWS, d->n_ctx_alloc, d->opt.attn_cap, d->n_heads, d->n_kv,
                                               d->hd);
    TRY(vxh_workspace_alloc(&d->pf_ws, 32, an));
    d->pf_ws_ctx = d->n_ctx_alloc;
    d->pf_ws_cap = d->opt.attn_cap;
    d->pf_ready = 1;
    return VX_OK;
}

/* M <= VX_PF_ROWS prompt rows at positions n_past .. n_past+M-1 (all below
 * n_ctx) as one batch: per layer RMSNorm rows, the large-M GEMMs, RoPE + KV
 * store, causal attention over the cache, SwiGLU (src/model.c:514-594).
 * With last_logits the last row's logits land in d->logits row 0. */
static vx_error forward_prefill(vx_model *m, const int *tokens, int M, int n_past, int last_logits)
{
    vx_dev *d = vx_dev_of(m);
    const int dd = d->d, kvd = d->kvd, n_ctx = d->n_ctx_alloc;
    vxh_stream s = d->stream;
    vx_error e = pf_alloc(d);
    if (e != VX_OK) return e;
    TRY(vxh_upload(d->pf_tok, tokens, sizeof(int) * (size_t)M, s));
    if (d->has_embd) TRY(vxh_qmat_gather_rows(&d->embd, d->pf_tok, M, vx_get_synthetic_weight_scale(), d->pf_x, dd, s));
    else TRY(vxh_fill_f32(d->pf_x, 0.0f, (size_t)M * dd, s));
    for (int l = 0; l < d->n_layers; l++) {
        vx_dev_layer *Ld = &d->layers[l];
        float *kc = m->k_cache + (size_t)l * n_ctx * kvd, *vc = m->v_cache + (size_t)l * n_ctx * kvd;
        TRY(vxh_rmsnorm(d->pf_x, dd, M, dd, Ld->attn_norm, d->pf_xn, dd, s));
        TRY(vxh_rows_panel(d->pf_xn, dd, M, dd, d->pf_px, s));
        TRY(vxh_gemm_rows(&Ld->wqkv, d->pf_px, M, d->pf_qkv, d->ld_qkv, dd + 2 * kvd, NULL, 0,
                          scale_for(d, Ld->wqkv.type), s));
        TRY(vxh_rope_kv_rows(d->pf_qkv, d->ld_qkv, M, n_past, n_ctx, d->n_heads, d->n_kv, d->hd, Ld->bq, Ld->bk,
                             Ld->bv, d->rope_cos, d->rope_sin, d->n_pos, d->pf_q, dd, kc, vc, s));
        TRY(vxh_attention(d->pf_q, M, n_past, n_ctx, d->n_heads, d->n_kv, d->hd, d->opt.attn_cap, kc, vc,
                          d->pf_att, dd, &d->pf_ws, s));
        if (Ld->has_o) {
            TRY(vxh_rows_panel(d->pf_att, dd, M, dd, d->pf_px, s));
            TRY(vxh_gemm_rows(&Ld->wo, d->pf_px, M, d->pf_x, dd, dd, d->pf_x, dd, scale_for(d, Ld->wo.type), s));
        } else
            TRY(vxh_add_rows(d->pf_x, dd, d->pf_att, dd, M, dd, s));
        TRY(vxh_rmsnorm(d->pf_x, dd, M, dd, Ld->ffn_norm, d->pf_xn, dd, s));
        TRY(vxh_rows_panel(d->pf_xn, dd, M, dd, d->pf_px, s));
        TRY(vxh_gemm_rows(&Ld->wgu, d->pf_px, M, d->pf_gu, d->ld_gu, d->ld_gu, NULL, 0,
                          scale_for(d, Ld->wgu.type), s));
        TRY(vxh_swiglu_rows(d->pf_gu, d->ld_gu, M, d->F, d->opt.ffn_gate_threshold, d->pf_h, d->F, s));
        TRY(vxh_rows_panel(d->pf_h, d->F, M, d->F, d->pf_px, s));
        TRY(vxh_gemm_rows(&Ld->wd, d->pf_px, M, d->pf_x, dd, dd, d->pf_x, dd, scale_for(d, Ld->wd.type), s));
    }
    if (!last_logits) return VX_OK;
    /* the last row's logits through the decode GEMM (src/model.c:598-615) */
    if ((d->acc_dirty || d->acc_x_rows) && (e = zero_acc(d)) != VX_OK) return e;
    const float *src = d->pf_x + (size_t)(M - 1) * dd;
    const int V = d->V, orows = d->has_out ? d->out_rows : 0;
    if (orows < V) TRY(vxh_fill_rows(d->logits, V, 1, orows, V - orows, -1e30f, s));
    if (d->has_out) {
        if (d->has_out_norm)
            TRY(vxh_rmsnorm_panel(src, dd, 1, dd, d->out_norm, 0, NULL, 4, &d->pan_d, NULL, 0, s));
        else
            TRY(vxh_prep_panel(&d->pan_d, src, dd, 1, dd, 0, NULL, 4, s));
        d->acc_dirty = 1;
        if ((e = gemm(d, &d->out, &d->pan_d, 1, d->acc_lg, d->ld_lg, orows, VX_PROF_OUTPUT, orows)) != VX_OK)
            return e;
        TRY(vxh_acc_store(d->acc_lg, d->ld_lg, 1, orows, d->logits, V, NULL, 0, s));
        d->acc_dirty = 0;
    }
    return VX_OK;
}

/* Runs n host tokens from cache_len on, with the reference's position clamp
 * (src/model.c:279-286): positions that fit run in batches of up to 16,
 * overflowing tokens one at a time on the last slot. */
vx_error vx_dev_run_tokens(vx_model *m, const int *tokens, int n, int logits_mode, float *logits_host)
{
    vx_dev *d = vx_dev_of(m);
    vx_error e = vx_dev_ensure_kv(m);
    if (e != VX_OK) return e;
    if (g_level != VX_COMPUTE_EXACT) {
        vx_set_error("compute levels other than VX_COMPUTE_EXACT are not supported");
        return VX_ERR_UNSUPPORTED;
    }
    double t0 = g_timing ? vx_now_ms() : 0.0;
    const int n_ctx = d->n_ctx_alloc, V = d->V;
    int i = 0;
    while (i < n) {
        int c = m->cache_len;
        if (c < 0) c = 0;
        /* long prompts: chunks of up to VX_PF_ROWS rows as one large-M batch */
        if (logits_mode != VX_LOGITS_ALL && pf_ok(d) && n - i >= d->opt.prefill_min_rows && c < n_ctx) {
            int P = n - i;
            if (P > VX_PF_ROWS) P = VX_PF_ROWS;
            if (P > n_ctx - c) P = n_ctx - c;
            if (P >= d->opt.prefill_min_rows) {
                const int last = i + P == n && logits_mode == VX_LOGITS_LAST;
                if ((e = forward_prefill(m, tokens + i, P, c, last)) != VX_OK) return e;
                if (last) TRY(vxh_download(logits_host, d->logits, sizeof(float) * (size_t)V, d->stream));
                m->cache_len = c + P;
                i += P;
                continue;
            }
        }
        int M, next_len;
        if (c < n_ctx) {
            M = n - i;
            if (M > VX_MAX_BATCH) M = VX_MAX_BATCH;
            if (M > n_ctx - c) M = n_ctx - c;
            next_len = c + M;
        } else {
            if (c >= d->n_pos) {
                vx_set_error("cache_len %d is past the RoPE table (%d positions)", c, d->n_pos);
                return VX_ERR_PARAM;
            }
            M = 1;
            next_len = n_ctx;
        }
        int last = i + M == n;
        int mode = VX_LOGITS_NONE;
        if (logits_mode == VX_LOGITS_ALL) mode = VX_LOGITS_ALL;
        else if (logits_mode == VX_LOGITS_LAST && last) mode = VX_LOGITS_LAST;
        TRY(vxh_upload(d->tok, tokens + i, sizeof(int) * (size_t)M, d->stream));
        if ((e = vx_dev_forward(m, M, c, mode)) != VX_OK) return e;
        if (mode == VX_LOGITS_ALL)
            TRY(vxh_download(logits_host + (size_t)i * V, d->logits, sizeof(float) * (size_t)M * V, d->stream));
        else if (mode == VX_LOGITS_LAST)
            TRY(vxh_download(logits_host, d->logits, sizeof(float) * (size_t)V, d->stream));
        m->cache_len = next_len;
        i += M;
    }
    TRY(vxh_stream_sync(d->stream));
    if (g_timing) {
        g_timing_ms += vx_now_ms() - t0;
        g_timing_tokens += n;
    }
    return VX_OK;
}

vx_error vx_model_forward(vx_model *m, const int *tokens, int n_tokens, float *logits)
{
    if (!m || !tokens || !logits) return VX_ERR_PARAM;
    if (!m->dev) return VX_ERR_NOMODEL;
    if (n_tokens <= 0) return VX_OK;
    return vx_dev_run_tokens(m, tokens, n_tokens, VX_LOGITS_LAST, logits);
}

vx_error vx_model_verify(vx_model *m, const int *tokens, int n_tokens, float *logits_all)
{
    if (!m || !tokens || !logits_all) return VX_ERR_PARAM;
    if (!m->dev) return VX_ERR_NOMODEL;
    if (n_tokens <= 0) return VX_OK;
    return vx_dev_run_tokens(m, tokens, n_tokens, VX_LOGITS_ALL, logits_all);
}

/* --------------------------------------------------------------------------- */
/* read-back                                                                     */
/* --------------------------------------------------------------------------- */
vx_error vx_model_read_tensor(const vx_model *m, const char *name, void *dst, size_t bytes)
{
    vx_dev *d = vx_dev_of(m);
    if (!d || !name || !dst) return VX_ERR_PARAM;
    const vxh_qmat *q = NULL;
    int rows = 0, group = 0, stride = 0, off = 0;
    int l = -1;
    char role[48] = {0};
    if (strcmp(name, "token_embd.weight") == 0 && d->has_embd) {
        q = &d->embd; rows = d->embd.n_rows; group = rows;
        rows = m->config.n_vocab;
        group = rows;
    } else if (strcmp(name, "output.weight") == 0 && d->has_out) {
        q = &d->out; rows = d->out_rows; group = rows;
    } else if (sscanf(name, "blk.%d.%47[^.].weight", &l, role) == 2 && l >= 0 && l < d->n_layers) {
        vx_dev_layer *Ld = &d->layers[l];
        if (!strcmp(role, "attn_q")) { q = &Ld->wqkv; rows = d->d; off = 0; }
        else if (!strcmp(role, "attn_k")) { q = &Ld->wqkv; rows = d->kvd; off = d->d; }
        else if (!strcmp(role, "attn_v")) { q = &Ld->wqkv; rows = d->kvd; off = d->d + d->kvd; }
        else if (!strcmp(role, "attn_output") && Ld->has_o) { q = &Ld->wo; rows = d->d; }
        else if (!strcmp(role, "ffn_gate")) { q = &Ld->wgu; rows = d->F; group = 16; stride = 32; off = 0; }
        else if (!strcmp(role, "ffn_up")) { q = &Ld->wgu; rows = d->F; group = 16; stride = 32; off = 16; }
        else if (!strcmp(role, "ffn_down")) { q = &Ld->wd; rows = d->d; }
        if (q && !group) group = rows;
    }
    if (!q) { vx_set_error("no device matrix named %s", name); return VX_ERR_PARAM; }
    size_t need = q->type == VX_TYPE_F32 ? (size_t)rows * q->n_cols * sizeof(float)
                                         : (size_t)rows * (q->n_cols / 32) * (q->type == VX_TYPE_Q4_0 ? 18 : 34);
    if (bytes < need) { vx_set_error("%s needs %zu bytes", name, need); return VX_ERR_PARAM; }
    TRY(vxh_qmat_get_rows(q, dst, rows, group, stride, off, d->stream));
    return VX_OK;
}

vx_error vx_model_read_kv(const vx_model *m, int layer, int n, float *k, float *v)
{
    vx_dev *d = vx_dev_of(m);
    if (!d || !m->k_cache || layer < 0 || layer >= d->n_layers || n < 0 || n > d->n_ctx_alloc)
        return VX_ERR_PARAM;
    size_t off = (size_t)layer * d->n_ctx_alloc * d->kvd;
    size_t cnt = (size_t)n * d->kvd;
    if (d->opt.kv_half) {
        /* halves widened exactly */
        uint16_t *h = (uint16_t *)malloc(2 * (cnt ? cnt : 1));
        if (!h) return VX_ERR_MEMORY;
        vx_error e = VX_OK;
        for (int w = 0; w < 2 && e == VX_OK; w++) {
            float *dst = w ? v : k;
            if (!dst) continue;
            const uint16_t *src = (const uint16_t *)(w ? m->v_cache : m->k_cache) + off;
            if (vxh_download(h, src, 2 * cnt, d->stream)) e = vx_from_vxh(-1);
            for (size_t i = 0; e == VX_OK && i < cnt; i++) dst[i] = vx_fp16_to_fp32(h[i]);
        }
        free(h);
        return e;
    }
    size_t bytes = sizeof(float) * cnt;
    if (k) TRY(vxh_download(k, m->k_cache + off, bytes, d->stream));
    if (v) TRY(vxh_download(v, m->v_cache + off, bytes, d->stream));
    return VX_OK;
}
