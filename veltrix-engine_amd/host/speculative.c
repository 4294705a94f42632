/*
 * speculative.c -- speculative decoding with a GPU-batched verify step
 * (reference include/speculative.h:8-15, src/speculative.c:109-300).
 *
 * State between rounds: committed tokens c[0..n); the target's KV cache holds
 * c[0..n-1) and t0 = c[n-1] is not yet in it.  One round:
 *
 *   draft:  the draft model catches up on the committed tokens it has not
 *           seen (one batch of 1-2 rows), then drafts d_0..d_{k-1}, each from
 *           the previous logits with the GPU sampler (nucleus of softmax(l/T)
 *           at a seeded uniform; argmax when T <= 0);
 *   verify: ONE target forward over [t0, d_0 .. d_{k-1}] at positions
 *           n-1 .. n-1+k gives logits L_0..L_k; the GPU decision kernel
 *           accepts d_j while u_j < min(1, p_j(d_j)/max(q_j(d_j), 1e-10))
 *           (greedy: while d_j == argmax L_j), then emits either the residual
 *           resample max(0, p_j - q_j) at the first rejection or a bonus token
 *           from p_k when every draft was accepted;
 *   commit: the accepted drafts and the emitted token are appended; both KV
 *           caches are rolled back to their valid prefix by cache_len, as
 *           vx_model_kv_truncate does (src/model.c:384-389).
 *
 * Deliberate differences from the reference loop (whose buffers overflow and
 * which compares raw logits, src/speculative.c:119,160,167,205): softmax
 * probabilities on both sides, the draft keeps its KV cache between rounds,
 * and the uniforms come from a seeded counter stream rather than rand().
 */
#include <stdlib.h>
#include <string.h>

#include "speculative.h"
#include "vx_host.h"

struct vx_speculative_state {
    vx_model *draft, *target;
    int k;
    float temperature, top_p;
    uint64_t seed;
    int Vd, Vt;
    float *D;           /* device [k][Vd] draft logits                 */
    float *nuc;         /* device [k][8] nucleus descriptors           */
    float *u_draft;     /* device [k]                                  */
    float *u_verify;    /* device [k+1]                                */
    int *dtok;          /* device [k+1]: t0, d_0 .. d_{k-1}            */
    int *out_dev;       /* device [k+3]                                */
    vxh_vocab_ws ws_d, ws_t; /* many-workgroup sampling workspaces, one per
                                model stream (draft draws, verify decision) */
    int *out_host;
    /* page-locked staging of a round's uploads (vxh_upload_async): the
     * draft's catch-up tokens, t0, the draft and verify uniforms.  Every
     * round ends with a synchronous download, so the copies of one round
     * have run before the next round writes here. */
    void *stage;
    int *st_tok;        /* [VX_MAX_BATCH] */
    int *st_t0;         /* [1]            */
    float *st_ud;       /* [k]            */
    float *st_uv;       /* [k+1]          */
    vx_speculative_stats st;
    int *tr_drafts, *tr_emitted, *tr_accepted, tr_max;
    /* state left by vx_speculative_prefill */
    int *committed;
    int cap;
    int n_prompt;         /* 0 = not prefilled */
    unsigned gen_t, gen_d;   /* the models' cache generations at prefill */
};

float vx_uniform(uint64_t seed, uint64_t stream, uint64_t index)
{
    uint64_t r = vx_splitmix64(seed ^ vx_splitmix64((stream << 48) ^ index));
    return (float)(r >> 40) * (1.0f / 16777216.0f);
}

vx_speculative_state *vx_speculative_create(vx_model *draft, vx_model *target, int max_draft_tokens)
{
    if (!draft || !target || !draft->dev || !target->dev || max_draft_tokens < 1 ||
        max_draft_tokens + 1 > VX_MAX_BATCH)
        return NULL;
    vx_speculative_state *s = (vx_speculative_state *)calloc(1, sizeof(*s));
    if (!s) return NULL;
    s->draft = draft;
    s->target = target;
    s->k = max_draft_tokens;
    s->temperature = 0.8f;   /* src/speculative.c:116-117 */
    s->top_p = 0.95f;
    s->seed = 0x5EEDull;
    s->Vd = draft->config.n_vocab;
    s->Vt = target->config.n_vocab;
    int k = s->k;
    int ok = vxh_malloc((void **)&s->D, sizeof(float) * (size_t)k * s->Vd) == VXH_OK &&
             vxh_malloc((void **)&s->nuc, sizeof(float) * 8 * (size_t)k) == VXH_OK &&
             vxh_malloc((void **)&s->u_draft, sizeof(float) * (size_t)k) == VXH_OK &&
             vxh_malloc((void **)&s->u_verify, sizeof(float) * (size_t)(k + 1)) == VXH_OK &&
             vxh_malloc((void **)&s->dtok, sizeof(int) * (size_t)(k + 1)) == VXH_OK &&
             vxh_malloc((void **)&s->out_dev, sizeof(int) * (size_t)(k + 3)) == VXH_OK &&
             vxh_vocab_ws_alloc(&s->ws_d, 1) == VXH_OK && vxh_vocab_ws_alloc(&s->ws_t, k + 1) == VXH_OK &&
             vxh_host_alloc(&s->stage, sizeof(int) * (VX_MAX_BATCH + 1) + sizeof(float) * (size_t)(2 * k + 1)) ==
                 VXH_OK;
    if (ok) {
        s->st_tok = (int *)s->stage;
        s->st_t0 = s->st_tok + VX_MAX_BATCH;
        s->st_ud = (float *)(s->st_t0 + 1);
        s->st_uv = s->st_ud + k;
    }
    s->out_host = (int *)calloc((size_t)(k + 3), sizeof(int));
    if (!ok || !s->out_host) {
        vx_speculative_destroy(s);
        return NULL;
    }
    return s;
}

void vx_speculative_destroy(vx_speculative_state *s)
{
    if (!s) return;
    vxh_free(s->D); vxh_free(s->nuc); vxh_free(s->u_draft); vxh_free(s->u_verify);
    vxh_free(s->dtok); vxh_free(s->out_dev);
    vxh_vocab_ws_free(&s->ws_d);
    vxh_vocab_ws_free(&s->ws_t);
    vxh_host_free(s->stage);
    free(s->out_host);
    free(s->committed);
    free(s);
}

void vx_speculative_set_temp(vx_speculative_state *s, float temp, float top_p)
{
    if (s) {
        s->temperature = temp;
        s->top_p = top_p;
    }
}

void vx_speculative_set_seed(vx_speculative_state *s, uint64_t seed)
{
    if (s) s->seed = seed;
}

void vx_speculative_get_stats(const vx_speculative_state *s, vx_speculative_stats *st)
{
    if (s && st) *st = s->st;
}

void vx_speculative_set_trace(vx_speculative_state *s, int *drafts, int *emitted, int *accepted,
                              int max_rounds)
{
    if (!s) return;
    s->tr_drafts = drafts;
    s->tr_emitted = emitted;
    s->tr_accepted = accepted;
    s->tr_max = max_rounds;
}

#define CHK(expr)                                                         \
    do {                                                                  \
        if ((expr) != VXH_OK) { vx_from_vxh(-1); goto done; }             \
    } while (0)
#define CHKE(expr)                                                        \
    do {                                                                  \
        if ((expr) != VX_OK) goto done;                                   \
    } while (0)

static int ensure_cap(vx_speculative_state *s, int need)
{
    if (s->cap >= need) return 1;
    int *p = (int *)realloc(s->committed, sizeof(int) * (size_t)need);
    if (!p) return 0;
    s->committed = p;
    s->cap = need;
    return 1;
}

int vx_speculative_prefill(vx_speculative_state *s, const int *prompt, int prompt_len)
{
    if (!s || !prompt || prompt_len < 1) return 0;
    vx_model *tm = s->target, *dm = s->draft;
    s->n_prompt = 0;
    if (!ensure_cap(s, prompt_len + s->k + 2)) return 0;
    memcpy(s->committed, prompt, sizeof(int) * (size_t)prompt_len);
    double t0 = vx_now_ms();
    if (vx_dev_ensure_kv(tm) != VX_OK || vx_dev_ensure_kv(dm) != VX_OK) return 0;
    tm->cache_len = 0;
    dm->cache_len = 0;
    if (prompt_len > 1) {
        if (vx_dev_run_tokens(tm, s->committed, prompt_len - 1, VX_LOGITS_NONE, NULL) != VX_OK) return 0;
        if (vx_dev_run_tokens(dm, s->committed, prompt_len - 1, VX_LOGITS_NONE, NULL) != VX_OK) return 0;
    }
    s->st.prefill_ms = vx_now_ms() - t0;
    s->gen_t = vx_dev_of(tm)->kv_gen;
    s->gen_d = vx_dev_of(dm)->kv_gen;
    s->n_prompt = prompt_len;
    return prompt_len;
}

int vx_speculative_decode(vx_speculative_state *s, int *output, int max_tokens)
{
    if (!s || !output || max_tokens < 1 || s->n_prompt < 1) return 0;
    vx_model *tm = s->target, *dm = s->draft;
    vx_dev *td = vx_dev_of(tm), *dd = vx_dev_of(dm);
    if (!tm->k_cache || !dm->k_cache || td->kv_gen != s->gen_t || dd->kv_gen != s->gen_d) {
        /* an option change dropped a cache after prefill: its rows are gone */
        vx_set_error("a model's KV cache changed since vx_speculative_prefill; prefill again");
        return 0;
    }
    const int k = s->k, Vd = s->Vd, Vt = s->Vt;
    const float T = s->temperature;
    int generated = 0;
    double prefill_ms = s->st.prefill_ms;
    memset(&s->st, 0, sizeof(s->st));
    s->st.prefill_ms = prefill_ms;
    if (!ensure_cap(s, s->n_prompt + max_tokens + k + 2)) return 0;
    int *committed = s->committed;
    int n = s->n_prompt;
    /* restart from the prefilled state: both caches hold committed[0..n-1) */
    tm->cache_len = n - 1;
    dm->cache_len = n - 1;
    int draft_len = n - 1;   /* committed tokens held in the draft's KV cache */
    const int tctx = td->n_ctx_alloc, dctx = dd->n_ctx_alloc;
    /* each draft forward writes its logits row straight into its slot of D
     * (which the decision reads), so the sampler copies nothing; the draft's
     * own buffer is put back below and on every exit */
    float *const dlogits = dd->logits;

    for (int round = 0; generated < max_tokens; round++) {
        /* drafts this round: the round emits up to kk+1 tokens, and positions
         * n-1 .. n-1+kk must fit the target's cache.  The loop is bounded by
         * the target's context only (src/speculative.c:244, :257); once the
         * draft's cache is full the rounds are target-only (kk = 0: the
         * target's own draw at position n-1) */
        int kk = k;
        if (kk > max_tokens - generated - 1) kk = max_tokens - generated - 1;
        if (kk > tctx - n) kk = tctx - n;
        if (kk > dctx - n) kk = dctx - n;
        if (n - 1 >= tctx) break;
        if (kk < 0) kk = 0;
        double ta = vx_now_ms();
        int t_last = committed[n - 1];
        if (kk > 0) {
            /* catch-up batch: committed[draft_len .. n) */
            int pend = n - draft_len;
            if (pend < 1 || pend > VX_MAX_BATCH) goto done;
            memcpy(s->st_tok, committed + draft_len, sizeof(int) * (size_t)pend);
            for (int i = 0; i < kk; i++) s->st_ud[i] = vx_uniform(s->seed, 1, (uint64_t)round * k + i);
            CHK(vxh_upload_async(dd->tok, s->st_tok, sizeof(int) * (size_t)pend, dd->stream));
            CHK(vxh_upload_async(s->u_draft, s->st_ud, sizeof(float) * (size_t)kk, dd->stream));
            dd->logits = s->D;
            CHKE(vx_dev_forward(dm, pend, draft_len, VX_LOGITS_LAST));
            draft_len = n;
            for (int i = 0; i < kk; i++) {
                dd->logits = s->D + (size_t)i * Vd;
                if (i > 0) CHKE(vx_dev_forward_ids(dm, s->dtok + i, 1, n + i - 1, VX_LOGITS_LAST));
                CHK(vxh_sample_keep_mc(dd->logits, Vd, T, s->top_p, s->u_draft + i, s->dtok + 1 + i,
                                       s->nuc + 8 * i, dd->logits, &s->ws_d, dd->stream));
            }
            dd->logits = dlogits;
            CHK(vxh_stream_sync(dd->stream));
        }
        double tb = vx_now_ms();
        s->st.draft_ms += tb - ta;

        /* verify: one target forward over [t0, d_0 .. d_{kk-1}] */
        s->st_t0[0] = t_last;
        for (int j = 0; j < kk; j++) s->st_uv[j] = vx_uniform(s->seed, 2, (uint64_t)round * (k + 1) + j);
        /* the resample / bonus draw always uses the stream's slot k */
        s->st_uv[kk] = vx_uniform(s->seed, 2, (uint64_t)round * (k + 1) + k);
        CHK(vxh_upload_async(s->dtok, s->st_t0, sizeof(int), td->stream));
        CHK(vxh_upload_async(s->u_verify, s->st_uv, sizeof(float) * (size_t)(kk + 1), td->stream));
        CHKE(vx_dev_forward_ids(tm, s->dtok, kk + 1, n - 1, VX_LOGITS_ALL));
        CHK(vxh_row_stats_mc(td->logits, Vt, kk + 1, Vt, T, td->stats, &s->ws_t, td->stream));
        CHK(vxh_accept_mc(td->logits, Vt, Vt, td->stats, s->D, Vd, Vd, s->nuc, s->dtok + 1, kk, T,
                          s->u_verify, s->out_dev, &s->ws_t, td->stream));
        CHK(vxh_download(s->out_host, s->out_dev, sizeof(int) * (size_t)(kk + 3), td->stream));
        s->st.verify_ms += vx_now_ms() - tb;

        int n_emit = s->out_host[0], n_acc = s->out_host[1];
        if (n_emit < 1 || n_emit > kk + 1 || n_acc < 0 || n_acc > kk) {
            vx_set_error("verify produced %d tokens / %d accepted", n_emit, n_acc);
            goto done;
        }
        if (s->tr_max > round) {
            if (s->tr_accepted) s->tr_accepted[round] = n_acc;
            if (s->tr_drafts && kk > 0) {
                int tmp[VX_MAX_BATCH + 1];
                CHK(vxh_download(tmp, s->dtok + 1, sizeof(int) * (size_t)kk, td->stream));
                for (int j = 0; j < k; j++) s->tr_drafts[round * k + j] = j < kk ? tmp[j] : -1;
            } else if (s->tr_drafts) {
                for (int j = 0; j < k; j++) s->tr_drafts[round * k + j] = -1;
            }
            if (s->tr_emitted)
                for (int j = 0; j <= k; j++)
                    s->tr_emitted[round * (k + 1) + j] = j < n_emit ? s->out_host[2 + j] : -1;
        }
        int n_old = n;
        for (int j = 0; j < n_emit && generated < max_tokens; j++) {
            output[generated++] = s->out_host[2 + j];
            committed[n++] = s->out_host[2 + j];
        }
        s->st.rounds++;
        s->st.drafted += kk;
        s->st.accepted += n_acc;
        s->st.emitted = generated;
        /* roll back to the valid prefixes: the target holds t0 and the
         * accepted drafts, the draft holds t0 and d_0 .. d_{kk-2} */
        tm->cache_len = n_old + n_acc;
        if (kk > 0) draft_len = n_old + (n_acc < kk - 1 ? n_acc : kk - 1);
        dm->cache_len = draft_len;
    }
done:
    dd->logits = dlogits;
    /* an error path may leave staged copies queued: let them run before the
     * next call rewrites the staging (a no-op after a normal round) */
    vxh_stream_sync(dd->stream);
    vxh_stream_sync(td->stream);
    return generated;
}

int vx_speculative_generate(vx_speculative_state *s, int *prompt, int prompt_len, int *output,
                            int max_tokens)
{
    if (!s || !prompt || !output || prompt_len < 1 || max_tokens < 1) return 0;
    if (vx_speculative_prefill(s, prompt, prompt_len) != prompt_len) return 0;
    return vx_speculative_decode(s, output, max_tokens);
}

int vx_speculative_generate_stream(vx_speculative_state *s, int token, int *output, int max_tokens)
{
    int prompt[1] = {token};
    return vx_speculative_generate(s, prompt, 1, output, max_tokens);
}
