/*
 * gguf.c -- GGUF v2/v3 reader for vx_model_create (host side, cold path).
 *
 * Follows the observable behaviour of the reference loader so that the same
 * file yields the same model configuration:
 *   - tensor data starts at the 32-byte aligned end of the tensor infos and
 *     each tensor at data_start + offset (src/gguf.c:112-218, 231-234);
 *   - hyper-parameters are found by SUBSTRING match on the key, scanning the
 *     KV section from a shared cursor that stays put after a hit and moves to
 *     the end of the section after a miss (src/gguf.c:293-489, 523-536), in
 *     the reference's order: block_count, head_count, head_count_kv,
 *     embedding_length, feedforward_length, vocab_size,
 *     vocabulary.vocab_size, rope.freq_base, general.architecture;
 *   - defaults 32 layers / 32 heads / n_embd 4096 / n_ctx 4096 / theta 1e4
 *     (src/gguf.c:525-548), the architecture table and weight-name patterns of
 *     src/format.c:84-203 and the dimension fallbacks of src/format.c:287-322.
 */
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "vx_host.h"

#define GGUF_MAGIC_LE 0x46554747u

static size_t scalar_size(uint32_t t)
{
    switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
    }
}

/* Advances *o past one KV value of type t.  Returns 0, or -1 when the value
 * runs past the buffer or has a type the reference does not skip. */
static int skip_value(const uint8_t *p, size_t size, uint64_t *o, uint32_t t)
{
    if (t == 8) {
        uint64_t n;
        if (*o + 8 > size) return -1;
        memcpy(&n, p + *o, 8);
        *o += 8;
        if (*o + n > size) return -1;
        *o += n;
        return 0;
    }
    if (t == 9) {
        uint32_t at;
        uint64_t n;
        if (*o + 4 > size) return -1;
        memcpy(&at, p + *o, 4);
        *o += 4;
        if (*o + 8 > size) return -1;
        memcpy(&n, p + *o, 8);
        *o += 8;
        for (uint64_t j = 0; j < n; j++) {
            if (at == 8) {
                if (skip_value(p, size, o, 8)) return -1;
            } else {
                size_t s = scalar_size(at);
                if (!s) return -1;
                *o += s;
            }
        }
        return 0;
    }
    size_t s = scalar_size(t);
    if (!s) return -1;
    *o += s;
    return 0;
}

/* One substring scan.  want: 1 = u32/i32, 2 = f32, 3 = string.  Returns 1 on a
 * hit (value copied to out), 0 on a miss (cursor moved to the section end) and
 * -1 when the walk stopped on malformed data (cursor unchanged). */
static int kv_scan(const uint8_t *p, size_t size, uint64_t *cursor, uint64_t n_kv,
                   const char *suffix, int want, void *out, int out_len)
{
    uint64_t o = *cursor;
    for (uint64_t i = 0; i < n_kv; i++) {
        uint64_t klen;
        if (o + 8 > size) return -1;
        memcpy(&klen, p + o, 8);
        o += 8;
        if (o + klen > size) return -1;
        char key[128];
        size_t nc = klen > 127 ? 127 : (size_t)klen;
        memcpy(key, p + o, nc);
        key[nc] = 0;
        o += klen;
        uint32_t t;
        if (o + 4 > size) return -1;
        memcpy(&t, p + o, 4);
        o += 4;
        int hit = strstr(key, suffix) != NULL &&
                  ((want == 1 && (t == 4 || t == 5)) || (want == 2 && t == 6) || (want == 3 && t == 8));
        if (hit) {
            if (want == 3) {
                uint64_t n;
                if (o + 8 > size) return -1;
                memcpy(&n, p + o, 8);
                if (o + 8 + n > size) return -1;
                size_t c = n > (uint64_t)(out_len - 1) ? (size_t)(out_len - 1) : (size_t)n;
                memcpy(out, p + o + 8, c);
                ((char *)out)[c] = 0;
            } else {
                if (o + 4 > size) return -1;
                memcpy(out, p + o, 4);
            }
            return 1;
        }
        if (skip_value(p, size, &o, t)) return -1;
    }
    *cursor = o;
    return 0;
}

static uint32_t scan_u32(const vx_gguf *g, uint64_t *cur, uint64_t n_kv, const char *sfx, uint32_t fb)
{
    uint32_t v;
    return kv_scan(g->buf, g->size, cur, n_kv, sfx, 1, &v, 0) == 1 ? v : fb;
}

static float scan_f32(const vx_gguf *g, uint64_t *cur, uint64_t n_kv, const char *sfx, float fb)
{
    float v;
    return kv_scan(g->buf, g->size, cur, n_kv, sfx, 2, &v, 0) == 1 ? v : fb;
}

/* --------------------------------------------------------------------------- */
/* architecture table (src/format.c:164-203)                                    */
/* --------------------------------------------------------------------------- */
typedef struct {
    const char *name;
    vx_arch arch;
    vx_mlp_type mlp;
    vx_norm_type norm;
    int rope_partial;
    bool qb, kb, vb, fb;
} arch_row;

static const arch_row k_arch[] = {
    {"qwen2", VX_ARCH_QWEN2, VX_MLP_SWIGLU, VX_NORM_RMS, 0, false, false, false, false},
    {"qwen2.5", VX_ARCH_QWEN2, VX_MLP_SWIGLU, VX_NORM_RMS, 0, false, false, false, false},
    {"qwen3", VX_ARCH_QWEN2, VX_MLP_SWIGLU, VX_NORM_RMS, 0, false, false, false, false},
    {"qwen3.5", VX_ARCH_QWEN2, VX_MLP_SWIGLU, VX_NORM_RMS, 0, false, false, false, false},
    {"qwen3.6", VX_ARCH_QWEN2, VX_MLP_SWIGLU, VX_NORM_RMS, 0, false, false, false, false},
    {"qwen3moe", VX_ARCH_QWEN2, VX_MLP_SWIGLU, VX_NORM_RMS, 0, false, false, false, false},
    {"llama", VX_ARCH_LLAMA, VX_MLP_SWIGLU, VX_NORM_RMS, 0, false, false, false, false},
    {"mistral", VX_ARCH_MISTRAL, VX_MLP_SWIGLU, VX_NORM_RMS, 0, false, false, false, false},
    {"mistralnemo", VX_ARCH_MISTRAL, VX_MLP_SWIGLU, VX_NORM_RMS, 0, false, false, false, false},
    {"gemma", VX_ARCH_GEMMA, VX_MLP_GEGLU, VX_NORM_RMS, 0, true, true, true, false},
    {"gemma2", VX_ARCH_GEMMA, VX_MLP_GEGLU, VX_NORM_RMS, 0, true, true, true, false},
    {"gemma3", VX_ARCH_GEMMA, VX_MLP_GEGLU, VX_NORM_RMS, 0, true, true, true, false},
    {"gemma-3", VX_ARCH_GEMMA, VX_MLP_GEGLU, VX_NORM_RMS, 0, true, true, true, false},
    {"gemma4", VX_ARCH_GEMMA, VX_MLP_GEGLU, VX_NORM_RMS, 0, true, true, true, false},
    {"gemma-4", VX_ARCH_GEMMA, VX_MLP_GEGLU, VX_NORM_RMS, 0, true, true, true, false},
    {"phi2", VX_ARCH_PHI, VX_MLP_CLASSIC, VX_NORM_LAYER, 64, true, true, true, true},
    {"phi3", VX_ARCH_PHI3, VX_MLP_SWIGLU, VX_NORM_LAYER, 0, false, false, false, false},
    {"starcoder2", VX_ARCH_STARCODER, VX_MLP_CLASSIC, VX_NORM_RMS, 0, false, false, false, false},
};

void vx_apply_arch(vx_model_config *cfg, const char *arch)
{
    for (size_t i = 0; i < sizeof(k_arch) / sizeof(k_arch[0]); i++) {
        if (strcmp(arch, k_arch[i].name) == 0) {
            cfg->arch = k_arch[i].arch;
            cfg->mlp_type = k_arch[i].mlp;
            cfg->norm_type = k_arch[i].norm;
            cfg->rope_partial_dims = k_arch[i].rope_partial;
            cfg->has_q_bias = k_arch[i].qb;
            cfg->has_k_bias = k_arch[i].kb;
            cfg->has_v_bias = k_arch[i].vb;
            cfg->has_ffn_bias = k_arch[i].fb;
            return;
        }
    }
    cfg->arch = VX_ARCH_LLAMA;
    cfg->mlp_type = VX_MLP_SWIGLU;
    cfg->norm_type = VX_NORM_RMS;
}

/* --------------------------------------------------------------------------- */
/* weight-name patterns (src/format.c:84-150): first pattern that exists wins    */
/* --------------------------------------------------------------------------- */
typedef struct {
    const char *role;
    const char *pat[7];
} role_row;

static const role_row k_roles[] = {
    {"tok_embd", {"token_embd.weight", "gpt_neox.embed_in.weight", "transformer.wte.weight",
                  "model.embed_tokens.weight", NULL}},
    {"output", {"output.weight", "lm_head.weight", "embed_out.weight", NULL}},
    {"output_norm", {"output_norm.weight", "norm.weight", "gpt_neox.final_layer_norm.weight",
                     "model.norm.weight", "transformer.ln_f.weight", NULL}},
    {"attn_norm", {"blk.%d.attn_norm.weight", "blk.%d.rms_norm.weight",
                   "model.layers.%d.input_layernorm.weight", "model.layers.%d.rms_norm.weight",
                   "h.%d.ln_1.weight", "transformer.h.%d.ln_1.weight", NULL}},
    {"ffn_norm", {"blk.%d.ffn_norm.weight", "blk.%d.post_attention_norm.weight",
                  "model.layers.%d.post_attention_layernorm.weight",
                  "model.layers.%d.rms_norm.weight", "h.%d.ln_2.weight",
                  "transformer.h.%d.ln_2.weight", NULL}},
    {"attn_q", {"blk.%d.attn_q.weight", "blk.%d.self_attn.q_proj.weight",
                "model.layers.%d.self_attn.q_proj.weight", "h.%d.attn.q_proj.weight",
                "transformer.h.%d.attn.q_proj.weight", NULL}},
    {"attn_k", {"blk.%d.attn_k.weight", "blk.%d.self_attn.k_proj.weight",
                "model.layers.%d.self_attn.k_proj.weight", "h.%d.attn.k_proj.weight",
                "transformer.h.%d.attn.k_proj.weight", NULL}},
    {"attn_v", {"blk.%d.attn_v.weight", "blk.%d.self_attn.v_proj.weight",
                "model.layers.%d.self_attn.v_proj.weight", "h.%d.attn.v_proj.weight",
                "transformer.h.%d.attn.v_proj.weight", NULL}},
    {"attn_q_bias", {"blk.%d.attn_q.bias", "blk.%d.self_attn.q_proj.bias",
                     "model.layers.%d.self_attn.q_proj.bias", "h.%d.attn.q_proj.bias", NULL}},
    {"attn_k_bias", {"blk.%d.attn_k.bias", "blk.%d.self_attn.k_proj.bias",
                     "model.layers.%d.self_attn.k_proj.bias", "h.%d.attn.k_proj.bias", NULL}},
    {"attn_v_bias", {"blk.%d.attn_v.bias", "blk.%d.self_attn.v_proj.bias",
                     "model.layers.%d.self_attn.v_proj.bias", "h.%d.attn.v_proj.bias", NULL}},
    {"attn_o", {"blk.%d.attn_output.weight", "blk.%d.self_attn.o_proj.weight",
                "model.layers.%d.self_attn.o_proj.weight", "h.%d.attn.out_proj.weight",
                "transformer.h.%d.attn.out_proj.weight", NULL}},
    {"ffn_gate", {"blk.%d.ffn_gate.weight", "blk.%d.mlp.gate_proj.weight",
                  "model.layers.%d.mlp.gate_proj.weight", "h.%d.mlp.gate_proj.weight", NULL}},
    {"ffn_up", {"blk.%d.ffn_up.weight", "blk.%d.mlp.up_proj.weight",
                "model.layers.%d.mlp.up_proj.weight", "h.%d.mlp.up_proj.weight",
                "model.layers.%d.mlp.fc1.weight", NULL}},
    {"ffn_down", {"blk.%d.ffn_down.weight", "blk.%d.mlp.down_proj.weight",
                  "model.layers.%d.mlp.down_proj.weight", "h.%d.mlp.down_proj.weight",
                  "model.layers.%d.mlp.fc2.weight", NULL}},
};

const vx_gguf_tensor *vx_gguf_find(const vx_gguf *g, const char *name)
{
    for (int i = 0; i < g->n_tensors; i++)
        if (strcmp(g->tensors[i].name, name) == 0) return &g->tensors[i];
    return NULL;
}

const vx_gguf_tensor *vx_gguf_find_role(const vx_gguf *g, const char *role, int layer)
{
    for (size_t r = 0; r < sizeof(k_roles) / sizeof(k_roles[0]); r++) {
        if (strcmp(k_roles[r].role, role) != 0) continue;
        for (int k = 0; k_roles[r].pat[k]; k++) {
            char name[128];
            if (layer >= 0) snprintf(name, sizeof(name), k_roles[r].pat[k], layer);
            else snprintf(name, sizeof(name), "%s", k_roles[r].pat[k]);
            const vx_gguf_tensor *t = vx_gguf_find(g, name);
            if (t) return t;
        }
        return NULL;
    }
    return NULL;
}

/* --------------------------------------------------------------------------- */
/* file                                                                         */
/* --------------------------------------------------------------------------- */
void vx_gguf_close(vx_gguf *g)
{
    free(g->buf);
    free(g->tensors);
    memset(g, 0, sizeof(*g));
}

vx_error vx_gguf_open(const char *path, vx_gguf *g)
{
    memset(g, 0, sizeof(*g));
    FILE *fp = fopen(path, "rb");
    if (!fp) { vx_set_error("cannot open %s", path); return VX_ERR_FILE; }
    fseek(fp, 0, SEEK_END);
    long sz = ftell(fp);
    fseek(fp, 0, SEEK_SET);
    if (sz < 24) { fclose(fp); vx_set_error("%s: too short for GGUF", path); return VX_ERR_FORMAT; }
    g->buf = (uint8_t *)malloc((size_t)sz);
    if (!g->buf) { fclose(fp); return VX_ERR_MEMORY; }
    if (fread(g->buf, 1, (size_t)sz, fp) != (size_t)sz) {
        fclose(fp);
        vx_gguf_close(g);
        return VX_ERR_PARAM;
    }
    fclose(fp);
    g->size = (size_t)sz;
    const uint8_t *p = g->buf;
    uint32_t magic;
    uint64_t n_tensors, n_kv;
    memcpy(&magic, p, 4);
    if (magic != GGUF_MAGIC_LE) {
        vx_set_error("%s: bad GGUF magic 0x%08X", path, magic);
        vx_gguf_close(g);
        return VX_ERR_FORMAT;
    }
    memcpy(&n_tensors, p + 8, 8);
    memcpy(&n_kv, p + 16, 8);

    /* tensor infos follow the KV section */
    uint64_t o = 24;
    for (uint64_t i = 0; i < n_kv; i++) {
        uint64_t klen;
        if (o + 8 > g->size) goto bad;
        memcpy(&klen, p + o, 8);
        o += 8 + klen;
        uint32_t t;
        if (o + 4 > g->size) goto bad;
        memcpy(&t, p + o, 4);
        o += 4;
        if (skip_value(p, g->size, &o, t)) goto bad;
    }
    if (n_tensors > 1000000) goto bad;
    g->n_tensors = (int)n_tensors;
    g->tensors = (vx_gguf_tensor *)calloc(n_tensors ? n_tensors : 1, sizeof(vx_gguf_tensor));
    if (!g->tensors) { vx_gguf_close(g); return VX_ERR_MEMORY; }
    uint64_t *offs = (uint64_t *)calloc(n_tensors ? n_tensors : 1, sizeof(uint64_t));
    if (!offs) { vx_gguf_close(g); return VX_ERR_MEMORY; }
    for (uint64_t i = 0; i < n_tensors; i++) {
        vx_gguf_tensor *t = &g->tensors[i];
        uint64_t nlen;
        if (o + 8 > g->size) { free(offs); goto bad; }
        memcpy(&nlen, p + o, 8);
        o += 8;
        if (o + nlen > g->size) { free(offs); goto bad; }
        size_t nc = nlen > VX_MAX_NAME - 1 ? VX_MAX_NAME - 1 : (size_t)nlen;
        memcpy(t->name, p + o, nc);
        t->name[nc] = 0;
        o += nlen;
        uint32_t nd;
        if (o + 4 > g->size) { free(offs); goto bad; }
        memcpy(&nd, p + o, 4);
        o += 4;
        if (nd > 4) { free(offs); goto bad; }
        t->n_dims = (int)nd;
        for (uint32_t d = 0; d < nd; d++) {
            if (o + 8 > g->size) { free(offs); goto bad; }
            uint64_t v;
            memcpy(&v, p + o, 8);
            t->ne[d] = (int64_t)(uint32_t)v;
            o += 8;
        }
        uint32_t gt;
        if (o + 12 > g->size) { free(offs); goto bad; }
        memcpy(&gt, p + o, 4);
        memcpy(&offs[i], p + o + 4, 8);
        o += 12;
        t->type = (int)gt;
    }
    uint64_t data0 = (o + 31) / 32 * 32;
    for (uint64_t i = 0; i < n_tensors; i++) {
        vx_gguf_tensor *t = &g->tensors[i];
        if (data0 > g->size || offs[i] > g->size - data0) {
            vx_set_error("GGUF tensor range invalid for %s", t->name);
            free(offs);
            vx_gguf_close(g);
            return VX_ERR_FORMAT;
        }
        uint64_t start = data0 + offs[i];
        uint64_t end = (i + 1 < n_tensors) ? data0 + offs[i + 1] : g->size;
        t->data = p + start;
        t->nbytes = end > start ? (size_t)(end - start) : 0;
        if (end > g->size) t->nbytes = g->size - start;
    }
    free(offs);

    /* configuration: the reference's scan order and defaults */
    vx_model_config *c = &g->cfg;
    memset(c, 0, sizeof(*c));
    uint64_t cur = 24;
    int n_layers = (int)scan_u32(g, &cur, n_kv, "block_count", 32);
    int n_heads = (int)scan_u32(g, &cur, n_kv, "head_count", 32);
    int n_kv_heads = (int)scan_u32(g, &cur, n_kv, "head_count_kv", (uint32_t)n_heads);
    int n_embd = (int)scan_u32(g, &cur, n_kv, "embedding_length", 4096);
    int n_ff = (int)scan_u32(g, &cur, n_kv, "feedforward_length", 0);
    int n_vocab = (int)scan_u32(g, &cur, n_kv, "vocab_size", 0);
    if (n_vocab == 0) n_vocab = (int)scan_u32(g, &cur, n_kv, "vocabulary.vocab_size", 0);
    float theta = scan_f32(g, &cur, n_kv, "rope.freq_base", 10000.0f);
    char arch[64] = {0};
    kv_scan(g->buf, g->size, &cur, n_kv, "general.architecture", 3, arch, (int)sizeof(arch));
    c->n_layers = n_layers;
    c->n_heads = n_heads;
    c->n_kv_heads = n_kv_heads > 0 ? n_kv_heads : n_heads;
    c->n_embd = n_embd;
    c->n_head_dim = n_embd / (n_heads > 0 ? n_heads : 1);
    c->n_ff = n_ff;
    c->n_vocab = n_vocab;
    c->n_ctx = 4096;
    c->rope_theta = theta;
    c->n_threads = 1;
    vx_apply_arch(c, arch);

    /* dimension fallbacks (src/format.c:287-322) */
    if (c->n_ff == 0) {
        for (int i = 0; i < g->n_tensors; i++) {
            const char *nm = g->tensors[i].name;
            if (strstr(nm, "ffn_gate") || strstr(nm, "gate_proj") || strstr(nm, ".fc1.")) {
                c->n_ff = (int)g->tensors[i].ne[1];
                break;
            }
            if (strstr(nm, "ffn_down") || strstr(nm, "down_proj") || strstr(nm, ".fc2.")) {
                c->n_ff = (int)g->tensors[i].ne[0];
                break;
            }
        }
    }
    if (c->n_vocab <= 32000) {
        for (int i = 0; i < g->n_tensors; i++) {
            const char *nm = g->tensors[i].name;
            if (strstr(nm, "token_embd") || strstr(nm, "tok_embeddings") || strstr(nm, "embed_tokens")) {
                int v = (int)g->tensors[i].ne[1];
                if (v > c->n_vocab) c->n_vocab = v;
                break;
            }
        }
    }
    return VX_OK;
bad:
    vx_set_error("%s: malformed GGUF", path);
    vx_gguf_close(g);
    return VX_ERR_FORMAT;
}
