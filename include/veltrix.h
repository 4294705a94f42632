/*
 * veltrix.h -- core types of the MI355X verify-step engine.
 *
 * Drop-in surface: every type and enum value below keeps the name, value and
 * member order of the CPU engine's public header (include/veltrix.h:15-183 in
 * the reference), so C callers written against it compile unchanged and read
 * the same fields (config, cache_len, k_cache, v_cache).  Differences:
 *
 *   - k_cache / v_cache hold DEVICE addresses (fp32 [layer][n_ctx][kv_dim],
 *     the reference's layout); they must not be dereferenced on the host.
 *   - tensor bytes live on the device after vx_model_create; vx_tensor.data is
 *     NULL for matrices that were uploaded.
 *   - the struct ends with one extra member, `dev`, the device-side state.
 *   - predictor / tokenizer members are kept as opaque pointers and stay NULL.
 */
#ifndef VELTRIX_H
#define VELTRIX_H

#include <stdint.h>
#include <stddef.h>
#include <stdbool.h>

#define VX_MAGIC "VX01"
#define VX_MAX_NAME 64
#define VX_MAX_LAYERS 256
#define VX_MAX_DIM 8192
#define VX_HEAD_DIM 128
#define VX_META_HDIM 128

/* Error codes (reference include/veltrix.h:15-24). */
typedef enum {
    VX_OK = 0,
    VX_ERR_FILE = -1,
    VX_ERR_FORMAT = -2,
    VX_ERR_MEMORY = -3,
    VX_ERR_PARAM = -4,
    VX_ERR_GGUF = -5,
    VX_ERR_NOMODEL = -6,
    VX_ERR_UNSUPPORTED = -7,
} vx_error;

/* Tensor element types; values are the GGML type ids (include/veltrix.h:26-47). */
typedef enum {
    VX_TYPE_F32 = 0,
    VX_TYPE_F16 = 1,
    VX_TYPE_Q4_0 = 2,
    VX_TYPE_Q4_1 = 3,
    VX_TYPE_Q5_0 = 6,
    VX_TYPE_Q5_1 = 7,
    VX_TYPE_Q8_0 = 8,
    VX_TYPE_Q8_1 = 9,
    VX_TYPE_Q2_K = 10,
    VX_TYPE_Q3_K = 11,
    VX_TYPE_Q4_K = 12,
    VX_TYPE_Q5_K = 13,
    VX_TYPE_Q6_K = 14,
    VX_TYPE_Q8_K = 15,
    VX_TYPE_IQ1_S = 20,
    VX_TYPE_IQ2_XXS = 21,
    VX_TYPE_IQ2_XS = 22,
    VX_TYPE_IQ3_XXS = 26,
    VX_TYPE_IQ1_M = 31,
    VX_TYPE_BF16 = 32,
} vx_type;

/* ne[] is in GGUF order: ne[0] = columns (K), ne[1] = rows (N). */
typedef struct {
    int32_t ne[4];
    size_t nbytes;
    vx_type type;
    uint8_t *data;
    bool owned;
    char name[VX_MAX_NAME];
} vx_tensor;

typedef enum {
    VX_ARCH_QWEN2 = 0,
    VX_ARCH_LLAMA,
    VX_ARCH_MISTRAL,
    VX_ARCH_GEMMA,
    VX_ARCH_PHI,
    VX_ARCH_PHI3,
    VX_ARCH_STARCODER,
    VX_ARCH_COUNT,
} vx_arch;

typedef enum {
    VX_MLP_SWIGLU = 0,
    VX_MLP_GEGLU,
    VX_MLP_CLASSIC,
} vx_mlp_type;

typedef enum {
    VX_NORM_RMS = 0,
    VX_NORM_LAYER,
} vx_norm_type;

/* Model hyper-parameters (include/veltrix.h:80-102). */
typedef struct {
    int n_layers;
    int n_heads;
    int n_kv_heads;
    int n_embd;
    int n_head_dim;
    int n_ff;
    int n_vocab;
    int n_ctx;
    float rope_theta;
    float rope_freq_base;
    int n_threads;
    vx_arch arch;
    vx_mlp_type mlp_type;
    vx_norm_type norm_type;
    int rope_partial_dims;
    bool has_q_bias;
    bool has_k_bias;
    bool has_v_bias;
    bool has_post_attn_norm;
    bool has_post_ffn_norm;
    bool has_ffn_bias;
} vx_model_config;

typedef enum {
    VX_COMPUTE_EXACT = 0,
    VX_COMPUTE_ATTN_ONLY,
    VX_COMPUTE_SKIP,
} vx_compute_level;

/* The reference's meta-predictor is not part of this engine; only its pointer
 * type is kept so the struct below stays source-compatible. */
typedef struct vx_meta_predictor vx_meta_predictor;
struct vx_tokenizer;

typedef struct vx_model {
    vx_model_config config;
    vx_tensor **tensors;
    int n_tensors;
    void *tensor_data;
    vx_tensor *tok_embd;
    vx_tensor **attn_q;
    vx_tensor **attn_k;
    vx_tensor **attn_v;
    vx_tensor **attn_o;
    vx_tensor **attn_q_bias;
    vx_tensor **attn_k_bias;
    vx_tensor **attn_v_bias;
    vx_tensor **ffn_gate;
    vx_tensor **ffn_up;
    vx_tensor **ffn_down;
    vx_tensor **ffn_gate_bias;
    vx_tensor **ffn_up_bias;
    vx_tensor **ffn_down_bias;
    vx_tensor **attn_norm;
    vx_tensor **ffn_norm;
    vx_tensor **attn_norm_bias;
    vx_tensor **ffn_norm_bias;
    vx_tensor *norm_w;
    vx_tensor *norm_bias_w;
    vx_tensor *output_w;
    vx_meta_predictor **layer_predictors;
    vx_meta_predictor *attn_pattern_predictor;
    vx_meta_predictor *token_exit_predictor;
    float *k_cache;            /* device address, fp32 [n_layers][n_ctx][kv_dim] */
    float *v_cache;            /* device address, same layout                     */
    int cache_len;             /* positions [0, cache_len) of the KV cache are valid */
    float *scratch;
    size_t scratch_size;
    float *dequant_tmp;
    size_t dequant_tmp_size;
    struct vx_tokenizer *tokenizer;
    void *dev;                 /* engine-private device state (appended member) */
} vx_model;

/* Model lifecycle and forward (include/veltrix.h:175-183, include/model.h:6-8). */
vx_error vx_model_create(const char *path, vx_model **model);
void vx_model_destroy(vx_model *model);
vx_error vx_model_forward(vx_model *model, const int *tokens, int n_tokens, float *logits);
void vx_model_kv_truncate(vx_model *model, int length);
void vx_set_compute_level(vx_compute_level level);
/* include/veltrix.h:180 of the reference declares it and src/ defines it
 * nowhere; here it is defined and ignored (meta-learning is not on the
 * verify path). */
void vx_enable_metalearn(bool enable);
void vx_set_n_threads(int n);
void vx_set_forward_timing_enabled(int enabled);
void vx_print_forward_timing(void);

#endif
