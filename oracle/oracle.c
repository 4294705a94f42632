/*
 * oracle.c -- CPU oracle (test infrastructure only; see oracle.h).
 *
 * Plain C11 + libm, single-threaded except for the row loops marked
 * `omp parallel for` (rows are independent, so results do not depend on the
 * thread count).  Built by oracle/Makefile with -O2 -fno-fast-math
 * -ffp-contract=off so every expression rounds the way the source text reads.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ===================================================================== */
/* fp16                                                                   */
/* ===================================================================== */

/* Exact IEEE half -> float, subnormals included (src/quantize.c:37-57). */
float or_fp16_to_fp32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t e = (uint32_t)(h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    float v;
    if (e == 0)
        v = ldexpf((float)m, -24);                 /* zero or subnormal, exact */
    else if (e == 31) {
        uint32_t bits = (sign << 31) | (0xffu << 23) | (m << 13);
        memcpy(&v, &bits, 4);
        return v;
    } else
        v = ldexpf((float)(m | 0x400u), (int)e - 25);
    return sign ? -v : v;
}

/* Truncating float -> half with flush-to-zero below the half normal range
 * and saturation to infinity above it (src/quantize.c:17-35). */
uint16_t or_fp32_to_fp16(float f)
{
    uint32_t bits;
    memcpy(&bits, &f, 4);
    uint16_t sign = (uint16_t)((bits >> 31) << 15);
    uint32_t e = (bits >> 23) & 0xffu;
    uint32_t m = bits & 0x7fffffu;
    if (e == 0) return sign;
    if (e == 0xff) return (uint16_t)(sign | 0x7c00u | (m >> 13));
    int he = (int)e - 112;                          /* rebias 127 -> 15 */
    if (he <= 0) return sign;
    if (he >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)he << 10) | (m >> 13));
}

/* ===================================================================== */
/* block formats                                                          */
/* ===================================================================== */

typedef struct { uint16_t d; uint8_t qs[16]; } or_blk4;
typedef struct { uint16_t d; int8_t qs[32]; } or_blk8;

/* Q4_0 writer: d = amax/7 (floored at 1e-10), stored truncated to half,
 * values truncated toward zero with the UNROUNDED 1/d, clamped to [-8,7],
 * offset by 8; element 2j -> low nibble of qs[j], 2j+1 -> high nibble.
 * Positions past n in the last block get nibble 0 (src/quantize.c:88-114). */
void or_quantize_row_q4_0(const float *x, void *vy, int n)
{
    or_blk4 *y = (or_blk4 *)vy;
    for (int base = 0; base < n; base += 32) {
        int rem = n - base < 32 ? n - base : 32;
        float amax = 0.0f;
        for (int j = 0; j < rem; j++) {
            float a = fabsf(x[base + j]);
            if (a > amax) amax = a;
        }
        float d = amax / 7.0f;
        if (d < 1e-10f) d = 1e-10f;
        or_blk4 *b = &y[base / 32];
        b->d = or_fp32_to_fp16(d);
        float inv = 1.0f / d;
        memset(b->qs, 0, 16);
        for (int j = 0; j < rem; j += 2) {
            int a0 = (int)(x[base + j] * inv);
            int a1 = (j + 1 < rem) ? (int)(x[base + j + 1] * inv) : 0;
            a0 = a0 < -8 ? -8 : (a0 > 7 ? 7 : a0);
            a1 = a1 < -8 ? -8 : (a1 > 7 ? 7 : a1);
            b->qs[j / 2] = (uint8_t)((a0 + 8) | ((a1 + 8) << 4));
        }
    }
}

/* value(t) = d * scale * (s_t - 8) (src/quantize.c:578-591). */
void or_dequantize_row_q4_0(const void *vx, float *y, int n, float scale)
{
    const or_blk4 *x = (const or_blk4 *)vx;
    for (int base = 0; base < n; base += 32) {
        float d = or_fp16_to_fp32(x[base / 32].d) * scale;
        for (int j = 0; j < 32 && base + j < n; j += 2) {
            uint8_t byte = x[base / 32].qs[j / 2];
            y[base + j] = (float)((int)(byte & 15) - 8) * d;
            if (base + j + 1 < n) y[base + j + 1] = (float)((int)(byte >> 4) - 8) * d;
        }
    }
}

/* value(t) = d * scale * qs[t] (src/quantize.c:642-651). */
void or_dequantize_row_q8_0(const void *vx, float *y, int n, float scale)
{
    const or_blk8 *x = (const or_blk8 *)vx;
    for (int base = 0; base < n; base += 32) {
        float d = or_fp16_to_fp32(x[base / 32].d) * scale;
        for (int j = 0; j < 32 && base + j < n; j++)
            y[base + j] = (float)x[base / 32].qs[j] * d;
    }
}

/* ===================================================================== */
/* matrix-vector                                                          */
/* ===================================================================== */

/* Exact Q4_0 GEMV in the order of the portable kernel: per pair,
 * sum += (v0*d)*x0 + (v1*d)*x1 (src/quantize.c:728-750). */
static float q4_row_exact(const or_blk4 *w, const float *x, int cols)
{
    int nb = (cols + 31) / 32;
    float sum = 0.0f;
    for (int b = 0, j = 0; b < nb; b++, j += 32) {
        float d = or_fp16_to_fp32(w[b].d);
        int lim = (j + 32 <= cols) ? 32 : cols - j;
        for (int k = 0; k < lim; k += 2) {
            uint8_t byte = w[b].qs[k / 2];
            float t0 = ((float)((int)(byte & 15) - 8) * d) * x[j + k];
            float t1 = ((float)((int)(byte >> 4) - 8) * d) * x[j + k + 1];
            sum = sum + (t0 + t1);
        }
    }
    return sum;
}

void or_gemv_q4_0(const void *A, const float *x, float *y, int rows, int cols)
{
    const or_blk4 *w = (const or_blk4 *)A;
    int nb = (cols + 31) / 32;
    #pragma omp parallel for
    for (int i = 0; i < rows; i++) y[i] = q4_row_exact(w + (size_t)i * nb, x, cols);
}

/* (src/quantize.c:680-704) */
void or_gemv_q4_0_sparse_rows(const void *A, const float *x, float *y, int rows, int cols,
                              const float *gate, float thr)
{
    const or_blk4 *w = (const or_blk4 *)A;
    int nb = (cols + 31) / 32;
    #pragma omp parallel for
    for (int i = 0; i < rows; i++)
        y[i] = fabsf(gate[i]) < thr ? 0.0f : q4_row_exact(w + (size_t)i * nb, x, cols);
}

/* Portable f32 GEMV: groups of four summed left to right, then added to the
 * running sum; scalar tail (src/tensor.c:103-120). */
static float f32_row(const float *a, const float *x, int cols)
{
    float sum = 0.0f;
    int j = 0;
    for (; j + 4 <= cols; j += 4) {
        float g = a[j] * x[j] + a[j + 1] * x[j + 1];
        g = g + a[j + 2] * x[j + 2];
        g = g + a[j + 3] * x[j + 3];
        sum = sum + g;
    }
    for (; j < cols; j++) sum = sum + a[j] * x[j];
    return sum;
}

void or_gemv_f32(float *y, const float *A, const float *x, int rows, int cols)
{
    #pragma omp parallel for
    for (int i = 0; i < rows; i++) y[i] = f32_row(A + (size_t)i * cols, x, cols);
}

/* (src/tensor.c:71-88) */
void or_gemv_f32_sparse_rows(float *y, const float *A, const float *x, int rows, int cols,
                             const float *gate, float thr)
{
    #pragma omp parallel for
    for (int i = 0; i < rows; i++)
        y[i] = fabsf(gate[i]) < thr ? 0.0f : f32_row(A + (size_t)i * cols, x, cols);
}

/* Horizontal sum of eight lanes in the order of hsum256 / the hadd tail:
 * ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)) (src/simd/avx2.c:215-222). */
static float hsum8(const float a[8])
{
    float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    return (s0 + s1) + (s2 + s3);
}

/* One row of the AVX2 Q4_0 kernel, lane by lane (src/simd/avx2.c:318-369).
 * Per block the 32 nibbles s_0..s_31 are unpacked in adjacent-pair order.
 * Group g (0..3) multiplies s_{8g..8g+7} by x[8g..8g+7] and, because the
 * second 8-float load is offset by 4 while the second nibble vector holds only
 * s_{8g+4..8g+7} followed by zeros, also s_{8g+4..8g+7} by x[8g+4..8g+7];
 * the x-sum collects x[8g..8g+7] and x[8g+4..8g+11].  acc = d*sum_qx + acc,
 * then acc -= (d*8)*sum_xv. */
static float q4_row_avx2lanes(const or_blk4 *w, const float *x, int cols)
{
    int nb = (cols + 31) / 32;
    float acc[8] = {0};
    for (int b = 0; b < nb; b++) {
        const float *xb = x + 32 * b;
        float d = or_fp16_to_fp32(w[b].d);
        float s[32];
        for (int j = 0; j < 16; j++) {
            s[2 * j] = (float)(w[b].qs[j] & 15);
            s[2 * j + 1] = (float)(w[b].qs[j] >> 4);
        }
        float sqx[8] = {0}, sxv[8] = {0};
        for (int g = 0; g < 4; g++) {
            for (int l = 0; l < 8; l++) {
                float e_lo = s[8 * g + l];
                float e_hi = l < 4 ? s[8 * g + 4 + l] : 0.0f;
                float x_lo = xb[8 * g + l];
                float x_hi = xb[8 * g + 4 + l];
                sqx[l] = fmaf(e_lo, x_lo, sqx[l]);
                sqx[l] = fmaf(e_hi, x_hi, sqx[l]);
                sxv[l] = sxv[l] + x_lo;
                sxv[l] = sxv[l] + x_hi;
            }
        }
        float d8 = d * 8.0f;
        for (int l = 0; l < 8; l++) {
            acc[l] = fmaf(d, sqx[l], acc[l]);
            acc[l] = acc[l] - d8 * sxv[l];
        }
    }
    return hsum8(acc);
}

void or_gemv_q4_0_avx2lanes(const void *A, const float *x, float *y, int rows, int cols)
{
    const or_blk4 *w = (const or_blk4 *)A;
    int nb = (cols + 31) / 32;
    #pragma omp parallel for
    for (int i = 0; i < rows; i++) y[i] = q4_row_avx2lanes(w + (size_t)i * nb, x, cols);
}

/* (src/simd/avx2.c:224-279) */
void or_gemv_q4_0_avx2lanes_sparse_rows(const void *A, const float *x, float *y, int rows,
                                        int cols, const float *gate, float thr)
{
    const or_blk4 *w = (const or_blk4 *)A;
    int nb = (cols + 31) / 32;
    #pragma omp parallel for
    for (int i = 0; i < rows; i++)
        y[i] = fabsf(gate[i]) < thr ? 0.0f : q4_row_avx2lanes(w + (size_t)i * nb, x, cols);
}

/* AVX2 f32 GEMV: eight FMA lanes over full groups of 8, hadd tail, then a
 * scalar remainder (src/simd/avx2.c:182-204). */
static float f32_row_avx2lanes(const float *a, const float *x, int cols)
{
    float acc[8] = {0};
    int j = 0;
    for (; j + 8 <= cols; j += 8)
        for (int l = 0; l < 8; l++) acc[l] = fmaf(a[j + l], x[j + l], acc[l]);
    float s = hsum8(acc);
    for (; j < cols; j++) s = s + a[j] * x[j];
    return s;
}

void or_gemv_f32_avx2lanes(float *y, const float *A, const float *x, int rows, int cols)
{
    #pragma omp parallel for
    for (int i = 0; i < rows; i++) y[i] = f32_row_avx2lanes(A + (size_t)i * cols, x, cols);
}

/* ===================================================================== */
/* elementwise                                                            */
/* ===================================================================== */

/* o = w * (x / sqrt(mean(x^2) + 1e-5)) (src/tensor.c:128-142, portable branch). */
void or_rms_norm(float *o, const float *x, const float *w, int n)
{
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss = ss + x[i] * x[i];
    float rms = sqrtf(ss / (float)n + 1e-5f);
    if (rms < 1e-10f) {
        for (int i = 0; i < n; i++) o[i] = 0.0f;
        return;
    }
    float inv = 1.0f / rms;
    for (int i = 0; i < n; i++) o[i] = w[i] * (x[i] * inv);
}

/* Max-subtracted softmax, 1/(sum + 1e-10) (src/tensor.c:156-171). */
void or_softmax(float *x, int n)
{
    if (n <= 0) return;
    float mx = x[0];
    for (int i = 1; i < n; i++) if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - mx); sum = sum + x[i]; }
    if (sum < 1e-10f) {
        for (int i = 0; i < n; i++) x[i] = 1.0f / (float)n;
        return;
    }
    float inv = 1.0f / (sum + 1e-10f);
    for (int i = 0; i < n; i++) x[i] = x[i] * inv;
}

/* x / (1 + exp(-x)) (src/tensor.c:273-279, portable branch). */
void or_silu(float *x, int n)
{
    for (int i = 0; i < n; i++) x[i] = x[i] / (1.0f + expf(-x[i]));
}

/* Adjacent-pair rotary embedding: pair i of every head is rotated by
 * pos * theta^(-2i/head_dim) (src/tensor.c:173-187 angle table,
 * src/tensor.c:249-270 rotation; the portable branch). */
void or_rope(float *q, float *k, int pos, int n_heads, int n_kv_heads, int head_dim,
             int rope_dims, float theta)
{
    if (rope_dims <= 0 || rope_dims > head_dim) rope_dims = head_dim;
    int nkh = n_kv_heads > 0 ? n_kv_heads : n_heads;
    int npairs = rope_dims / 2;
    float *c = (float *)malloc(sizeof(float) * (size_t)(npairs > 0 ? npairs : 1));
    float *s = (float *)malloc(sizeof(float) * (size_t)(npairs > 0 ? npairs : 1));
    for (int i = 0; i < npairs; i++) {
        float freq = 1.0f / powf(theta, (float)(i * 2) / (float)head_dim);
        float ang = (float)pos * freq;
        c[i] = cosf(ang);
        s[i] = sinf(ang);
    }
    int maxh = n_heads > nkh ? n_heads : nkh;
    for (int h = 0; h < maxh; h++) {
        if (h < n_heads) {
            float *v = q + (size_t)h * head_dim;
            for (int i = 0; i < rope_dims; i += 2) {
                float a = v[i], b = v[i + 1];
                v[i] = a * c[i / 2] - b * s[i / 2];
                v[i + 1] = a * s[i / 2] + b * c[i / 2];
            }
        }
        if (h < nkh) {
            float *v = k + (size_t)h * head_dim;
            for (int i = 0; i < rope_dims; i += 2) {
                float a = v[i], b = v[i + 1];
                v[i] = a * c[i / 2] - b * s[i / 2];
                v[i + 1] = a * s[i / 2] + b * c[i / 2];
            }
        }
    }
    free(c);
    free(s);
}

/* ===================================================================== */
/* model                                                                  */
/* ===================================================================== */

static void dequant_any(int type, const void *src, float *dst, size_t n, float scale)
{
    if (type == OR_TYPE_Q4_0) or_dequantize_row_q4_0(src, dst, (int)n, scale);
    else if (type == OR_TYPE_Q8_0) or_dequantize_row_q8_0(src, dst, (int)n, scale);
    else memcpy(dst, src, n * sizeof(float));
}

/* The forward's matrix dispatch (src/model.c:203-245): absent -> zeros; F32 ->
 * f32 GEMV; Q4_0 -> lane kernel (x86 build) or dequantize + f32 GEMV
 * (portable build); other types -> dequantize + f32 GEMV.  `gate` selects the
 * sparse-row variant (src/model.c:169-201).  `inplace` reproduces a call with
 * y == x in a one-thread run: row i sees rows < i already overwritten. */
static void apply_mat(const or_model *m, const or_mat *w, const float *x, float *y,
                      int rows, int cols, const float *gate, float thr, int inplace,
                      float *tmp)
{
    if (!w || !w->data) { memset(y, 0, sizeof(float) * (size_t)rows); return; }
    int avx2 = m->q4_mode == OR_Q4_AVX2LANES;
    if (w->type == OR_TYPE_Q4_0 && avx2) {
        const or_blk4 *wb = (const or_blk4 *)w->data;
        int nb = (cols + 31) / 32;
        if (inplace) {
            for (int i = 0; i < rows; i++) {
                float v = (gate && fabsf(gate[i]) < thr) ? 0.0f
                         : q4_row_avx2lanes(wb + (size_t)i * nb, y, cols);
                y[i] = v;
            }
        } else if (gate) {
            or_gemv_q4_0_avx2lanes_sparse_rows(w->data, x, y, rows, cols, gate, thr);
        } else {
            or_gemv_q4_0_avx2lanes(w->data, x, y, rows, cols);
        }
        return;
    }
    const float *A;
    if (w->type == OR_TYPE_F32) {
        A = (const float *)w->data;
    } else {
        dequant_any(w->type, w->data, tmp, (size_t)rows * cols, m->wscale);
        A = tmp;
    }
    if (inplace) {
        for (int i = 0; i < rows; i++) {
            float v;
            if (gate && fabsf(gate[i]) < thr) v = 0.0f;
            else v = avx2 ? f32_row_avx2lanes(A + (size_t)i * cols, y, cols)
                          : f32_row(A + (size_t)i * cols, y, cols);
            y[i] = v;
        }
        return;
    }
    if (avx2) {
        if (gate) {
            for (int i = 0; i < rows; i++)
                y[i] = fabsf(gate[i]) < thr ? 0.0f : f32_row_avx2lanes(A + (size_t)i * cols, x, cols);
        } else {
            or_gemv_f32_avx2lanes(y, A, x, rows, cols);
        }
    } else {
        if (gate) or_gemv_f32_sparse_rows(y, A, x, rows, cols, gate, thr);
        else or_gemv_f32(y, A, x, rows, cols);
    }
}

/* apply_norm: the weight is used only when it is an F32 tensor, otherwise a
 * vector of ones (src/model.c:247-273). */
static void apply_norm(float *x, float *tmp, const float *w, int n, float *ones)
{
    or_rms_norm(tmp, x, w ? w : ones, n);
    memcpy(x, tmp, sizeof(float) * (size_t)n);
}

/* One head loop of the reference attention (src/model.c:275-341): write k,v at
 * pos = cache_len (clamped to n_ctx-1), then every query head h reads kv head
 * h*n_kv/n_heads over positions [0, min(pos+1, cap)), cap = 4096 in the
 * reference (src/model.c:304-305). */
/* binary16: 10 fraction bits, normal exponents -14..15, subnormal quantum
 * 2^-24, largest finite 65504; values from 65520 on round to infinity.
 * Scaling by powers of two is exact, nearbyint rounds ties to even. */
float or_round_half(float x)
{
    if (x != x) return x;
    double a = fabs((double)x);
    if (a == 0.0) return x;
    double q;
    if (a < 0x1p-14) {
        q = 0x1p-24;
    } else {
        int e;
        frexp(a, &e);                /* a = f * 2^e, f in [0.5, 1) */
        q = ldexp(1.0, e - 1 - 10);
    }
    double r = nearbyint(a / q) * q;
    if (r > 65504.0) r = INFINITY;
    return (float)(x < 0 ? -r : r);
}

static void attention(or_model *m, const float *q, const float *k, const float *v,
                      float *out, int layer, float *scores_all)
{
    int hd = m->n_head_dim, nh = m->n_heads, nkv = m->n_kv_heads;
    int kvd = nkv * hd;
    int pos = m->cache_len;
    int max_ctx = m->n_ctx < 1 ? 4096 : m->n_ctx;
    if (pos >= max_ctx) { pos = max_ctx - 1; m->cache_len = pos; }
    int cache_size = pos + 1;
    size_t loff = (size_t)layer * (size_t)max_ctx * kvd;
    float *kr = m->k_cache + loff + (size_t)pos * kvd, *vr = m->v_cache + loff + (size_t)pos * kvd;
    if (m->kv_keep) {   /* test hook: the caller's row stays; ours goes aside */
        kr = m->kv_own_k ? m->kv_own_k + (size_t)layer * kvd : NULL;
        vr = m->kv_own_v ? m->kv_own_v + (size_t)layer * kvd : NULL;
    }
    if (kr) memcpy(kr, k, sizeof(float) * (size_t)kvd);
    if (vr) memcpy(vr, v, sizeof(float) * (size_t)kvd);
    if (m->kv_half)
        for (int i = 0; i < kvd; i++) {
            if (kr) kr[i] = or_round_half(kr[i]);
            if (vr) vr[i] = or_round_half(vr[i]);
        }
    memset(out, 0, sizeof(float) * (size_t)nh * hd);
    int cs = cache_size;
    if (m->attn_cap > 0 && cs > m->attn_cap) cs = m->attn_cap;
    float scale = 1.0f / sqrtf((float)hd);
    /* heads are independent: each has its own scores row */
    #pragma omp parallel for schedule(static)
    for (int h = 0; h < nh; h++) {
        float *scores = scores_all + (size_t)h * (size_t)(max_ctx + 8);
        const float *qh = q + (size_t)h * hd;
        int kvh = nkv == 1 ? 0 : h * nkv / nh;
        for (int t = 0; t < cs; t++) {
            const float *kt = m->k_cache + loff + (size_t)t * kvd + (size_t)kvh * hd;
            float s = 0.0f;
            for (int d = 0; d < hd; d++) s = s + qh[d] * kt[d];
            scores[t] = (t <= pos) ? s * scale : -1e9f;
        }
        or_softmax(scores, cs);
        for (int d = 0; d < hd; d++) {
            float acc = 0.0f;
            for (int t = 0; t < cs; t++)
                acc = acc + scores[t] * m->v_cache[loff + (size_t)t * kvd + (size_t)kvh * hd + d];
            out[(size_t)h * hd + d] = acc;
        }
    }
}

/* Token embedding row (src/model.c:454-500): zeros for negative ids. */
static void embed(const or_model *m, int token, float *x, float *tmp)
{
    int n = m->n_embd;
    memset(x, 0, sizeof(float) * (size_t)n);
    const or_mat *e = &m->tok_embd;
    if (!e->data || token < 0) return;
    int stride = e->cols > 0 ? e->cols : n;
    if (e->type == OR_TYPE_F32) {
        long off = (long)token * stride;
        if (off + n <= (long)e->rows * e->cols)
            memcpy(x, (const float *)e->data + off, sizeof(float) * (size_t)n);
        return;
    }
    long start = (long)token * stride;
    int inblk = (int)(start % 32);
    size_t bsz = e->type == OR_TYPE_Q4_0 ? 18 : 34;
    const uint8_t *src = (const uint8_t *)e->data + (size_t)(start / 32) * bsz;
    dequant_any(e->type, src, tmp, (size_t)(stride + inblk), m->wscale);
    memcpy(x, tmp + inblk, sizeof(float) * (size_t)stride);
}

/* Test hook: the FFN column of token ti, layer l whose |silu(g)| is closest to
 * the skip threshold, and that distance. */
static void gate_log(const or_model *m, const float *g, int F, int ti, int l)
{
    float best = INFINITY;
    int bi = -1;
    for (int i = 0; i < F; i++) {
        float dist = fabsf(fabsf(g[i]) - m->gate_thr);
        if (dist < best) { best = dist; bi = i; }
    }
    size_t at = (size_t)ti * m->n_layers + l;
    if (m->gate_near) m->gate_near[at] = best;
    if (m->gate_near_idx) m->gate_near_idx[at] = bi;
}

/* Test hook: invert the skip decision of column i: a skipped up row is
 * computed (the same row product as an unskipped one), a computed one is zero. */
static void gate_flip(const or_model *m, const or_mat *w, const float *xn, const float *g, float *u,
                      int F, int d, float *tmp, int i)
{
    if (!(fabsf(g[i]) < m->gate_thr)) { u[i] = 0.0f; return; }
    if (!w->data) return;
    or_mat row = *w;
    size_t bsz = w->type == OR_TYPE_Q4_0 ? 18 : (w->type == OR_TYPE_Q8_0 ? 34 : 0);
    if (bsz) row.data = (const uint8_t *)w->data + (size_t)i * ((size_t)(d + 31) / 32) * bsz;
    else row.data = (const float *)w->data + (size_t)i * d;
    row.rows = 1;
    apply_mat(m, &row, xn, &u[i], 1, d, NULL, 0, 0, tmp);
    (void)F;
}

static int forward_impl(or_model *m, const int *tokens, int n, float *logits, int all)
{
    int d = m->n_embd, hd = m->n_head_dim, nh = m->n_heads, nkv = m->n_kv_heads;
    int kvd = nkv * hd, F = m->n_ff, V = m->n_vocab;
    if (d <= 0 || d > 8192) return -4;
    size_t big = (size_t)d;
    if ((size_t)F > big) big = F;
    size_t tmpn = 0;
    const or_mat *all_m[7];
    for (int l = 0; l < m->n_layers; l++) {
        all_m[0] = &m->wq[l]; all_m[1] = &m->wk[l]; all_m[2] = &m->wv[l]; all_m[3] = &m->wo[l];
        all_m[4] = &m->wg[l]; all_m[5] = &m->wu[l]; all_m[6] = &m->wd[l];
        for (int i = 0; i < 7; i++)
            if (all_m[i]->data) {
                size_t e = (size_t)all_m[i]->rows * all_m[i]->cols;
                if (e > tmpn) tmpn = e;
            }
    }
    if (m->output.data && (size_t)m->output.rows * m->output.cols > tmpn)
        tmpn = (size_t)m->output.rows * m->output.cols;
    if ((size_t)(m->tok_embd.cols + 32) > tmpn) tmpn = (size_t)m->tok_embd.cols + 32;
    int max_ctx = m->n_ctx < 1 ? 4096 : m->n_ctx;
    float *tmp = (float *)malloc(sizeof(float) * (tmpn + 64));
    float *x = (float *)calloc(big + 8, sizeof(float));
    float *xo = (float *)calloc(big + 8, sizeof(float));
    float *xn = (float *)calloc(big + 8, sizeof(float));   /* normed x incl. 4-float tail */
    float *ntmp = (float *)calloc(big + 8, sizeof(float));
    float *q = (float *)calloc((size_t)nh * hd + 8, sizeof(float));
    float *kk = (float *)calloc((size_t)kvd + 8, sizeof(float));
    float *vv = (float *)calloc((size_t)kvd + 8, sizeof(float));
    float *ao = (float *)calloc(big + 8, sizeof(float));
    float *g = (float *)calloc((size_t)F + 8, sizeof(float));
    float *u = (float *)calloc((size_t)F + 8, sizeof(float));
    float *ones = (float *)malloc(sizeof(float) * (big + 8));
    float *scores = (float *)malloc(sizeof(float) * (size_t)nh * (size_t)(max_ctx + 8));
    if (!tmp || !x || !xo || !xn || !ntmp || !q || !kk || !vv || !ao || !g || !u || !ones || !scores) {
        free(tmp); free(x); free(xo); free(xn); free(ntmp); free(q); free(kk); free(vv);
        free(ao); free(g); free(u); free(ones); free(scores);
        return -3;
    }
    for (size_t i = 0; i < big + 8; i++) ones[i] = 1.0f;
    int avx2 = m->q4_mode == OR_Q4_AVX2LANES;

    for (int ti = 0; ti < n; ti++) {
        int cache_pos = m->cache_len;
        embed(m, tokens[ti], x, tmp);
        for (int l = 0; l < m->n_layers; l++) {
            memcpy(xo, x, sizeof(float) * (size_t)d);
            memcpy(xn, x, sizeof(float) * (size_t)d);
            apply_norm(xn, ntmp, m->attn_norm ? m->attn_norm[l] : NULL, d, ones);
            /* x86-build tails: the four floats after the normed x are x_orig[0..3]
             * (src/model.c:425-427) */
            if (avx2) memcpy(xn + d, xo, 4 * sizeof(float));
            apply_mat(m, &m->wq[l], xn, q, nh * hd, d, NULL, 0, 0, tmp);
            if (m->bq && m->bq[l]) for (int i = 0; i < nh * hd; i++) q[i] += m->bq[l][i];
            apply_mat(m, &m->wk[l], xn, kk, kvd, d, NULL, 0, 0, tmp);
            if (m->bk && m->bk[l]) for (int i = 0; i < kvd; i++) kk[i] += m->bk[l][i];
            apply_mat(m, &m->wv[l], xn, vv, kvd, d, NULL, 0, 0, tmp);
            if (m->bv && m->bv[l]) for (int i = 0; i < kvd; i++) vv[i] += m->bv[l][i];
            or_rope(q, kk, cache_pos, nh, nkv, hd, 0, m->rope_theta);
            attention(m, q, kk, vv, ao, l, scores);
            if (m->wo[l].data) {
                /* attn_out's tail is norm_tmp[0..3] = the normed x of this layer
                 * (src/model.c:431-435) */
                if (avx2) memcpy(ao + nh * hd, xn, 4 * sizeof(float));
                if (m->attn_o_inplace) {
                    apply_mat(m, &m->wo[l], ao, ao, d, nh * hd, NULL, 0, 1, tmp);
                } else {
                    apply_mat(m, &m->wo[l], ao, q, d, nh * hd, NULL, 0, 0, tmp);
                    memcpy(ao, q, sizeof(float) * (size_t)d);
                }
            }
            for (int i = 0; i < d; i++) x[i] = xo[i] + ao[i];
            memcpy(xo, x, sizeof(float) * (size_t)d);
            memcpy(xn, x, sizeof(float) * (size_t)d);
            apply_norm(xn, ntmp, m->ffn_norm ? m->ffn_norm[l] : NULL, d, ones);
            if (avx2) memcpy(xn + d, xo, 4 * sizeof(float));
            memset(g, 0, sizeof(float) * (size_t)F);
            memset(u, 0, sizeof(float) * (size_t)F);
            apply_mat(m, &m->wg[l], xn, g, F, d, NULL, 0, 0, tmp);
            or_silu(g, F);
            apply_mat(m, &m->wu[l], xn, u, F, d, g, m->gate_thr, 0, tmp);
            if (m->gate_near || m->gate_near_idx) gate_log(m, g, F, ti, l);
            for (int f = 0; f < m->flip && f < OR_MAX_FLIPS; f++)
                if (m->flip_tok[f] == ti && m->flip_layer[f] == l && m->flip_col[f] >= 0 && m->flip_col[f] < F)
                    gate_flip(m, &m->wu[l], xn, g, u, F, d, tmp, m->flip_col[f]);
            for (int i = 0; i < F; i++) g[i] = g[i] * u[i];
            /* the down projection's tail is an unwritten pad in the reference
             * (src/model.c:432-433); it is read as zeros here */
            if (avx2) memset(g + F, 0, 4 * sizeof(float));
            apply_mat(m, &m->wd[l], g, ao, d, F, NULL, 0, 0, tmp);
            for (int i = 0; i < d; i++) x[i] = xo[i] + ao[i];
        }
        m->cache_len++;
        if (all || ti == n - 1) {
            float *lg = all ? logits + (size_t)ti * V : logits;
            float *xf = xn;
            memcpy(xf, x, sizeof(float) * (size_t)d);
            if (m->has_out_norm) apply_norm(xf, ntmp, m->out_norm, d, ones);
            if (avx2) memcpy(xf + d, xo, 4 * sizeof(float));
            for (int i = 0; i < V; i++) lg[i] = -1e30f;
            if (m->output.data) {
                int orows = m->output.rows;
                int ocols = m->output.cols > 0 ? m->output.cols : d;
                if (orows > 0 && orows <= V)
                    apply_mat(m, &m->output, xf, lg, orows, ocols, NULL, 0, 0, tmp);
            }
        }
    }
    free(tmp); free(x); free(xo); free(xn); free(ntmp); free(q); free(kk); free(vv);
    free(ao); free(g); free(u); free(ones); free(scores);
    return 0;
}

/* ===================================================================== */
/* layer-major forward (same results as forward_impl, faster)             */
/* ===================================================================== */

/* forward_impl runs each token through every layer before the next token,
 * dequantising every matrix once per token.  The functions below run a
 * chunk of tokens one layer at a time: each matrix is dequantised once per
 * chunk and multiplied with all of the chunk's tokens, with the token index
 * in the lanes of a GCC vector.  Every lane performs, for its (row, token),
 * the same sequence of fp32 operations as f32_row, the attention of token t
 * at layer l runs after tokens < t wrote their rows of layer l, and the
 * elementwise steps run per token in the same order as forward_impl: the
 * results are bit-identical to forward_impl's (or_forward_tokenwise), which
 * tests/test_oracle_forward.py checks.  The x86 lane mode (its 4-float
 * tails) is served by forward_impl only. */
typedef float or_v8 __attribute__((vector_size(32)));
#define OR_LANES 16        /* tokens per lane block: two vectors */
#define OR_CHUNK 256       /* tokens per layer-major chunk */

/* Dequantisation split over rows; every element is computed as in
 * dequant_any. */
static void dequant_rows_par(const or_mat *w, float *dst, int rows, int cols, float scale)
{
    if (w->type == OR_TYPE_F32) { memcpy(dst, w->data, sizeof(float) * (size_t)rows * cols); return; }
    if (cols % 32) { dequant_any(w->type, w->data, dst, (size_t)rows * cols, scale); return; }
    size_t bsz = w->type == OR_TYPE_Q4_0 ? 18 : 34;
    int nb = cols / 32;
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < rows; i++)
        dequant_any(w->type, (const uint8_t *)w->data + (size_t)i * nb * bsz, dst + (size_t)i * cols,
                    (size_t)cols, scale);
}

/* f32_row of one matrix row against 16 tokens: xb holds the tokens' vectors
 * as [k][16]. */
static void f32_row_lanes(const float *a, const float *xb, int cols, float *out)
{
    or_v8 s0 = {0}, s1 = {0};
    int j = 0;
    for (; j + 4 <= cols; j += 4) {
        const or_v8 *x = (const or_v8 *)(xb + (size_t)j * OR_LANES);
        or_v8 a0 = {a[j], a[j], a[j], a[j], a[j], a[j], a[j], a[j]};
        or_v8 a1 = {a[j + 1], a[j + 1], a[j + 1], a[j + 1], a[j + 1], a[j + 1], a[j + 1], a[j + 1]};
        or_v8 a2 = {a[j + 2], a[j + 2], a[j + 2], a[j + 2], a[j + 2], a[j + 2], a[j + 2], a[j + 2]};
        or_v8 a3 = {a[j + 3], a[j + 3], a[j + 3], a[j + 3], a[j + 3], a[j + 3], a[j + 3], a[j + 3]};
        or_v8 g0 = a0 * x[0] + a1 * x[2];
        or_v8 g1 = a0 * x[1] + a1 * x[3];
        g0 = g0 + a2 * x[4];
        g1 = g1 + a2 * x[5];
        g0 = g0 + a3 * x[6];
        g1 = g1 + a3 * x[7];
        s0 = s0 + g0;
        s1 = s1 + g1;
    }
    for (; j < cols; j++) {
        const or_v8 *x = (const or_v8 *)(xb + (size_t)j * OR_LANES);
        or_v8 aj = {a[j], a[j], a[j], a[j], a[j], a[j], a[j], a[j]};
        s0 = s0 + aj * x[0];
        s1 = s1 + aj * x[1];
    }
    memcpy(out, &s0, 32);
    memcpy(out + 8, &s1, 32);
}

/* The chunk's tokens X[t][.] (row stride ldx) in lane blocks [tb][k][16],
 * zero past n. */
static void to_lanes(const float *X, int ldx, int n, int cols, float *xb)
{
    int ntb = (n + OR_LANES - 1) / OR_LANES;
    for (int tb = 0; tb < ntb; tb++)
        for (int k = 0; k < cols; k++)
            for (int l = 0; l < OR_LANES; l++) {
                int t = tb * OR_LANES + l;
                xb[((size_t)tb * cols + k) * OR_LANES + l] = t < n ? X[(size_t)t * ldx + k] : 0.0f;
            }
}

/* apply_mat (not in place) for n tokens: Y[t][i] = f32_row(A_i, X[t]), or 0
 * where gate[t][i] is below thr. */
static void apply_mat_tokens(const or_model *m, const or_mat *w, const float *X, int ldx, int n, float *Y,
                             int ldy, int rows, int cols, const float *gate, int ldg, float thr, float *A,
                             float *xb)
{
    if (!w || !w->data) {
        for (int t = 0; t < n; t++) memset(Y + (size_t)t * ldy, 0, sizeof(float) * (size_t)rows);
        return;
    }
    dequant_rows_par(w, A, rows, cols, m->wscale);
    to_lanes(X, ldx, n, cols, xb);
    int ntb = (n + OR_LANES - 1) / OR_LANES;
    #pragma omp parallel for schedule(dynamic, 1)
    for (int ib = 0; ib < rows; ib += 8)
        for (int tb = 0; tb < ntb; tb++)
            for (int i = ib; i < ib + 8 && i < rows; i++) {
                float o[OR_LANES];
                f32_row_lanes(A + (size_t)i * cols, xb + (size_t)tb * cols * OR_LANES, cols, o);
                for (int l = 0; l < OR_LANES; l++) {
                    int t = tb * OR_LANES + l;
                    if (t >= n) break;
                    Y[(size_t)t * ldy + i] = (gate && fabsf(gate[(size_t)t * ldg + i]) < thr) ? 0.0f : o[l];
                }
            }
}

/* apply_mat in place for n tokens: row i of token t reads token t's vector
 * (cols elements) with rows < i already overwritten; xb has room for
 * max(rows, cols) elements per token. */
static void apply_mat_tokens_inplace(const or_model *m, const or_mat *w, float *X, int ldx, int n, int rows,
                                     int cols, float *A, float *xb)
{
    int w_ld = rows > cols ? rows : cols;
    dequant_rows_par(w, A, rows, cols, m->wscale);
    int ntb = (n + OR_LANES - 1) / OR_LANES;
    #pragma omp parallel for schedule(dynamic, 1)
    for (int tb = 0; tb < ntb; tb++) {
        float *blk = xb + (size_t)tb * w_ld * OR_LANES;
        for (int k = 0; k < w_ld; k++)
            for (int l = 0; l < OR_LANES; l++) {
                int t = tb * OR_LANES + l;
                blk[(size_t)k * OR_LANES + l] = t < n ? X[(size_t)t * ldx + k] : 0.0f;
            }
        for (int i = 0; i < rows; i++) {
            float o[OR_LANES];
            f32_row_lanes(A + (size_t)i * cols, blk, cols, o);
            memcpy(blk + (size_t)i * OR_LANES, o, sizeof o);
        }
        for (int l = 0; l < OR_LANES; l++) {
            int t = tb * OR_LANES + l;
            if (t >= n) break;
            for (int i = 0; i < rows; i++) X[(size_t)t * ldx + i] = blk[(size_t)i * OR_LANES + l];
        }
    }
}

static int forward_chunk(or_model *m, const int *tokens, int n, int t_base, float *logits, int all, float *A,
                         float *xb, float *wk)
{
    int d = m->n_embd, hd = m->n_head_dim, nh = m->n_heads, nkv = m->n_kv_heads;
    int kvd = nkv * hd, F = m->n_ff, V = m->n_vocab, qd = nh * hd;
    int big = d > F ? d : F;
    if (qd > big) big = qd;
    int max_ctx = m->n_ctx < 1 ? 4096 : m->n_ctx;
    /* per-token state, token-major: [n][ld] */
    int ld = big + 8;
    float *X = wk, *XO = X + (size_t)n * ld, *XN = XO + (size_t)n * ld, *Q = XN + (size_t)n * ld;
    float *K = Q + (size_t)n * ld, *Vv = K + (size_t)n * ld, *AO = Vv + (size_t)n * ld;
    float *G = AO + (size_t)n * ld, *U = G + (size_t)n * ld, *T = U + (size_t)n * ld;
    float *ntmp = T + (size_t)n * ld, *ones = ntmp + ld, *scores = ones + ld;
    int *rope_pos = (int *)malloc(sizeof(int) * (size_t)n), *att_pos = (int *)malloc(sizeof(int) * (size_t)n);
    if (!rope_pos || !att_pos) { free(rope_pos); free(att_pos); return -3; }
    for (int i = 0; i < ld; i++) ones[i] = 1.0f;
    /* the cache positions forward_impl's attention() uses, clamp included */
    int c = m->cache_len;
    for (int t = 0; t < n; t++) {
        rope_pos[t] = c;
        att_pos[t] = c >= max_ctx ? max_ctx - 1 : c;
        c = att_pos[t] + 1;
    }
    for (int t = 0; t < n; t++) embed(m, tokens[t], X + (size_t)t * ld, A);
    for (int l = 0; l < m->n_layers; l++) {
        for (int t = 0; t < n; t++) {
            float *xo = XO + (size_t)t * ld, *xn = XN + (size_t)t * ld, *x = X + (size_t)t * ld;
            memcpy(xo, x, sizeof(float) * (size_t)d);
            memcpy(xn, x, sizeof(float) * (size_t)d);
            apply_norm(xn, ntmp, m->attn_norm ? m->attn_norm[l] : NULL, d, ones);
        }
        apply_mat_tokens(m, &m->wq[l], XN, ld, n, Q, ld, qd, d, NULL, 0, 0.0f, A, xb);
        apply_mat_tokens(m, &m->wk[l], XN, ld, n, K, ld, kvd, d, NULL, 0, 0.0f, A, xb);
        apply_mat_tokens(m, &m->wv[l], XN, ld, n, Vv, ld, kvd, d, NULL, 0, 0.0f, A, xb);
        for (int t = 0; t < n; t++) {
            float *q = Q + (size_t)t * ld, *kk = K + (size_t)t * ld, *vv = Vv + (size_t)t * ld;
            if (m->bq && m->bq[l]) for (int i = 0; i < qd; i++) q[i] += m->bq[l][i];
            if (m->bk && m->bk[l]) for (int i = 0; i < kvd; i++) kk[i] += m->bk[l][i];
            if (m->bv && m->bv[l]) for (int i = 0; i < kvd; i++) vv[i] += m->bv[l][i];
            or_rope(q, kk, rope_pos[t], nh, nkv, hd, 0, m->rope_theta);
            m->cache_len = att_pos[t];
            attention(m, q, kk, vv, AO + (size_t)t * ld, l, scores);
        }
        if (m->wo[l].data) {
            if (m->attn_o_inplace) {
                apply_mat_tokens_inplace(m, &m->wo[l], AO, ld, n, d, qd, A, xb);
            } else {
                apply_mat_tokens(m, &m->wo[l], AO, ld, n, Q, ld, d, qd, NULL, 0, 0.0f, A, xb);
                for (int t = 0; t < n; t++)
                    memcpy(AO + (size_t)t * ld, Q + (size_t)t * ld, sizeof(float) * (size_t)d);
            }
        }
        for (int t = 0; t < n; t++) {
            float *x = X + (size_t)t * ld, *xo = XO + (size_t)t * ld, *xn = XN + (size_t)t * ld;
            float *ao = AO + (size_t)t * ld;
            for (int i = 0; i < d; i++) x[i] = xo[i] + ao[i];
            memcpy(xo, x, sizeof(float) * (size_t)d);
            memcpy(xn, x, sizeof(float) * (size_t)d);
            apply_norm(xn, ntmp, m->ffn_norm ? m->ffn_norm[l] : NULL, d, ones);
        }
        apply_mat_tokens(m, &m->wg[l], XN, ld, n, G, ld, F, d, NULL, 0, 0.0f, A, xb);
        for (int t = 0; t < n; t++) or_silu(G + (size_t)t * ld, F);
        apply_mat_tokens(m, &m->wu[l], XN, ld, n, U, ld, F, d, G, ld, m->gate_thr, A, xb);
        for (int t = 0; t < n; t++) {
            float *g = G + (size_t)t * ld, *u = U + (size_t)t * ld, *xn = XN + (size_t)t * ld;
            int ti = t_base + t;
            if (m->gate_near || m->gate_near_idx) gate_log(m, g, F, ti, l);
            for (int f = 0; f < m->flip && f < OR_MAX_FLIPS; f++)
                if (m->flip_tok[f] == ti && m->flip_layer[f] == l && m->flip_col[f] >= 0 && m->flip_col[f] < F)
                    gate_flip(m, &m->wu[l], xn, g, u, F, d, T + (size_t)t * ld, m->flip_col[f]);
            for (int i = 0; i < F; i++) g[i] = g[i] * u[i];
        }
        apply_mat_tokens(m, &m->wd[l], G, ld, n, AO, ld, d, F, NULL, 0, 0.0f, A, xb);
        for (int t = 0; t < n; t++) {
            float *x = X + (size_t)t * ld, *xo = XO + (size_t)t * ld, *ao = AO + (size_t)t * ld;
            for (int i = 0; i < d; i++) x[i] = xo[i] + ao[i];
        }
    }
    m->cache_len = c;
    /* logits: every token, or the last one of the call */
    int t0 = all ? 0 : n - 1;
    if (!all && !logits) { free(rope_pos); free(att_pos); return 0; }
    int nl = n - t0;
    for (int t = t0; t < n; t++) {
        float *xf = XN + (size_t)t * ld;
        memcpy(xf, X + (size_t)t * ld, sizeof(float) * (size_t)d);
        if (m->has_out_norm) apply_norm(xf, ntmp, m->out_norm, d, ones);
    }
    for (int t = t0; t < n; t++) {
        float *lg = all ? logits + (size_t)(t_base + t) * V : logits;
        for (int i = 0; i < V; i++) lg[i] = -1e30f;
    }
    if (m->output.data) {
        int orows = m->output.rows;
        int ocols = m->output.cols > 0 ? m->output.cols : d;
        if (orows > 0 && orows <= V)
            apply_mat_tokens(m, &m->output, XN + (size_t)t0 * ld, ld, nl, all ? logits + (size_t)(t_base + t0) * V
                                                                              : logits,
                             V, orows, ocols, NULL, 0, 0.0f, A, xb);
    }
    free(rope_pos);
    free(att_pos);
    return 0;
}

static int forward_layers(or_model *m, const int *tokens, int n, float *logits, int all)
{
    int d = m->n_embd, hd = m->n_head_dim, nh = m->n_heads, F = m->n_ff;
    if (d <= 0 || d > 8192) return -4;
    if (n <= 0) return 0;
    int big = d > F ? d : F;
    if (nh * hd > big) big = nh * hd;
    size_t tmpn = 0;
    const or_mat *all_m[7];
    for (int l = 0; l < m->n_layers; l++) {
        all_m[0] = &m->wq[l]; all_m[1] = &m->wk[l]; all_m[2] = &m->wv[l]; all_m[3] = &m->wo[l];
        all_m[4] = &m->wg[l]; all_m[5] = &m->wu[l]; all_m[6] = &m->wd[l];
        for (int i = 0; i < 7; i++)
            if (all_m[i]->data) {
                size_t e = (size_t)all_m[i]->rows * all_m[i]->cols;
                if (e > tmpn) tmpn = e;
            }
    }
    if (m->output.data && (size_t)m->output.rows * m->output.cols > tmpn)
        tmpn = (size_t)m->output.rows * m->output.cols;
    if ((size_t)(m->tok_embd.cols + 32) > tmpn) tmpn = (size_t)m->tok_embd.cols + 32;
    int max_ctx = m->n_ctx < 1 ? 4096 : m->n_ctx;
    int chunk = n < OR_CHUNK ? n : OR_CHUNK;
    size_t ld = (size_t)big + 8;
    float *A = (float *)malloc(sizeof(float) * (tmpn + 64));
    float *xb = (float *)aligned_alloc(64, sizeof(float) * (size_t)((chunk + OR_LANES - 1) / OR_LANES) *
                                               OR_LANES * ld);
    float *wk = (float *)calloc(11 * (size_t)chunk * ld + 2 * ld + (size_t)nh * (size_t)(max_ctx + 8),
                                sizeof(float));
    int rc = (A && xb && wk) ? 0 : -3;
    for (int t0 = 0; t0 < n && rc == 0; t0 += chunk) {
        int nc = n - t0 < chunk ? n - t0 : chunk;
        int last = t0 + nc == n;
        rc = forward_chunk(m, tokens + t0, nc, t0, all ? logits : (last ? logits : NULL), all, A, xb, wk);
    }
    free(A);
    free(xb);
    free(wk);
    return rc;
}

int or_forward(or_model *m, const int *tokens, int n, float *logits)
{
    if (m->q4_mode == OR_Q4_AVX2LANES) return forward_impl(m, tokens, n, logits, 0);
    return forward_layers(m, tokens, n, logits, 0);
}

int or_forward_all(or_model *m, const int *tokens, int n, float *logits_all)
{
    if (m->q4_mode == OR_Q4_AVX2LANES) return forward_impl(m, tokens, n, logits_all, 1);
    return forward_layers(m, tokens, n, logits_all, 1);
}

int or_forward_tokenwise(or_model *m, const int *tokens, int n, float *logits, int all)
{
    return forward_impl(m, tokens, n, logits, all);
}

/* ===================================================================== */
/* acceptance                                                             */
/* ===================================================================== */

/* First index of the maximum, strict '>' (src/speculative.c:93-98). */
int or_argmax(const float *x, int n)
{
    int best = 0;
    for (int i = 1; i < n; i++) if (x[i] > x[best]) best = i;
    return best;
}

/* p_i = exp((l_i - max)/T) / (sum + 1e-30) (src/speculative.c:44-53). */
void or_softmax_temp(const float *l, int n, float T, float *p)
{
    float mx = l[0];
    for (int i = 1; i < n; i++) if (l[i] > mx) mx = l[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) { p[i] = expf((l[i] - mx) / T); sum = sum + p[i]; }
    float inv = 1.0f / (sum + 1e-30f);
    for (int i = 0; i < n; i++) p[i] = p[i] * inv;
}

static uint64_t fixed32(float w)
{
    if (!(w > 0.0f)) return 0;
    return (uint64_t)((double)w * 4294967296.0 + 0.5);
}

/* First v whose fixed-point prefix sum reaches max(1, ceil(U*S/2^24)). */
int or_inverse_cdf_fixed(const float *w, int n, float u)
{
    uint64_t S = 0;
    for (int v = 0; v < n; v++) S += fixed32(w[v]);
    if (S == 0) return -1;
    uint64_t U = (uint64_t)(u * 16777216.0f);
    uint64_t thr = (U * S + 16777215ull) >> 24;
    if (thr == 0) thr = 1;                 /* never land on a zero-mass token */
    uint64_t c = 0;
    for (int v = 0; v < n; v++) {
        c += fixed32(w[v]);
        if (c >= thr) return v;
    }
    return n - 1;
}

typedef struct { float p; int i; } or_pi;
static int cmp_desc(const void *a, const void *b)
{
    const or_pi *x = (const or_pi *)a, *y = (const or_pi *)b;
    if (x->p > y->p) return -1;
    if (x->p < y->p) return 1;
    return x->i - y->i;
}

/* Nucleus sampling (src/speculative.c:35-91): T <= 0 -> argmax.  Otherwise the
 * nucleus is the shortest prefix of tokens sorted by descending probability
 * (ties: lower index first) whose fixed-point mass reaches top_p (all tokens
 * when top_p >= 1); the draw is the fixed-point inverse CDF of u over the
 * nucleus in index order.  q_out (optional) receives the renormalised
 * nucleus distribution p_v / mass. */
int or_sample_top_p(const float *l, int n, float T, float top_p, float u, float *q_out)
{
    if (T <= 0.0f) {
        int a = or_argmax(l, n);
        if (q_out) { for (int i = 0; i < n; i++) q_out[i] = 0.0f; q_out[a] = 1.0f; }
        return a;
    }
    float *p = (float *)malloc(sizeof(float) * (size_t)n);
    float *w = (float *)malloc(sizeof(float) * (size_t)n);
    or_softmax_temp(l, n, T, p);
    if (top_p >= 1.0f) {
        memcpy(w, p, sizeof(float) * (size_t)n);
    } else {
        or_pi *s = (or_pi *)malloc(sizeof(or_pi) * (size_t)n);
        for (int i = 0; i < n; i++) { s[i].p = p[i]; s[i].i = i; }
        qsort(s, (size_t)n, sizeof(or_pi), cmp_desc);
        /* top_p <= 0: the first sorted token alone (src/speculative.c:67-74) */
        uint64_t TP = top_p > 0.0f ? (uint64_t)ceil((double)top_p * 4294967296.0) : 0;
        uint64_t c = 0;
        int cut = n;
        for (int r = 0; r < n; r++) {
            c += fixed32(s[r].p);
            if (c >= TP) { cut = r + 1; break; }
        }
        for (int i = 0; i < n; i++) w[i] = 0.0f;
        for (int r = 0; r < cut; r++) w[s[r].i] = s[r].p;
        free(s);
    }
    int tok = or_inverse_cdf_fixed(w, n, u);
    if (tok < 0) tok = or_argmax(p, n);
    if (q_out) {
        uint64_t S = 0;
        for (int i = 0; i < n; i++) S += fixed32(w[i]);
        float mass = (float)((double)S / 4294967296.0);
        for (int i = 0; i < n; i++) q_out[i] = w[i] > 0.0f ? w[i] / mass : 0.0f;
    }
    free(p);
    free(w);
    return tok;
}

/* Greedy verify: accept d_j iff it is the first-max of L_j; on the first
 * mismatch emit argmax(L_j); after k accepts emit argmax(L_k).  Returns the
 * number of emitted tokens (accepted + 1). */
int or_accept_greedy(const float *L, int V, const int *draft, int k, int *out)
{
    for (int j = 0; j < k; j++) {
        int a = or_argmax(L + (size_t)j * V, V);
        out[j] = a;
        if (a != draft[j]) return j + 1;
    }
    out[k] = or_argmax(L + (size_t)k * V, V);
    return k + 1;
}

/* Sampled verify (ratio test and residual resample of
 * src/speculative.c:186-233 on softmax(L/T) probabilities):
 * accept d_j iff u_j < min(1, p_j(d_j)/max(q_j(d_j), 1e-10)); on the first
 * reject resample from max(0, p_j - q_j) with u_k (argmax of the residual
 * when its mass is zero); after k accepts sample the bonus token from p_k
 * with u_k.  Q holds k rows of the draft distributions (Vd wide). */
int or_accept_sampled(const float *L, int V, const float *Q, int Vd, const int *draft, int k,
                      float T, const float *u, int *out, int *n_accepted)
{
    float *p = (float *)malloc(sizeof(float) * (size_t)V);
    for (int j = 0; j < k; j++) {
        or_softmax_temp(L + (size_t)j * V, V, T, p);
        const float *q = Q + (size_t)j * Vd;
        int dj = draft[j];
        float pt = (dj >= 0 && dj < V) ? p[dj] : 0.0f;
        float qd = (dj >= 0 && dj < Vd) ? q[dj] : 0.0f;
        float alpha = fminf(1.0f, pt / fmaxf(qd, 1e-10f));
        if (u[j] < alpha) { out[j] = dj; continue; }
        for (int v = 0; v < V; v++) {
            float qv = v < Vd ? q[v] : 0.0f;
            p[v] = fmaxf(0.0f, p[v] - qv);
        }
        int t = or_inverse_cdf_fixed(p, V, u[k]);
        if (t < 0) t = or_argmax(p, V);
        out[j] = t;
        *n_accepted = j;
        free(p);
        return j + 1;
    }
    or_softmax_temp(L + (size_t)k * V, V, T, p);
    int t = or_inverse_cdf_fixed(p, V, u[k]);
    if (t < 0) t = or_argmax(p, V);
    out[k] = t;
    *n_accepted = k;
    free(p);
    return k + 1;
}
