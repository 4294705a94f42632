/*
 * quantize.c -- the quantize.h API (reference include/quantize.h:94-139).
 *
 * Format helpers (fp16 conversion, the Q4_0 writer, sizes) are host bit
 * manipulation.  Everything that computes over a matrix -- dequantize, dot,
 * GEMV, GEMM -- uploads the blocks once per call and runs the GPU kernels of
 * vxh.h; results come back to host memory before the call returns.  The void
 * entry points have no error channel in the reference; on failure they fill
 * the output with NaN and report through vx_last_error() and stderr.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "vx_host.h"

static float g_wscale = 1.0f;

void vx_set_synthetic_weight_scale(float scale) { g_wscale = scale; }
float vx_get_synthetic_weight_scale(void) { return g_wscale; }

/* Truncating float -> half, flush-to-zero below the half normal range
 * (src/quantize.c:17-35). */
uint16_t vx_fp32_to_fp16(float f)
{
    uint32_t b;
    memcpy(&b, &f, 4);
    uint16_t sign = (uint16_t)((b >> 31) << 15);
    uint32_t e = (b >> 23) & 0xffu, mant = b & 0x7fffffu;
    if (e == 0) return sign;
    if (e == 0xff) return (uint16_t)(sign | 0x7c00u | (mant >> 13));
    int he = (int)e - 112;
    if (he <= 0) return sign;
    if (he >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)he << 10) | (mant >> 13));
}

/* Exact half -> float (src/quantize.c:37-57). */
float vx_fp16_to_fp32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15) & 1u, e = (uint32_t)(h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 31) {
        uint32_t b = (sign << 31) | (0xffu << 23) | (m << 13);
        float f;
        memcpy(&f, &b, 4);
        return f;
    }
    float v = e ? ldexpf((float)(m | 0x400u), (int)e - 25) : ldexpf((float)m, -24);
    return sign ? -v : v;
}

size_t vx_quantized_size(int n, vx_type type)
{
    int bs = (type >= VX_TYPE_Q2_K && type <= VX_TYPE_Q8_K) ? 256 : 32;
    size_t nb = (size_t)((n + bs - 1) / bs);
    switch (type) {
    case VX_TYPE_Q4_0: return nb * 18;
    case VX_TYPE_Q4_1: return nb * 20;
    case VX_TYPE_Q5_0: return nb * 22;
    case VX_TYPE_Q5_1: return nb * 24;
    case VX_TYPE_Q8_0: return nb * 34;
    case VX_TYPE_Q8_1: return nb * 40;
    case VX_TYPE_Q2_K: return nb * 84;
    case VX_TYPE_Q3_K: return nb * 110;
    case VX_TYPE_Q4_K: return nb * 144;
    case VX_TYPE_Q5_K: return nb * 176;
    case VX_TYPE_Q6_K: return nb * 210;
    case VX_TYPE_Q8_K: return nb * 292;
    default: return (size_t)n * 4;
    }
}

/* Q4_0 writer (src/quantize.c:88-114): d = amax/7 floored at 1e-10 and stored
 * truncated to half; q = trunc(x * (1/d)) with the unrounded d, clamped to
 * [-8, 7], + 8; element 2j in the low nibble of qs[j]. */
void vx_quantize_row_q4_0(const float *x, void *vy, int n)
{
    block_q4_0 *y = (block_q4_0 *)vy;
    for (int base = 0; base < n; base += 32) {
        int rem = n - base < 32 ? n - base : 32;
        float amax = 0.0f;
        for (int j = 0; j < rem; j++) amax = fabsf(x[base + j]) > amax ? fabsf(x[base + j]) : amax;
        float d = amax / 7.0f;
        if (d < 1e-10f) d = 1e-10f;
        block_q4_0 *b = &y[base / 32];
        b->d = vx_fp32_to_fp16(d);
        float inv = 1.0f / d;
        memset(b->qs, 0, sizeof(b->qs));
        for (int j = 0; j < rem; j += 2) {
            int a0 = (int)(x[base + j] * inv);
            int a1 = j + 1 < rem ? (int)(x[base + j + 1] * inv) : 0;
            a0 = a0 < -8 ? -8 : (a0 > 7 ? 7 : a0);
            a1 = a1 < -8 ? -8 : (a1 > 7 ? 7 : a1);
            b->qs[j / 2] = (uint8_t)((a0 + 8) | ((a1 + 8) << 4));
        }
    }
}

/* --------------------------------------------------------------------------- */
/* GPU-backed operations                                                        */
/* --------------------------------------------------------------------------- */
typedef struct {
    int ready;
    vxh_stream s;
    vxh_workspace ws;
    vxh_panel pan;
    int pan_K;
    float *x, *y, *g, *tail;
    size_t x_cap, y_cap, g_cap;
    int *ids;
} op_ctx;

static op_ctx g_op;

static int op_init(void)
{
    if (g_op.ready) return VXH_OK;
    int rc = vx_gpu_ready();
    if (rc) return rc;
    if ((rc = vxh_stream_create(&g_op.s))) return rc;
    if ((rc = vxh_malloc((void **)&g_op.tail, sizeof(float) * VX_MAX_BATCH * 4))) return rc;
    if ((rc = vxh_malloc((void **)&g_op.ids, sizeof(int) * 4))) return rc;
    g_op.ready = 1;
    return VXH_OK;
}

static int grow(float **p, size_t *cap, size_t n)
{
    if (*cap >= n) return VXH_OK;
    vxh_free(*p);
    *p = NULL;
    *cap = 0;
    int rc = vxh_malloc((void **)p, n * sizeof(float));
    if (rc == VXH_OK) *cap = n;
    return rc;
}

static int op_panel(int K)
{
    if (g_op.pan.data && g_op.pan_K == K) return VXH_OK;
    vxh_panel_free(&g_op.pan);
    g_op.pan_K = 0;
    int rc = vxh_panel_alloc(&g_op.pan, VX_MAX_BATCH, K);
    if (rc == VXH_OK) g_op.pan_K = K;
    return rc;
}

static int op_workspace(int rows)
{
    size_t n = vxh_gemm_workspace_elems(rows, VX_MAX_BATCH);
    if (g_op.ws.acc && g_op.ws.acc_elems >= n) return VXH_OK;
    vxh_workspace_free(&g_op.ws);
    return vxh_workspace_alloc(&g_op.ws, n, 32);
}

static void report(const char *what, int rc)
{
    vx_from_vxh(rc);
    fprintf(stderr, "veltrix-amd: %s failed: %s\n", what, vx_last_error());
}

static void fill_nan(float *y, size_t n)
{
    for (size_t i = 0; i < n; i++) y[i] = NAN;
}

/* Core of every matrix entry point: Y[M][rows] (ldy) = X . A^T.
 * kind = VXH_EPI_STORE or VXH_EPI_GATE (gate[rows], same for every row). */
static int run_gemm(int type, const void *A, const float *X, int ldx, float *Y, int ldy, int M,
                    int rows, int cols, int avx2, const float *gate, float thr, float scale)
{
    int rc = op_init();
    if (rc) return rc;
    if (rows <= 0 || M <= 0) return VXH_OK;
    if (cols <= 0) return vxh_set_error(VXH_ERR_PARAM, "cols %d", cols);
    if (avx2 && cols % 32) return vxh_set_error(VXH_ERR_PARAM, "the lane pattern needs cols %% 32 == 0");
    int K = (cols + 31) / 32 * 32;
    vxh_qmat W;
    if ((rc = vxh_qmat_alloc(&W, type, rows, K))) return rc;
    if ((rc = vxh_qmat_set_rows(&W, A, 0, rows, rows, 0, 0, g_op.s))) goto out;
    if ((rc = op_panel(K)) || (rc = op_workspace(rows))) goto out;
    if ((rc = grow(&g_op.x, &g_op.x_cap, (size_t)VX_MAX_BATCH * K))) goto out;
    if ((rc = grow(&g_op.y, &g_op.y_cap, (size_t)VX_MAX_BATCH * rows))) goto out;
    if (gate) {
        if ((rc = grow(&g_op.g, &g_op.g_cap, (size_t)VX_MAX_BATCH * rows))) goto out;
    }
    for (int m0 = 0; m0 < M; m0 += VX_MAX_BATCH) {
        int mb = M - m0 < VX_MAX_BATCH ? M - m0 : VX_MAX_BATCH;
        /* rows padded with zeros to K; lane-pattern tails are the 4 floats
         * after each row, as the x86 kernel reads them */
        float *hx = (float *)calloc((size_t)mb * K, sizeof(float));
        float *ht = (float *)calloc((size_t)mb * 4, sizeof(float));
        if (!hx || !ht) { free(hx); free(ht); rc = vxh_set_error(VXH_ERR_ALLOC, "host buffer"); goto out; }
        for (int m = 0; m < mb; m++) {
            memcpy(hx + (size_t)m * K, X + (size_t)(m0 + m) * ldx, sizeof(float) * (size_t)cols);
            if (avx2) memcpy(ht + (size_t)m * 4, X + (size_t)(m0 + m) * ldx + cols, 4 * sizeof(float));
        }
        rc = vxh_upload(g_op.x, hx, sizeof(float) * (size_t)mb * K, g_op.s);
        if (!rc && avx2) rc = vxh_upload(g_op.tail, ht, sizeof(float) * (size_t)mb * 4, g_op.s);
        free(hx);
        free(ht);
        if (rc) goto out;
        if (gate) {
            for (int m = 0; m < mb; m++)
                if ((rc = vxh_upload(g_op.g + (size_t)m * rows, gate, sizeof(float) * (size_t)rows, g_op.s)))
                    goto out;
        }
        if ((rc = vxh_prep_panel(&g_op.pan, g_op.x, K, mb, K, avx2, avx2 ? g_op.tail : NULL, 4, g_op.s)))
            goto out;
        vxh_epilogue ep = {gate ? VXH_EPI_GATE : VXH_EPI_STORE, g_op.y, rows, gate ? g_op.g : NULL, rows,
                           thr, scale, rows};
        if ((rc = vxh_gemm(&W, &g_op.pan, mb, &ep, &g_op.ws, VXH_PATH_AUTO, g_op.s))) goto out;
        float *hy = (float *)malloc(sizeof(float) * (size_t)mb * rows);
        if (!hy) { rc = vxh_set_error(VXH_ERR_ALLOC, "host buffer"); goto out; }
        rc = vxh_download(hy, g_op.y, sizeof(float) * (size_t)mb * rows, g_op.s);
        if (!rc)
            for (int m = 0; m < mb; m++)
                memcpy(Y + (size_t)(m0 + m) * ldy, hy + (size_t)m * rows, sizeof(float) * (size_t)rows);
        free(hy);
        if (rc) goto out;
    }
out:
    vxh_stream_sync(g_op.s);
    /* a failed call may leave part of a GEMM in the accumulator */
    if (rc && g_op.ws.acc) {
        vxh_fill_f32((float *)g_op.ws.acc, 0.0f, 2 * g_op.ws.acc_elems, g_op.s);
        vxh_stream_sync(g_op.s);
    }
    vxh_qmat_free(&W);
    return rc;
}

void vx_gemv_q4_0(const void *restrict A, const float *restrict x, float *restrict y, int rows, int cols)
{
    int rc = run_gemm(VX_TYPE_Q4_0, A, x, cols, y, rows, 1, rows, cols, 0, NULL, 0.0f, 1.0f);
    if (rc) { report("vx_gemv_q4_0", rc); fill_nan(y, (size_t)(rows > 0 ? rows : 0)); }
}

void vx_gemv_q4_0_sparse_rows(const void *restrict A, const float *restrict x, float *restrict y,
                              int rows, int cols, const float *restrict gate, float threshold)
{
    int rc = run_gemm(VX_TYPE_Q4_0, A, x, cols, y, rows, 1, rows, cols, 0, gate, threshold, 1.0f);
    if (rc) { report("vx_gemv_q4_0_sparse_rows", rc); fill_nan(y, (size_t)(rows > 0 ? rows : 0)); }
}

void vx_gemv_q4_0_avx2(const void *A, const float *x, float *y, int rows, int cols)
{
    int rc = run_gemm(VX_TYPE_Q4_0, A, x, cols, y, rows, 1, rows, cols, 1, NULL, 0.0f, 1.0f);
    if (rc) { report("vx_gemv_q4_0_avx2", rc); fill_nan(y, (size_t)(rows > 0 ? rows : 0)); }
}

void vx_gemv_q4_0_avx2_sparse_rows(const void *A, const float *x, float *y, int rows, int cols,
                                   const float *gate, float threshold)
{
    int rc = run_gemm(VX_TYPE_Q4_0, A, x, cols, y, rows, 1, rows, cols, 1, gate, threshold, 1.0f);
    if (rc) { report("vx_gemv_q4_0_avx2_sparse_rows", rc); fill_nan(y, (size_t)(rows > 0 ? rows : 0)); }
}

void vx_dot_q4_0(const void *x, const float *y, float *dst, int n)
{
    int rc = run_gemm(VX_TYPE_Q4_0, x, y, n, dst, 1, 1, 1, n, 0, NULL, 0.0f, 1.0f);
    if (rc) { report("vx_dot_q4_0", rc); *dst = NAN; }
}

vx_error vx_gemm_q4_0(const void *A, const float *X, int ldx, float *Y, int M, int rows, int cols, int flags)
{
    if (!A || !X || !Y) return VX_ERR_PARAM;
    int avx2 = (flags & VX_GEMM_AVX2_LANES) != 0;
    if (ldx < cols + (avx2 ? 4 : 0)) return VX_ERR_PARAM;
    int rc = run_gemm(VX_TYPE_Q4_0, A, X, ldx, Y, rows, M, rows, cols, avx2, NULL, 0.0f, 1.0f);
    return vx_from_vxh(rc);
}

vx_error vx_gemm_q8_0(const void *A, const float *X, int ldx, float *Y, int M, int rows, int cols)
{
    if (!A || !X || !Y || ldx < cols) return VX_ERR_PARAM;
    /* the reference dequantizes Q8_0 (applying the synthetic scale) and runs
     * an f32 GEMV (src/model.c:234-244) */
    int rc = run_gemm(VX_TYPE_Q8_0, A, X, ldx, Y, rows, M, rows, cols, 0, NULL, 0.0f, g_wscale);
    return vx_from_vxh(rc);
}

static int run_dequant(int type, const void *x, float *y, int n)
{
    int rc = op_init();
    if (rc) return rc;
    if (n <= 0) return VXH_OK;
    int K = (n + 31) / 32 * 32;
    vxh_qmat W;
    if ((rc = vxh_qmat_alloc(&W, type, 1, K))) return rc;
    int zero = 0;
    if ((rc = vxh_qmat_set_rows(&W, x, 0, 1, 1, 0, 0, g_op.s))) goto out;
    if ((rc = grow(&g_op.x, &g_op.x_cap, (size_t)K))) goto out;
    if ((rc = vxh_upload(g_op.ids, &zero, sizeof(int), g_op.s))) goto out;
    if ((rc = vxh_qmat_gather_rows(&W, g_op.ids, 1, g_wscale, g_op.x, K, g_op.s))) goto out;
    rc = vxh_download(y, g_op.x, sizeof(float) * (size_t)n, g_op.s);
out:
    vxh_stream_sync(g_op.s);
    /* a failed call may leave part of a GEMM in the accumulator */
    if (rc && g_op.ws.acc) {
        vxh_fill_f32((float *)g_op.ws.acc, 0.0f, 2 * g_op.ws.acc_elems, g_op.s);
        vxh_stream_sync(g_op.s);
    }
    vxh_qmat_free(&W);
    return rc;
}

void vx_dequantize_row_q4_0(const void *x, float *y, int n)
{
    int rc = run_dequant(VX_TYPE_Q4_0, x, y, n);
    if (rc) { report("vx_dequantize_row_q4_0", rc); fill_nan(y, (size_t)(n > 0 ? n : 0)); }
}

void vx_dequantize_row_q8_0(const void *x, float *y, int n)
{
    int rc = run_dequant(VX_TYPE_Q8_0, x, y, n);
    if (rc) { report("vx_dequantize_row_q8_0", rc); fill_nan(y, (size_t)(n > 0 ? n : 0)); }
}
