// GEMM whose workgroups build their own K slice of the activation panel
// (vxh_gemm_pro): the residual add, RMSNorm weight, SwiGLU and the panel
// conversion of the forward (src/model.c:514-594) run inside the GEMM that
// consumes them instead of in a row kernel of their own, and the RMSNorm's
// 1/rms is applied to the product by its consumer; or the attention combine
// runs inside the output projection.  The residual and SwiGLU kinds have
// translation units of their own (vxh_pro_resid.hip, vxh_pro_swiglu.hip) so
// that the template instances compile in parallel.
#include "vxh_gemm_core.h"

int vx_gemm_pro_resid(const vxh_qmat *W, int M, vx_gemm_args &a, hipStream_t st, hipEvent_t e0,
                      hipEvent_t e1);
int vx_gemm_pro_swiglu(const vxh_qmat *W, int M, vx_gemm_args &a, hipStream_t st, hipEvent_t e0,
                       hipEvent_t e1);

static bool vx_overlap(const void *a, size_t an, const void *b, size_t bn)
{
    if (!a || !b || !an || !bn) return false;
    const char *pa = (const char *)a, *pb = (const char *)b;
    return pa < pb + bn && pb < pa + an;
}

static bool vx_al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// Whether M strided rows [a + m*lda, + na) and M rows [b + m*ldb, + nb) of
// doubles share an element (rows of two buffers may interleave: the decode
// forward's per-layer accumulators put every layer's rows side by side).
static bool vx_overlap_rows(const double *a, size_t lda, size_t na, const double *b, size_t ldb, size_t nb, int M)
{
    if (!a || !b || !na || !nb) return false;
    for (int i = 0; i < M; i++)
        for (int j = 0; j < M; j++)
            if (vx_overlap(a + (size_t)i * lda, na * sizeof(double), b + (size_t)j * ldb, nb * sizeof(double)))
                return true;
    return false;
}

extern "C" int vxh_gemm_pro(const vxh_qmat *W, int M, const vxh_pro *p, double *acc, int ld_acc,
                            int n_out, float scale, vxh_event start, vxh_event stop, vxh_stream s)
{
    if (!W || !p || M < 1 || M > 16)
        return vxh_fail(VXH_ERR_PARAM, "gemm_pro: M %d", M);
    const int K = W->n_cols;
    if (n_out < 0 || n_out > W->n_rows || (n_out > ld_acc && M > 1))
        return vxh_fail(VXH_ERR_PARAM, "gemm_pro: n_out %d (rows %d, ld %d)", n_out, W->n_rows, ld_acc);
    const size_t acc_bytes = ((size_t)(M - 1) * ld_acc + n_out) * sizeof(double);
    switch (p->kind) {
    case VXH_PRO_ROWS:
    case VXH_PRO_RESID: {
        const bool resid = p->kind == VXH_PRO_RESID;
        if (!p->x || p->ldx < K || p->ldx % 4 || !vx_al16(p->x) || (p->w && !vx_al16(p->w)))
            return vxh_fail(VXH_ERR_PARAM, "gemm_pro: rows x (ld %d, K %d) must be 16-byte aligned", p->ldx, K);
        if (resid && (!p->src || p->ld_src < K || p->ld_src % 2 || !vx_al16(p->src)))
            return vxh_fail(VXH_ERR_PARAM, "gemm_pro: residual sums (ld %d, K %d)", p->ld_src, K);
        if (resid && p->x_out) {
            if (p->ld_xout < K || p->ld_xout % 4 || !vx_al16(p->x_out))
                return vxh_fail(VXH_ERR_PARAM, "gemm_pro: x_out (ld %d, K %d)", p->ld_xout, K);
            if (vx_overlap(p->x, ((size_t)(M - 1) * p->ldx + K) * 4, p->x_out,
                           ((size_t)(M - 1) * p->ld_xout + K) * 4))
                return vxh_fail(VXH_ERR_PARAM, "gemm_pro: x_out overlaps x");
        }
        break;
    }
    case VXH_PRO_ATTN:
        if (M > VX_PRO_ATTN_MAX_M || !p->part || p->n_chunks < 1 || p->n_kv_heads < 1 || p->head_dim < 4 ||
            p->head_dim % 4 || p->n_heads % p->n_kv_heads || p->n_heads * p->head_dim != K)
            return vxh_fail(VXH_ERR_PARAM, "gemm_pro: attention slice (M %d, %d heads of %d, K %d)", M,
                            p->n_heads, p->head_dim, K);
        break;
    case VXH_PRO_SWIGLU: {
        const int phys = (K + 15) / 16 * 32;
        if (!p->src || p->ld_src < phys || p->ld_src % 2 || !vx_al16(p->src))
            return vxh_fail(VXH_ERR_PARAM, "gemm_pro: gate/up sums (ld %d, need %d)", p->ld_src, phys);
        if (p->ss_in && p->ss_K < 1) return vxh_fail(VXH_ERR_PARAM, "gemm_pro: norm length %d", p->ss_K);
        break;
    }
    default:
        return vxh_fail(VXH_ERR_PARAM, "gemm_pro: kind %d", p->kind);
    }
    if (p->n_clear && !p->clear) return vxh_fail(VXH_ERR_PARAM, "gemm_pro: clear range without a pointer");
    if (p->src) {
        const size_t src_n = p->kind == VXH_PRO_SWIGLU ? (K + 15) / 16 * 32 : K;
        if (vx_overlap_rows(acc, M > 1 ? ld_acc : 0, n_out, p->src, p->ld_src, src_n, M))
            return vxh_fail(VXH_ERR_PARAM, "gemm_pro: acc overlaps the source sums");
    }
    if (vx_overlap(acc, acc_bytes, p->clear, p->n_clear * sizeof(double)))
        return vxh_fail(VXH_ERR_PARAM, "gemm_pro: acc overlaps the clear range");
    if (n_out == 0 && !p->n_clear && !p->ss && !p->x_out) return VXH_OK;

    vx_gemm_args a;
    memset(&a, 0, sizeof(a));
    a.wq = (const uint4 *)W->qs;
    a.wcache = W->cached;
    a.wd = (const uint32_t *)W->d;
    a.rs_ld = 1;
    a.rs_chunk = 1 << 30;
    a.acc = acc;
    a.ld_acc = ld_acc;
    a.n_out = n_out;
    a.scale = scale;
    a.p.x = p->x;
    a.p.ldx = p->ldx;
    a.p.src = p->src;
    a.p.ld_src = p->ld_src;
    a.p.w = p->w;
    a.p.x_out = p->kind == VXH_PRO_RESID ? p->x_out : nullptr;
    a.p.ld_xout = p->ld_xout;
    a.p.ss = p->kind == VXH_PRO_SWIGLU ? nullptr : p->ss;
    a.p.ss_in = p->kind == VXH_PRO_SWIGLU ? p->ss_in : nullptr;
    a.p.ss_K = p->ss_K;
    a.p.thr = p->thr;
    a.p.K = K;
    a.p.clr = p->n_clear ? p->clear : nullptr;
    a.p.n_clr = (long)p->n_clear;
    if (p->kind == VXH_PRO_ATTN) {
        a.p.part = p->part;
        a.p.n_chunks = p->n_chunks;
        a.p.G = p->n_heads / p->n_kv_heads;
        a.p.hd = p->head_dim;
    }
    hipStream_t st = vxh_hs(s);
    hipEvent_t e0 = (hipEvent_t)start, e1 = (hipEvent_t)stop;
    switch (p->kind) {
    case VXH_PRO_ROWS: return vx_dispatch<VX_PRO_ROWS>(W, M, 0, a, st, e0, e1);
    case VXH_PRO_RESID: return vx_gemm_pro_resid(W, M, a, st, e0, e1);
    case VXH_PRO_ATTN:
        if (M == 1) return vx_dispatch_m<1, VX_PRO_ATTN>(W, 0, a, st, e0, e1);
        return vx_dispatch_m<2, VX_PRO_ATTN>(W, 0, a, st, e0, e1);
    default: return vx_gemm_pro_swiglu(W, M, a, st, e0, e1);
    }
}

__global__ void vx_acc_store_norm_kernel(double *__restrict__ acc, int ld_acc, int n,
                                         float *__restrict__ y, int ldy, const double *__restrict__ ss,
                                         int ss_K)
{
    const int m = blockIdx.y;
    const float rin = vx_rms_inv((float)ss[m], ss_K);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        double *p = acc + (size_t)m * ld_acc + i;
        const float v = (float)*p;
        *p = 0.0;
        y[(size_t)m * ldy + i] = v * rin;
    }
}

extern "C" int vxh_acc_store_norm(double *acc, int ld_acc, int M, int n, float *y, int ldy,
                                  const double *ss, int ss_K, vxh_stream s)
{
    if (M <= 0 || n <= 0) return VXH_OK;
    if (!ss || ss_K < 1) return vxh_fail(VXH_ERR_PARAM, "acc_store_norm: ss %p K %d", (const void *)ss, ss_K);
    int gx = (n + 255) / 256;
    if (gx > 256) gx = 256;
    vx_acc_store_norm_kernel<<<dim3(gx, M), 256, 0, vxh_hs(s)>>>(acc, ld_acc, n, y, ldy, ss, ss_K);
    VXH_LAUNCHED();
    return VXH_OK;
}
