// Skinny-M dequant GEMM for GGUF Q4_0 / Q8_0 weights on gfx950, and the
// row kernels that build its activation panels.
//
//   acc[m][n] += scale * sum_k X[m][k] * W[n][k],  1 <= M <= 16
//
// MFMA path: v_mfma_f32_32x32x16_f16 with the activations as the A operand
// (32 rows: rows m as fp16 hi parts in slots 0..M-1, lo parts in M..2M-1)
// and 32 weight rows as the B operand.  Weights are exact small integers in
// fp16 (s-8 for Q4_0, q for Q8_0) unpacked in registers from the tiled
// nibble/byte plane; one Q4_0/Q8_0 block is exactly K=32 = two MFMAs, after
// which the 32x32 block product is scaled by the block's fp16 scale d and
// accumulated in fp32.  x = hi + lo carries 22 significant bits, so the
// products match fp32 arithmetic to ~1e-7 relative.
//
// Work split: a workgroup is 4 wavefronts = 4 tiles of 32 weight rows that
// share one K slice of PPW block pairs.  Each wavefront keeps RING pairs of
// weight loads in flight.  The K slices of a tile (split-K) are summed with
// fp64 atomic adds into an fp64 accumulator: a handful of fp32 partials add
// exactly in fp64, so the result does not depend on their arrival order and
// no workgroup waits for another.  Consumers read the accumulator and clear
// it (vxh_acc_*, the residual/SwiGLU panels, RoPE), so it is all zeros again
// before the next GEMM that targets it.
#include "vxh_gemm_core.h"

// ---------------------------------------------------------------------------
// panels
// ---------------------------------------------------------------------------
extern "C" size_t vxh_panel_bytes(int M, int K)
{
    int nb = (K / 32 + 1) / 2 * 2;   // blocks padded to an even count
    return (size_t)nb * vxh_panel_units_per_block(M) * 16;
}

extern "C" int vxh_panel_alloc(vxh_panel *p, int max_M, int K)
{
    p->data = nullptr;
    p->corr = nullptr;
    p->xs = nullptr;
    p->rscale = nullptr;
    p->M = 0;
    p->K = K;
    p->avx2 = 0;
    p->rs_ld = 0;
    if (max_M < 1 || max_M > 16 || K % 32 || K > VXH_MAX_K)
        return vxh_fail(VXH_ERR_PARAM, "panel_alloc: M %d K %d", max_M, K);
    int rc = vxh_malloc(&p->data, vxh_panel_bytes(max_M, K));
    if (rc) return rc;
    int nb = (K / 32 + 1) / 2 * 2;
    rc = vxh_malloc((void **)&p->corr, (size_t)nb * max_M * sizeof(float));
    if (rc) return rc;
    rc = vxh_malloc((void **)&p->rscale, (size_t)16 * ((K + VX_CHUNK - 1) / VX_CHUNK) * sizeof(float));
    if (rc) return rc;
    // padded blocks must read as zeros
    VXH_CHECK(hipMemset(p->data, 0, vxh_panel_bytes(max_M, K)));
    VXH_CHECK(hipMemset(p->corr, 0, (size_t)nb * max_M * sizeof(float)));
    VXH_CHECK(hipDeviceSynchronize());
    return VXH_OK;
}

extern "C" int vxh_panel_free(vxh_panel *p)
{
    vxh_free(p->data);
    vxh_free(p->corr);
    vxh_free(p->xs);
    vxh_free(p->rscale);
    p->data = nullptr;
    p->corr = nullptr;
    p->xs = nullptr;
    p->rscale = nullptr;
    return VXH_OK;
}

// ---------------------------------------------------------------------------
// row kernels: one 1024-thread workgroup per row; every thread first loads
// the groups of 8 elements it owns (so a row costs one memory round trip),
// then the row reductions run in registers and LDS.
// ---------------------------------------------------------------------------
#define VX_ROW_THREADS 1024

enum { VX_ROW_PLAIN = 0, VX_ROW_NORM = 1, VX_ROW_RESID_NORM = 2, VX_ROW_SWIGLU = 3 };

struct vx_row_args {
    float *x;            // PLAIN/NORM: input rows; RESID_NORM: residual rows (updated in place)
    int ldx;
    double *acc;         // RESID_NORM: pending GEMM sum added to x; SWIGLU: gate/up accumulator
    int ld_acc;
    int K;               // row length (F for SWIGLU)
    const float *w;      // norm weight (NULL = ones)
    int avx2;
    const float *tail;   // AVX2 tail rows [M][ld_tail] (NULL = zeros)
    int ld_tail;
    int tail_self;       // AVX2 tail = this row's own values 0..3 before normalisation
    float thr;           // SWIGLU gate threshold
    int M;
    uint4 *panel;
    float *corr;
    float *rscale;
    float *out;          // optional fp32 copy of the panel's values (normalised x / h)
    int ld_out;
    const double *ss_in; // SWIGLU: gate/up sums times 1/sqrt(ss_in[m]/ss_K + 1e-5) (NULL: times 1)
    int ss_K;
    double *clr;         // n_clr doubles zeroed by the launch (an accumulator already consumed)
    long n_clr;
};

__device__ __forceinline__ float vx_block_sum(float v, float *red)
{
    v = vx_wave_sum64(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) red[w] = v;
    __syncthreads();
    const int nw = (blockDim.x + 63) >> 6;
    float t = 0.0f;
    for (int i = 0; i < nw; i++) t += red[i];
    __syncthreads();
    return t;
}

__device__ __forceinline__ float vx_block_max(float v, float *red)
{
    v = vx_wave_max64(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) red[w] = v;
    __syncthreads();
    const int nw = (blockDim.x + 63) >> 6;
    float r = red[0];
    for (int i = 1; i < nw; i++) r = fmaxf(r, red[i]);
    __syncthreads();
    return r;
}

// G = groups of 8 elements per thread (K <= 8192 * G <= VXH_MAX_K).
template <int MODE, int G>
__global__ __launch_bounds__(VX_ROW_THREADS) void vx_row_panel_kernel(vx_row_args a)
{
    __shared__ float red[VX_ROW_THREADS / 64];
    __shared__ float s4[VXH_MAX_K / 8 + 8];
    __shared__ float s_tail;
    const int m = blockIdx.x;
    const int K = a.K, nb = K / 32, nbp = (nb + 1) / 2 * 2;
    const int ng = nb * 4, ngp = nbp * 4;
    float v[G][8];
    if (a.clr) {
        const long per = (a.n_clr + gridDim.x - 1) / gridDim.x;
        const long b = (long)blockIdx.x * per, e = min(b + per, a.n_clr);
        for (long i = b + threadIdx.x; i < e; i += blockDim.x) a.clr[i] = 0.0;
    }
    const float rin = (MODE == VX_ROW_SWIGLU && a.ss_in) ? vx_rms_inv((float)a.ss_in[m], a.ss_K) : 1.0f;

    // ---- load (and, for the accumulator modes, consume) ----
#pragma unroll
    for (int j = 0; j < G; j++) {
        const int g = threadIdx.x + j * blockDim.x;
#pragma unroll
        for (int kk = 0; kk < 8; kk++) v[j][kk] = 0.0f;
        if (g >= ng) continue;
        const int e0 = 8 * g;
        if (MODE == VX_ROW_SWIGLU) {
            // h index i -> tile i/16: gate at physical row 32(i/16) + i%16, up 16 rows later
            double *ar = a.acc + (size_t)m * a.ld_acc;
            const int pg = 32 * (e0 / 16) + e0 % 16;
            double2 gv[4], uv[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                gv[q] = *(const double2 *)(ar + pg + 2 * q);
                uv[q] = *(const double2 *)(ar + pg + 16 + 2 * q);
            }
#pragma unroll
            for (int q = 0; q < 4; q++) {
                *(double2 *)(ar + pg + 2 * q) = make_double2(0.0, 0.0);
                *(double2 *)(ar + pg + 16 + 2 * q) = make_double2(0.0, 0.0);
            }
#pragma unroll
            for (int q = 0; q < 4; q++) {
                // as the SwiGLU prologue of the GEMM: g, u rounded to fp32, times 1/rms
                const float g0 = vx_silu((float)gv[q].x * rin), g1 = vx_silu((float)gv[q].y * rin);
                const float u0 = (float)uv[q].x * rin, u1 = (float)uv[q].y * rin;
                v[j][2 * q] = fabsf(g0) < a.thr ? 0.0f : g0 * u0;
                v[j][2 * q + 1] = fabsf(g1) < a.thr ? 0.0f : g1 * u1;
            }
        } else {
            float *xr = a.x + (size_t)m * a.ldx + e0;
            float4 x0 = *(const float4 *)xr, x1 = *(const float4 *)(xr + 4);
            float t[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            if (MODE == VX_ROW_RESID_NORM) {
                double *ar = a.acc + (size_t)m * a.ld_acc + e0;
                double2 p[4];
#pragma unroll
                for (int q = 0; q < 4; q++) p[q] = *(const double2 *)(ar + 2 * q);
#pragma unroll
                for (int q = 0; q < 4; q++) *(double2 *)(ar + 2 * q) = make_double2(0.0, 0.0);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    t[2 * q] = t[2 * q] + (float)p[q].x;
                    t[2 * q + 1] = t[2 * q + 1] + (float)p[q].y;
                }
                *(float4 *)xr = make_float4(t[0], t[1], t[2], t[3]);
                *(float4 *)(xr + 4) = make_float4(t[4], t[5], t[6], t[7]);
            }
#pragma unroll
            for (int kk = 0; kk < 8; kk++) v[j][kk] = t[kk];
        }
    }
    if (a.avx2 && a.tail_self && threadIdx.x == 0)
        s_tail = v[0][0] + v[0][1] + v[0][2] + v[0][3];

    // ---- RMSNorm ----
    if (MODE == VX_ROW_NORM || MODE == VX_ROW_RESID_NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < G; j++)
#pragma unroll
            for (int kk = 0; kk < 8; kk++) ss += v[j][kk] * v[j][kk];
        ss = vx_block_sum(ss, red);
        const float inv = vx_rms_inv(ss, K);
#pragma unroll
        for (int j = 0; j < G; j++) {
            const int g = threadIdx.x + j * blockDim.x;
            if (g >= ng) continue;
            float wv[8];
            if (a.w) {
                float4 w0 = *(const float4 *)(a.w + 8 * g), w1 = *(const float4 *)(a.w + 8 * g + 4);
                wv[0] = w0.x; wv[1] = w0.y; wv[2] = w0.z; wv[3] = w0.w;
                wv[4] = w1.x; wv[5] = w1.y; wv[6] = w1.z; wv[7] = w1.w;
            } else {
#pragma unroll
                for (int kk = 0; kk < 8; kk++) wv[kk] = 1.0f;
            }
#pragma unroll
            for (int kk = 0; kk < 8; kk++) v[j][kk] = wv[kk] * (v[j][kk] * inv);
        }
    }
    if (a.out) {
#pragma unroll
        for (int j = 0; j < G; j++) {
            const int g = threadIdx.x + j * blockDim.x;
            if (g >= ng) continue;
            float *o = a.out + (size_t)m * a.ld_out + 8 * g;
            *(float4 *)o = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
            *(float4 *)(o + 4) = make_float4(v[j][4], v[j][5], v[j][6], v[j][7]);
        }
    }

    // ---- row scale and panel ----
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < G; j++)
#pragma unroll
        for (int kk = 0; kk < 8; kk++) amax = fmaxf(amax, fabsf(v[j][kk]));
    amax = vx_block_max(amax, red);
    float rs;
    const float sc = vx_row_scale(a.avx2 ? 2.0f * amax : amax, &rs);
    if (threadIdx.x == 0) a.rscale[m] = rs;
#pragma unroll
    for (int j = 0; j < G; j++) {
        const int g = threadIdx.x + j * blockDim.x;
        if (g >= ngp) continue;   // groups of the padding block are zeros
        float u[8];
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
            const float xv = v[j][kk] * sc;
            u[kk] = (a.avx2 && kk >= 4) ? 2.0f * xv : xv;
        }
        vx_panel_store(a.panel, a.M, g, m, u);
        if (a.avx2) s4[g] = (v[j][0] + v[j][1] + v[j][2] + v[j][3]) * sc;
    }
    if (a.avx2) {
        // AVX2-lane correction of block b: x at offsets 8..11, 16..19, 24..27
        // and 32..35 (the next block's first four, or the caller's tail).
        __syncthreads();
        for (int b = threadIdx.x; b < nbp; b += blockDim.x) {
            float c = 0.0f;
            if (b < nb) {
                c = s4[4 * b + 1] + s4[4 * b + 2] + s4[4 * b + 3];
                if (b + 1 < nb) {
                    c += s4[4 * b + 4];
                } else if (a.tail_self) {
                    c += s_tail * sc;
                } else if (a.tail) {
                    const float *t = a.tail + (size_t)m * a.ld_tail;
                    c += (t[0] + t[1] + t[2] + t[3]) * sc;
                }
            }
            a.corr[(size_t)b * a.M + m] = c;
        }
    }
}

template <int MODE>
static int vx_launch_row(const vx_row_args &a, vxh_stream s)
{
    // G groups of 8 per thread, the workgroup just large enough for the row
    // (padding block included): short rows sync fewer wavefronts
    const int ngp = (a.K / 32 + 1) / 2 * 2 * 4;
    const int G = (ngp + VX_ROW_THREADS - 1) / VX_ROW_THREADS;
    const int threads = ((ngp + G - 1) / G + 63) / 64 * 64;
    if (G == 1)
        vx_row_panel_kernel<MODE, 1><<<a.M, threads, 0, vxh_hs(s)>>>(a);
    else if (G == 2)
        vx_row_panel_kernel<MODE, 2><<<a.M, threads, 0, vxh_hs(s)>>>(a);
    else if (G == 3)
        vx_row_panel_kernel<MODE, 3><<<a.M, threads, 0, vxh_hs(s)>>>(a);
    else
        return vxh_fail(VXH_ERR_PARAM, "row length %d above %d", a.K, VXH_MAX_K);
    VXH_LAUNCHED();
    return VXH_OK;
}

static int vx_row_check(const vxh_panel *p, int M, int K, const char *what)
{
    if (M < 1 || M > 16 || K != p->K || K % 32 || K > VXH_MAX_K)
        return vxh_fail(VXH_ERR_PARAM, "%s: M %d K %d (panel K %d)", what, M, K, p->K);
    return VXH_OK;
}

static vx_row_args vx_row_base(vxh_panel *p, int M, int K, int avx2)
{
    vx_row_args a;
    memset(&a, 0, sizeof(a));
    a.K = K;
    a.M = M;
    a.avx2 = avx2;
    a.panel = (uint4 *)p->data;
    a.corr = p->corr;
    a.rscale = p->rscale;
    p->M = M;
    p->avx2 = avx2;
    p->rs_ld = 0;
    return a;
}

extern "C" int vxh_prep_panel(vxh_panel *p, const float *x, int ldx, int M, int K, int avx2,
                              const float *tail, int ld_tail, vxh_stream s)
{
    int rc = vx_row_check(p, M, K, "prep_panel");
    if (rc) return rc;
    vx_row_args a = vx_row_base(p, M, K, avx2);
    a.x = (float *)x;
    a.ldx = ldx;
    a.tail = tail;
    a.ld_tail = ld_tail;
    return vx_launch_row<VX_ROW_PLAIN>(a, s);
}

extern "C" int vxh_rmsnorm_panel(const float *x, int ldx, int M, int K, const float *w, int avx2,
                                 const float *tail, int ld_tail, vxh_panel *p, float *xn_out,
                                 int ld_xn, vxh_stream s)
{
    int rc = vx_row_check(p, M, K, "rmsnorm_panel");
    if (rc) return rc;
    vx_row_args a = vx_row_base(p, M, K, avx2);
    a.x = (float *)x;
    a.ldx = ldx;
    a.w = w;
    a.tail = tail;
    a.ld_tail = ld_tail;
    a.tail_self = tail == x && ld_tail == ldx;
    a.out = xn_out;
    a.ld_out = ld_xn;
    return vx_launch_row<VX_ROW_NORM>(a, s);
}

extern "C" int vxh_resid_rmsnorm_panel(float *x, int ldx, double *acc, int ld_acc, int M, int K,
                                       const float *w, int avx2, int tail_self, vxh_panel *p,
                                       float *xn_out, int ld_xn, vxh_stream s)
{
    int rc = vx_row_check(p, M, K, "resid_rmsnorm_panel");
    if (rc) return rc;
    vx_row_args a = vx_row_base(p, M, K, avx2);
    a.x = x;
    a.ldx = ldx;
    a.acc = acc;
    a.ld_acc = ld_acc;
    a.w = w;
    a.tail_self = tail_self;
    a.out = xn_out;
    a.ld_out = ld_xn;
    return vx_launch_row<VX_ROW_RESID_NORM>(a, s);
}

extern "C" int vxh_swiglu_panel(double *acc, int ld_acc, int M, int F, float thr, int avx2,
                                vxh_panel *p, float *h_out, int ldh, vxh_stream s)
{
    int rc = vx_row_check(p, M, F, "swiglu_panel");
    if (rc) return rc;
    vx_row_args a = vx_row_base(p, M, F, avx2);
    a.acc = acc;
    a.ld_acc = ld_acc;
    a.thr = thr;
    a.out = h_out;
    a.ld_out = ldh;
    return vx_launch_row<VX_ROW_SWIGLU>(a, s);
}

// SwiGLU panel of M rows x F with one power-of-two scale per VX_CHUNK
// columns: workgroup (chunk c, row m) forms h for columns [c*VX_CHUNK,
// (c+1)*VX_CHUNK), one thread per 8 columns, as the VXH_PRO_SWIGLU prologue
// does (src/model.c:582-585), clears the gate/up sums it read, and writes
// its part of the panel; the launch also zeroes `clr`.
#define VX_SWC_THREADS (VX_CHUNK / 8)
__global__ __launch_bounds__(VX_SWC_THREADS) void vx_swiglu_chunk_kernel(
    double *__restrict__ acc, int ld_acc, int M, int F, float thr, const double *__restrict__ ss_in, int ss_K,
    uint4 *__restrict__ panel, float *__restrict__ rscale, int rs_ld, double *__restrict__ clr, long n_clr)
{
    __shared__ float red[VX_SWC_THREADS / 64];
    const int c = blockIdx.x, m = blockIdx.y;
    if (clr) {
        const long nb = (long)gridDim.x * gridDim.y, bi = (long)m * gridDim.x + c;
        const long per = (n_clr + nb - 1) / nb;
        const long b = bi * per, e = min(b + per, n_clr);
        for (long i = b + threadIdx.x; i < e; i += VX_SWC_THREADS) clr[i] = 0.0;
    }
    const int nb = F / 32, nbp = (nb + 1) / 2 * 2, ng = nb * 4, ngp = nbp * 4;
    const int g = c * VX_SWC_THREADS + threadIdx.x;   // group of 8 columns
    const float rin = ss_in ? vx_rms_inv((float)ss_in[m], ss_K) : 1.0f;
    float v[8];
#pragma unroll
    for (int kk = 0; kk < 8; kk++) v[kk] = 0.0f;
    if (g < ng) {
        const int e0 = 8 * g;
        double *ar = acc + (size_t)m * ld_acc + 32 * (e0 / 16) + e0 % 16;
        double2 gv[4], uv[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            gv[q] = *(const double2 *)(ar + 2 * q);
            uv[q] = *(const double2 *)(ar + 16 + 2 * q);
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
            *(double2 *)(ar + 2 * q) = make_double2(0.0, 0.0);
            *(double2 *)(ar + 16 + 2 * q) = make_double2(0.0, 0.0);
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float g0 = vx_silu((float)gv[q].x * rin), g1 = vx_silu((float)gv[q].y * rin);
            const float u0 = (float)uv[q].x * rin, u1 = (float)uv[q].y * rin;
            v[2 * q] = fabsf(g0) < thr ? 0.0f : g0 * u0;
            v[2 * q + 1] = fabsf(g1) < thr ? 0.0f : g1 * u1;
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int kk = 0; kk < 8; kk++) amax = fmaxf(amax, fabsf(v[kk]));
    amax = vx_block_max(amax, red);
    float rs;
    const float sc = vx_row_scale(amax, &rs);
    if (threadIdx.x == 0) rscale[m * rs_ld + c] = rs;
    if (g < ngp) {   // groups of the padding block are zeros
        float x[8];
#pragma unroll
        for (int kk = 0; kk < 8; kk++) x[kk] = v[kk] * sc;
        vx_panel_store(panel, M, g, m, x);
    }
}

extern "C" int vxh_swiglu_panel_norm(double *acc, int ld_acc, int M, int F, float thr, const double *ss_in,
                                     int ss_K, double *clear, size_t n_clear, vxh_panel *p, vxh_stream s)
{
    return vxh_swiglu_panel_norm_timed(acc, ld_acc, M, F, thr, ss_in, ss_K, clear, n_clear, p, nullptr, nullptr, s);
}

extern "C" int vxh_swiglu_panel_norm_timed(double *acc, int ld_acc, int M, int F, float thr, const double *ss_in,
                                           int ss_K, double *clear, size_t n_clear, vxh_panel *p, vxh_event e0,
                                           vxh_event e1, vxh_stream s)
{
    int rc = vx_row_check(p, M, F, "swiglu_panel_norm");
    if (rc) return rc;
    if (ss_in && ss_K < 1) return vxh_fail(VXH_ERR_PARAM, "swiglu_panel_norm: norm length %d", ss_K);
    if (n_clear && !clear) return vxh_fail(VXH_ERR_PARAM, "swiglu_panel_norm: clear range without a pointer");
    const int chunks = (F + VX_CHUNK - 1) / VX_CHUNK;
    p->M = M;
    p->avx2 = 0;
    p->rs_ld = chunks;
    if (e0 || e1)   // events recorded by the dispatch itself around the kernel
        hipExtLaunchKernelGGL(vx_swiglu_chunk_kernel, dim3(chunks, M), dim3(VX_SWC_THREADS), 0, vxh_hs(s),
                              (hipEvent_t)e0, (hipEvent_t)e1, 0, acc, ld_acc, M, F, thr, ss_in, ss_K,
                              (uint4 *)p->data, p->rscale, chunks, n_clear ? clear : nullptr, (long)n_clear);
    else
        vx_swiglu_chunk_kernel<<<dim3(chunks, M), VX_SWC_THREADS, 0, vxh_hs(s)>>>(
            acc, ld_acc, M, F, thr, ss_in, ss_K, (uint4 *)p->data, p->rscale, chunks, n_clear ? clear : nullptr,
            (long)n_clear);
    VXH_LAUNCHED();
    return VXH_OK;
}

__global__ void vx_rmsnorm_kernel(const float *__restrict__ x, int ldx, int K,
                                  const float *__restrict__ w, float *__restrict__ out, int ld_out)
{
    __shared__ float red[16];
    int m = blockIdx.x;
    const float *xr = x + (size_t)m * ldx;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < K; i += blockDim.x) ss += xr[i] * xr[i];
    ss = vx_block_sum(ss, red);
    float inv = vx_rms_inv(ss, K);
    for (int i = threadIdx.x; i < K; i += blockDim.x)
        out[(size_t)m * ld_out + i] = (w ? w[i] : 1.0f) * (xr[i] * inv);
}

extern "C" int vxh_rmsnorm(const float *x, int ldx, int M, int K, const float *w, float *out,
                           int ld_out, vxh_stream s)
{
    if (M <= 0) return VXH_OK;
    vx_rmsnorm_kernel<<<M, 256, 0, vxh_hs(s)>>>(x, ldx, K, w, out, ld_out);
    VXH_LAUNCHED();
    return VXH_OK;
}

// ---------------------------------------------------------------------------
// dot-product path (VXH_PATH_DOT): the same GEMM without MFMA
// ---------------------------------------------------------------------------
// Same workgroup shape, K slices, weight stream and LDS panel slice as
// vx_gemm_kernel.  Lane (j, h) of a wavefront takes row j of its tile and the
// K half h (elements 16h..16h+15) of both blocks of every pair: the nibbles
// or bytes unpack to exact fp16 (s - 8, resp. q) as on the MFMA path, and
// every activation row m accumulates d * sum (w * x_hi + w * x_lo) with
// v_dot2_f32_f16 from the panel's hi and lo parts.  The two K halves of a row
// meet with one lane swap before the fp64 atomic add.  Exists to measure the
// MFMA path against (src/simd/avx2.c:311-370 is a dot product per row).
#define VX_DOT_PPW 8

__device__ __forceinline__ float vx_dot8(const vx_half8 &w, const vx_half8 &x, float t)
{
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const vx_half2 a = {w[2 * q], w[2 * q + 1]};
        const vx_half2 b = {x[2 * q], x[2 * q + 1]};
        t = __builtin_amdgcn_fdot2(a, b, t, false);
    }
    return t;
}

template <int QT, int M>
__global__ __launch_bounds__(256) void vx_gemm_dot_kernel(vx_gemm_args a)
{
    constexpr int PPW = VX_DOT_PPW;
    constexpr int NS = 2 * M;
    constexpr int WPP = QT == 2 ? 1 : 2;
    constexpr int UNITS = PPW * 8 * NS;
    constexpr int UPT = (UNITS + 255) / 256;
    __shared__ uint4 lds[UPT * 256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = blockIdx.x / a.n_splits, split = blockIdx.x % a.n_splits;
    const int T = grp * 4 + wave;
    const bool tile_ok = T < a.n_tiles;
    const int Tc = tile_ok ? T : 0;
    const int p0 = split * PPW;
    const int np = min(PPW, a.n_pairs - p0);
    const int units = np * 8 * NS;
    const int c = lane & 31, h = lane >> 5;
    const uint32_t magic = 0x64006400u;
    uint4 pv[UPT];
    const uint4 *psrc = a.panel + (size_t)p0 * 8 * NS;
#pragma unroll
    for (int j = 0; j < UPT; j++) pv[j] = psrc[min(j * 256 + (int)threadIdx.x, units - 1)];
    const uint4 *wp = a.wq + ((size_t)Tc * a.n_pairs + p0) * WPP * 64 + lane;
    const uint32_t *sp = a.wd + ((size_t)Tc * a.n_pairs + p0) * 32 + c;
    uint4 w[VX_RING][WPP];
    uint32_t sc[VX_RING];
#pragma unroll
    for (int i = 0; i < VX_RING; i++) {
        const int pi = min(i, np - 1);
#pragma unroll
        for (int q = 0; q < WPP; q++) w[i][q] = wp[((size_t)pi * WPP + q) * 64];
        sc[i] = sp[(size_t)pi * 32];
    }
#pragma unroll
    for (int j = 0; j < UPT; j++) lds[j * 256 + threadIdx.x] = pv[j];
    __syncthreads();
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; m++) acc[m] = 0.0f;
#pragma unroll
    for (int i = 0; i < PPW; i++) {
        uint4 wv[WPP];
#pragma unroll
        for (int q = 0; q < WPP; q++) wv[q] = w[i % VX_RING][q];
        const uint32_t sv = sc[i % VX_RING];
        if (i + VX_RING < PPW) {
            const int pi = min(i + VX_RING, np - 1);
#pragma unroll
            for (int q = 0; q < WPP; q++) w[i % VX_RING][q] = wp[((size_t)pi * WPP + q) * 64];
            sc[i % VX_RING] = sp[(size_t)pi * 32];
        }
        if (i < np) {
#pragma unroll
            for (int blk = 0; blk < 2; blk++) {
                const int bl = 2 * i + blk;
                vx_half8 b0, b1;
                if (QT == 2) {
                    b0 = vx_unpack_q4(blk ? wv[0].z : wv[0].x, magic);
                    b1 = vx_unpack_q4(blk ? wv[0].w : wv[0].y, magic);
                } else {
                    b0 = vx_unpack_q8(wv[blk].x, wv[blk].y, magic);
                    b1 = vx_unpack_q8(wv[blk].z, wv[blk].w, magic);
                }
                const float d = vx_half_bits_to_float((sv >> (16 * blk)) & 0xFFFFu);
                const uint4 *u0 = lds + ((bl * 2 + 0) * 2 + h) * NS, *u1 = lds + ((bl * 2 + 1) * 2 + h) * NS;
#pragma unroll
                for (int m = 0; m < M; m++) {
                    float t = 0.0f;
                    t = vx_dot8(b0, __builtin_bit_cast(vx_half8, u0[m]), t);
                    t = vx_dot8(b0, __builtin_bit_cast(vx_half8, u0[M + m]), t);
                    t = vx_dot8(b1, __builtin_bit_cast(vx_half8, u1[m]), t);
                    t = vx_dot8(b1, __builtin_bit_cast(vx_half8, u1[M + m]), t);
                    acc[m] = fmaf(d, t, acc[m]);
                }
            }
        }
    }
    // row j's two K halves live in lanes j and j + 32
#pragma unroll
    for (int m = 0; m < M; m++) acc[m] = vx_sum_x32(acc[m]);
    const int n = T * 32 + c;
    if (h == 0 && tile_ok && n < a.n_out) {
        const int chunk = p0 / a.rs_chunk;
#pragma unroll
        for (int m = 0; m < M; m++) {
            if (a.gate && fabsf(a.gate[(size_t)m * a.ld_gate + n]) < a.thr) continue;
            const float osc = a.rscale[m * a.rs_ld + chunk] * a.scale;
            __hip_atomic_fetch_add(&a.acc[(size_t)m * a.ld_acc + n], (double)(acc[m] * osc), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int QT, int M>
static int vx_launch_dot(const vxh_qmat *W, vx_gemm_args &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1)
{
    a.n_tiles = W->n_rows / 32;
    a.n_pairs = W->n_pairs;
    a.n_splits = (W->n_pairs + VX_DOT_PPW - 1) / VX_DOT_PPW;
    if (a.rs_ld > 1 && a.rs_chunk % VX_DOT_PPW)
        return vxh_fail(VXH_ERR_PARAM, "gemm: K slice of %d pairs crosses a %d-pair scale chunk", VX_DOT_PPW,
                        a.rs_chunk);
    const int groups = (a.n_tiles + 3) / 4;
    if (e0 || e1)
        hipExtLaunchKernelGGL(vx_gemm_dot_kernel<QT, M>, dim3(groups * a.n_splits), dim3(256), 0, st, e0, e1, 0,
                              a);
    else
        vx_gemm_dot_kernel<QT, M><<<groups * a.n_splits, 256, 0, st>>>(a);
    VXH_LAUNCHED();
    return VXH_OK;
}

template <int M>
static int vx_dot_m(const vxh_qmat *W, vx_gemm_args &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1)
{
    return W->type == 2 ? vx_launch_dot<2, M>(W, a, st, e0, e1) : vx_launch_dot<8, M>(W, a, st, e0, e1);
}

static int vx_dot_dispatch(const vxh_qmat *W, int M, vx_gemm_args &a, hipStream_t st, hipEvent_t e0,
                           hipEvent_t e1)
{
    switch (M) {
    case 1: return vx_dot_m<1>(W, a, st, e0, e1);
    case 2: return vx_dot_m<2>(W, a, st, e0, e1);
    case 3: return vx_dot_m<3>(W, a, st, e0, e1);
    case 4: return vx_dot_m<4>(W, a, st, e0, e1);
    case 5: return vx_dot_m<5>(W, a, st, e0, e1);
    case 6: return vx_dot_m<6>(W, a, st, e0, e1);
    case 7: return vx_dot_m<7>(W, a, st, e0, e1);
    case 8: return vx_dot_m<8>(W, a, st, e0, e1);
    case 9: return vx_dot_m<9>(W, a, st, e0, e1);
    case 10: return vx_dot_m<10>(W, a, st, e0, e1);
    case 11: return vx_dot_m<11>(W, a, st, e0, e1);
    case 12: return vx_dot_m<12>(W, a, st, e0, e1);
    case 13: return vx_dot_m<13>(W, a, st, e0, e1);
    case 14: return vx_dot_m<14>(W, a, st, e0, e1);
    case 15: return vx_dot_m<15>(W, a, st, e0, e1);
    default: return vx_dot_m<16>(W, a, st, e0, e1);
    }
}

// ---------------------------------------------------------------------------
// F32 weight matrices (src/model.c:174-179, 206-211 dispatch them to the fp32
// GEMV): the workgroup decodes its 512-column slice of the panel to fp32
// (hi + lo, exact) in LDS; wavefront w takes 16 output rows, 4 lanes per row
// with float4 weight loads; the products of an fp32 weight and a 22-bit
// activation are exact in fp64, so each row's slice sum is accumulated in
// fp64 and added to the accumulator with the slice's row scale.
// ---------------------------------------------------------------------------
#define VX_F32_KS 512    // columns per workgroup slice (divides the 1024-column scale chunk)
#define VX_F32_ROWS 64   // output rows per workgroup

template <int M>
__global__ __launch_bounds__(256) void vx_gemm_f32_kernel(vx_gemm_args a, int K, int n_ks)
{
    __shared__ float4 xs[M][VX_F32_KS / 4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = blockIdx.x / n_ks, ks = blockIdx.x % n_ks;
    const int k0 = ks * VX_F32_KS, kn = min(VX_F32_KS, K - k0);   // K % 32 == 0, so kn % 32 == 0
    // panel unit of column group g, row m: ((g/4 * 2 + g%2) * 2 + (g/2)%2) * 2M + m (hi), + M (lo)
    for (int it = threadIdx.x; it < M * (VX_F32_KS / 8); it += 256) {
        const int m = it / (VX_F32_KS / 8), gl = it % (VX_F32_KS / 8), g = k0 / 8 + gl;
        float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (8 * gl < kn) {
            const size_t base = ((size_t)((g >> 2) * 2 + (g & 1)) * 2 + ((g >> 1) & 1)) * (2 * M);
            const vx_half8 hi = __builtin_bit_cast(vx_half8, a.panel[base + m]);
            const vx_half8 lo = __builtin_bit_cast(vx_half8, a.panel[base + M + m]);
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = (float)hi[e] + (float)lo[e];
        }
        xs[m][2 * gl] = make_float4(v[0], v[1], v[2], v[3]);
        xs[m][2 * gl + 1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    __syncthreads();
    const int r = lane >> 2, kq = lane & 3;
    const int n = grp * VX_F32_ROWS + wave * 16 + r;
    const int ldw = a.n_pairs * 64;
    const float *wr = (const float *)a.wq + (size_t)min(n, a.n_tiles * 32 - 1) * ldw + k0;
    double acc[M];
#pragma unroll
    for (int m = 0; m < M; m++) acc[m] = 0.0;
#pragma unroll 8
    for (int j = 0; j < VX_F32_KS / 16; j++) {
        const int k = 16 * j + 4 * kq;
        if (k >= kn) break;
        const float4 w = *(const float4 *)(wr + k);
#pragma unroll
        for (int m = 0; m < M; m++) {
            const float4 x = xs[m][k / 4];
            acc[m] = fma((double)w.x, (double)x.x, acc[m]);
            acc[m] = fma((double)w.y, (double)x.y, acc[m]);
            acc[m] = fma((double)w.z, (double)x.z, acc[m]);
            acc[m] = fma((double)w.w, (double)x.w, acc[m]);
        }
    }
#pragma unroll
    for (int m = 0; m < M; m++) {
        acc[m] += __shfl_xor(acc[m], 1);
        acc[m] += __shfl_xor(acc[m], 2);
    }
    if (kq != 0 || n >= a.n_out) return;
    const int chunk = (k0 / 64) / a.rs_chunk;
    float osc[M];
#pragma unroll
    for (int m = 0; m < M; m++) osc[m] = a.rscale[m * a.rs_ld + chunk] * a.scale;
    bool keep[M];
#pragma unroll
    for (int m = 0; m < M; m++) keep[m] = true;
    if (a.gate) {
        float gv[M];
#pragma unroll
        for (int m = 0; m < M; m++) gv[m] = a.gate[(size_t)m * a.ld_gate + n];
#pragma unroll
        for (int m = 0; m < M; m++) keep[m] = !(fabsf(gv[m]) < a.thr);
    }
#pragma unroll
    for (int m = 0; m < M; m++)
        if (keep[m])
            __hip_atomic_fetch_add(&a.acc[(size_t)m * a.ld_acc + n], acc[m] * (double)osc[m], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
}

template <int M>
static int vx_launch_f32(const vxh_qmat *W, vx_gemm_args &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1)
{
    a.n_tiles = W->n_rows / 32;
    a.n_pairs = W->n_pairs;
    const int K = W->n_cols;
    const int n_ks = (K + VX_F32_KS - 1) / VX_F32_KS;
    const int groups = (a.n_out + VX_F32_ROWS - 1) / VX_F32_ROWS;
    if (a.rs_ld > 1 && (a.rs_chunk * 64) % VX_F32_KS)
        return vxh_fail(VXH_ERR_PARAM, "gemm f32: slice of %d columns crosses a scale chunk", VX_F32_KS);
    if (e0 || e1)
        hipExtLaunchKernelGGL(vx_gemm_f32_kernel<M>, dim3(groups * n_ks), dim3(256), 0, st, e0, e1, 0, a, K, n_ks);
    else
        vx_gemm_f32_kernel<M><<<groups * n_ks, 256, 0, st>>>(a, K, n_ks);
    VXH_LAUNCHED();
    return VXH_OK;
}

static int vx_f32_dispatch(const vxh_qmat *W, int M, vx_gemm_args &a, hipStream_t st, hipEvent_t e0,
                           hipEvent_t e1)
{
    switch (M) {
    case 1: return vx_launch_f32<1>(W, a, st, e0, e1);
    case 2: return vx_launch_f32<2>(W, a, st, e0, e1);
    case 3: return vx_launch_f32<3>(W, a, st, e0, e1);
    case 4: return vx_launch_f32<4>(W, a, st, e0, e1);
    case 5: return vx_launch_f32<5>(W, a, st, e0, e1);
    case 6: return vx_launch_f32<6>(W, a, st, e0, e1);
    case 7: return vx_launch_f32<7>(W, a, st, e0, e1);
    case 8: return vx_launch_f32<8>(W, a, st, e0, e1);
    case 9: return vx_launch_f32<9>(W, a, st, e0, e1);
    case 10: return vx_launch_f32<10>(W, a, st, e0, e1);
    case 11: return vx_launch_f32<11>(W, a, st, e0, e1);
    case 12: return vx_launch_f32<12>(W, a, st, e0, e1);
    case 13: return vx_launch_f32<13>(W, a, st, e0, e1);
    case 14: return vx_launch_f32<14>(W, a, st, e0, e1);
    case 15: return vx_launch_f32<15>(W, a, st, e0, e1);
    default: return vx_launch_f32<16>(W, a, st, e0, e1);
    }
}

extern "C" int vxh_gemm_acc_timed(const vxh_qmat *W, const vxh_panel *X, int M, double *acc,
                                  int ld_acc, int n_out, float scale, const float *gate, int ld_gate,
                                  float thr, int path, vxh_event start, vxh_event stop, vxh_stream s)
{
    if (M != X->M || M < 1 || M > 16)
        return vxh_fail(VXH_ERR_PARAM, "gemm: M %d (panel M %d)", M, X->M);
    if (W->n_cols != X->K)
        return vxh_fail(VXH_ERR_PARAM, "gemm: W has K %d, panel %d", W->n_cols, X->K);
    if (n_out < 0 || n_out > W->n_rows || (n_out > ld_acc && M > 1))
        return vxh_fail(VXH_ERR_PARAM, "gemm: n_out %d (rows %d, ld %d)", n_out, W->n_rows, ld_acc);
    if (path == VXH_PATH_DOT && X->avx2)
        return vxh_fail(VXH_ERR_UNSUPPORTED, "dot-product path: exact Q4_0/Q8_0 panels only");
    if (n_out == 0) return VXH_OK;
    vx_gemm_args a;
    memset(&a, 0, sizeof(a));
    a.wq = (const uint4 *)W->qs;
    a.wcache = W->cached;
    a.wd = (const uint32_t *)W->d;
    a.panel = (const uint4 *)X->data;
    a.corr = X->corr;
    a.rscale = X->rscale;
    a.rs_ld = X->rs_ld > 0 ? X->rs_ld : 1;
    a.rs_chunk = X->rs_ld > 0 ? VX_CHUNK / 64 : 1 << 30;   // block pairs per scale chunk
    a.acc = acc;
    a.ld_acc = ld_acc;
    a.n_out = n_out;
    a.scale = scale;
    a.gate = gate;
    a.ld_gate = ld_gate;
    a.thr = thr;
    if (W->type == 0) {
        if (X->avx2) return vxh_fail(VXH_ERR_UNSUPPORTED, "F32 matrices take exact panels");
        return vx_f32_dispatch(W, M, a, vxh_hs(s), (hipEvent_t)start, (hipEvent_t)stop);
    }
    if (path == VXH_PATH_DOT) return vx_dot_dispatch(W, M, a, vxh_hs(s), (hipEvent_t)start, (hipEvent_t)stop);
    return vx_dispatch<>(W, M, X->avx2, a, vxh_hs(s), (hipEvent_t)start, (hipEvent_t)stop);
}

extern "C" int vxh_gemm_acc(const vxh_qmat *W, const vxh_panel *X, int M, double *acc, int ld_acc,
                            int n_out, float scale, const float *gate, int ld_gate, float thr,
                            int path, vxh_stream s)
{
    return vxh_gemm_acc_timed(W, X, M, acc, ld_acc, n_out, scale, gate, ld_gate, thr, path, nullptr,
                              nullptr, s);
}

// ---------------------------------------------------------------------------
// accumulator consumers
// ---------------------------------------------------------------------------
// y may alias r (x += acc in place)
__global__ void vx_acc_store_kernel(double *__restrict__ acc, int ld_acc, int n, float *y, int ldy,
                                    const float *r, int ldr)
{
    const int m = blockIdx.y;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        double *p = acc + (size_t)m * ld_acc + i;
        const float v = (float)*p;
        *p = 0.0;
        y[(size_t)m * ldy + i] = r ? r[(size_t)m * ldr + i] + v : v;
    }
}

extern "C" int vxh_acc_store(double *acc, int ld_acc, int M, int n, float *y, int ldy,
                             const float *r, int ldr, vxh_stream s)
{
    if (M <= 0 || n <= 0) return VXH_OK;
    int gx = (n + 255) / 256;
    if (gx > 256) gx = 256;
    vx_acc_store_kernel<<<dim3(gx, M), 256, 0, vxh_hs(s)>>>(acc, ld_acc, n, y, ldy, r, ldr);
    VXH_LAUNCHED();
    return VXH_OK;
}

__global__ void vx_acc_swiglu_kernel(double *__restrict__ acc, int ld_acc, int F, float thr,
                                     float *__restrict__ h, int ldh)
{
    const int m = blockIdx.y;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < F; i += gridDim.x * blockDim.x) {
        double *pg = acc + (size_t)m * ld_acc + 32 * (i / 16) + i % 16;
        const float g = vx_silu((float)pg[0]), u = (float)pg[16];
        pg[0] = 0.0;
        pg[16] = 0.0;
        h[(size_t)m * ldh + i] = fabsf(g) < thr ? 0.0f : g * u;
    }
}

extern "C" int vxh_acc_swiglu(double *acc, int ld_acc, int M, int F, float thr, float *h, int ldh,
                              vxh_stream s)
{
    if (M <= 0 || F <= 0) return VXH_OK;
    int gx = (F + 255) / 256;
    if (gx > 256) gx = 256;
    vx_acc_swiglu_kernel<<<dim3(gx, M), 256, 0, vxh_hs(s)>>>(acc, ld_acc, F, thr, h, ldh);
    VXH_LAUNCHED();
    return VXH_OK;
}

extern "C" size_t vxh_gemm_workspace_elems(int n_rows, int M)
{
    return (size_t)M * (size_t)((n_rows + 31) / 32 * 32);
}

extern "C" int vxh_gemm(const vxh_qmat *W, const vxh_panel *X, int M, const vxh_epilogue *e,
                        vxh_workspace *ws, int path, vxh_stream s)
{
    const int ld = W->n_rows;
    if (!ws->acc || ws->acc_elems < vxh_gemm_workspace_elems(W->n_rows, M))
        return vxh_fail(VXH_ERR_PARAM, "gemm workspace too small: need %zu elements",
                        vxh_gemm_workspace_elems(W->n_rows, M));
    int rc;
    switch (e->kind) {
    case VXH_EPI_STORE:
    case VXH_EPI_RESID:
        rc = vxh_gemm_acc(W, X, M, ws->acc, ld, e->n_out, e->scale, NULL, 0, 0.0f, path, s);
        if (rc) return rc;
        return vxh_acc_store(ws->acc, ld, M, e->n_out, e->y, e->ldy,
                             e->kind == VXH_EPI_RESID ? e->r : NULL, e->ldr, s);
    case VXH_EPI_GATE:
        rc = vxh_gemm_acc(W, X, M, ws->acc, ld, e->n_out, e->scale, e->r, e->ldr, e->thr, path, s);
        if (rc) return rc;
        return vxh_acc_store(ws->acc, ld, M, e->n_out, e->y, e->ldy, NULL, 0, s);
    case VXH_EPI_SWIGLU: {
        const int phys = (e->n_out + 15) / 16 * 32;
        if (phys > W->n_rows)
            return vxh_fail(VXH_ERR_PARAM, "swiglu: F %d needs %d rows", e->n_out, phys);
        rc = vxh_gemm_acc(W, X, M, ws->acc, ld, phys, e->scale, NULL, 0, 0.0f, path, s);
        if (rc) return rc;
        return vxh_acc_swiglu(ws->acc, ld, M, e->n_out, e->thr, e->y, e->ldy, s);
    }
    default:
        return vxh_fail(VXH_ERR_PARAM, "gemm: epilogue kind %d", e->kind);
    }
}
