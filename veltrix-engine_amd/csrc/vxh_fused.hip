// Fused forward path: GEMMs whose last-arriving workgroup per super-group of
// output rows runs the follow-up elementwise work, and panels built by their
// producers.
//
// A plain layer needs a row kernel after each GEMM (RoPE/KV write, residual
// add + RMSNorm panel, SwiGLU panel), each one workgroup per row and one more
// dependent launch.  Here that work moves into the GEMM:
//
//   * RMSNorm commutes with the product: W (w.x / rms) = (W (w.x)) / rms.
//     The producer of x writes the panel of w.x and adds sum(x^2) per row
//     into an fp64 accumulator; the consuming GEMM scales its output by
//     1/rms computed from that sum.  No full-row reduction precedes the panel.
//   * The fp16 hi/lo panel keeps full precision within a power-of-two window
//     of its magnitude; each chunk of VX_CHUNK columns carries its own
//     power-of-two scale (chosen from the chunk's max |value|), which the
//     consuming GEMM applies per K slice (a slice never crosses a chunk).
//   * Super-group = the workgroups covering VX_CHUNK output columns (2*VX_CHUNK
//     gate/up rows).  Each workgroup adds its fp32 partial sums into the fp64
//     accumulator with device-scope atomics, waits for them to complete, and
//     counts itself in; the last one to arrive reads the final sums with
//     device-scope loads, runs the epilogue, clears the accumulator and
//     resets the counter.  No workgroup waits for another.
#include "vxh_gemm_core.h"

#define VX_EPI_THREADS 256

// The last arriver reads the final sums with plain loads after an
// agent-scope acquire (the caller's fence invalidated the stale lines).
__device__ __forceinline__ double vx_load_agent(const double *p) { return *p; }

// Chunk scale for max |v| = amax: values are multiplied by s_in so that the
// chunk's maximum lies in [2^13, 2^14); the GEMM output is multiplied by
// s_out = 1/s_in.
__device__ __forceinline__ void vx_chunk_scale(float amax, float *s_in, float *s_out)
{
    if (!(amax > 0.0f) || !isfinite(amax)) {
        *s_in = 1.0f;
        *s_out = 1.0f;
        return;
    }
    int ex;
    frexpf(amax, &ex);
    *s_in = ldexpf(1.0f, 14 - ex);
    *s_out = ldexpf(1.0f, ex - 14);
}

__device__ __forceinline__ float vx_wave_max(float v) { return vx_wave_max64(v); }

__device__ __forceinline__ double vx_wave_sum_f64(double v)
{
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Epilogue thread layout: thread t owns output group g = t % 128 (8
// consecutive outputs) of rows m = t/128 + 2j.  Each wavefront sees one row
// per j, so row reductions are a wavefront shuffle plus two partials in LDS.
#define VX_EPI_J(M) (((M) + 1) / 2)

// Reduces per-row (sum x^2, max |v|) partials of this thread's rows across
// the workgroup; returns the chunk input scale of each row in scl_out (LDS)
// after writing the output scale to rs[m * rs_ld + chunk] and adding the sum
// of squares to ss[m] (when ss != NULL).
template <int M>
__device__ void vx_epi_row_stats(const double *ss_part, const float *am_part, double *ss, float *rs,
                                 int rs_ld, int chunk, uint4 *lds, float *scl_out)
{
    double *red_ss = (double *)lds;                 // [16][2]
    float *red_am = (float *)(red_ss + 32);         // [16][2]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, rh = threadIdx.x >> 7;
#pragma unroll
    for (int j = 0; j < VX_EPI_J(M); j++) {
        const int m = rh + 2 * j;
        const double s = vx_wave_sum_f64(ss_part[j]);
        const float a = vx_wave_max(am_part[j]);
        if (lane == 0 && m < M) {
            red_ss[m * 2 + (wave & 1)] = s;
            red_am[m * 2 + (wave & 1)] = a;
        }
    }
    __syncthreads();
    if ((int)threadIdx.x < M) {
        const int m = threadIdx.x;
        if (ss) atomicAdd(&ss[m], red_ss[m * 2] + red_ss[m * 2 + 1]);
        float s_in, s_out;
        vx_chunk_scale(fmaxf(red_am[m * 2], red_am[m * 2 + 1]), &s_in, &s_out);
        rs[m * rs_ld + chunk] = s_out;
        scl_out[m] = s_in;
    }
    __syncthreads();
}

// Epilogue thread layout.  Pass 1 (the final sums, read with device-scope
// loads) is coalesced: thread t = (rh, g), rh = t / 128, g = t % 128, takes
// column c0 + 128 k + g (k = 0..7) of rows m = rh + 2 j, so each load of a
// wavefront covers 64 consecutive columns.  Pass 2 (the panel) takes the 8
// consecutive columns c0 + 8 g .. + 7 of the same rows, reading back what
// pass 1 stored.
template <int EPI, int M>
__device__ void vx_gemm_epilogue(const vx_gemm_args &a, int sg, uint4 *lds, int lds_units)
{
    constexpr int J = VX_EPI_J(M);
    constexpr int JB = 2;                 // rows per batch of loads
    const vx_epi_args &e = a.e;
    const int g = threadIdx.x & 127, rh = threadIdx.x >> 7;
    float *scl = (float *)lds + 256;      // [16], after the reduction scratch
    const int c0 = sg * VX_CHUNK;

    if constexpr (EPI == VX_EPI_STORE || EPI == VX_EPI_ROPE) {
        const int c1 = min(c0 + VX_CHUNK, a.n_out);
        const int qd = e.n_heads * e.hd, kvd = e.n_kv * e.hd, half = e.hd / 2;
#pragma unroll
        for (int jb = 0; jb < J; jb += JB) {
            float v[JB][8];
#pragma unroll
            for (int b = 0; b < JB; b++) {
                const int m = rh + 2 * (jb + b);
                if (jb + b >= J || m >= M) continue;
                const double *ar = a.acc + (size_t)m * a.ld_acc + c0 + g;
#pragma unroll
                for (int k = 0; k < 8; k++)
                    v[b][k] = c0 + 128 * k + g < c1 ? (float)vx_load_agent(ar + 128 * k) : 0.0f;
            }
#pragma unroll
            for (int b = 0; b < JB; b++) {
                const int m = rh + 2 * (jb + b);
                if (jb + b >= J || m >= M) continue;     // uniform per wavefront
                double *ar = a.acc + (size_t)m * a.ld_acc + c0 + g;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const int n = c0 + 128 * k + g;
                    if (n < c1) ar[128 * k] = 0.0;
                    if constexpr (EPI == VX_EPI_STORE) {
                        if (n < c1 && (!e.last_only || m == M - 1))
                            e.x[(size_t)(e.last_only ? 0 : m) * e.ldx + n] = v[b][k];
                    } else {
                        // q | k | v element n; the rotation partner of an
                        // element is the neighbouring lane (n ^ 1)
                        const int region = n < qd ? 0 : (n < qd + kvd ? 1 : 2);
                        const int el = region == 0 ? n : (region == 1 ? n - qd : n - qd - kvd);
                        const float *bias = region == 0 ? e.bq : (region == 1 ? e.bk : e.bv);
                        float x = v[b][k];
                        if (n < c1 && bias) x += bias[el];
                        const float xp = __shfl_xor(x, 1, 64);
                        if (n >= c1) continue;
                        const int rope_pos = e.n_past + m;
                        const int pos = rope_pos < e.n_ctx ? rope_pos : e.n_ctx - 1;
                        float o = x;
                        if (region < 2) {
                            const int i = (el % e.hd) / 2;
                            const float c = e.cs[(size_t)rope_pos * half + i];
                            const float sn = e.sn[(size_t)rope_pos * half + i];
                            o = (el & 1) ? vx_rope_rot(xp, x, c, sn).y : vx_rope_rot(x, xp, c, sn).x;
                        }
                        float *dst = region == 0 ? e.q_out + (size_t)m * qd + el
                                                 : (region == 1 ? e.kc : e.vc) + (size_t)pos * kvd + el;
                        *dst = o;
                    }
                }
            }
        }
    } else if constexpr (EPI == VX_EPI_RESID || EPI == VX_EPI_SWIGLU) {
        // RESID: x[m] += y over columns [c0, c0 + VX_CHUNK), the next panel
        // from w.x; SWIGLU: h over h indices [c0, c0 + VX_CHUNK) into the h
        // rows, then its panel.
        const int n_cols = EPI == VX_EPI_RESID ? a.n_out : e.ldh;   // d or F
        const int c1 = min(c0 + VX_CHUNK, n_cols);
        float *rows = EPI == VX_EPI_RESID ? e.x : e.h;
        const int ldr = EPI == VX_EPI_RESID ? e.ldx : e.ldh;
        double ss_part[J];
        float am_part[J];
        float wv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int n = c0 + 128 * k + g;
            wv[k] = (EPI == VX_EPI_RESID && e.w && n < c1) ? e.w[n] : 1.0f;
        }
#pragma unroll
        for (int j = 0; j < J; j++) {
            ss_part[j] = 0.0;
            am_part[j] = 0.0f;
        }
#pragma unroll
        for (int jb = 0; jb < J; jb += JB) {
            float y[JB][8], u[JB][8];
#pragma unroll
            for (int b = 0; b < JB; b++) {
                const int m = rh + 2 * (jb + b);
                if (jb + b >= J || m >= M) continue;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const int n = c0 + 128 * k + g;
                    y[b][k] = u[b][k] = 0.0f;
                    if (n >= c1) continue;
                    if constexpr (EPI == VX_EPI_RESID) {
                        y[b][k] = (float)vx_load_agent(a.acc + (size_t)m * a.ld_acc + n);
                        u[b][k] = e.x[(size_t)m * e.ldx + n];
                    } else {
                        // h index n -> gate row 32(n/16) + n%16, up row 16 further
                        const double *ar = a.acc + (size_t)m * a.ld_acc + 32 * (n / 16) + n % 16;
                        y[b][k] = (float)vx_load_agent(ar);
                        u[b][k] = (float)vx_load_agent(ar + 16);
                    }
                }
            }
#pragma unroll
            for (int b = 0; b < JB; b++) {
                const int j = jb + b, m = rh + 2 * j;
                if (j >= J || m >= M) continue;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const int n = c0 + 128 * k + g;
                    if (n >= c1) continue;
                    float r;
                    if constexpr (EPI == VX_EPI_RESID) {
                        a.acc[(size_t)m * a.ld_acc + n] = 0.0;
                        r = u[b][k] + y[b][k];
                        ss_part[j] += (double)r * (double)r;
                        am_part[j] = fmaxf(am_part[j], fabsf(wv[k] * r));
                    } else {
                        double *ar = a.acc + (size_t)m * a.ld_acc + 32 * (n / 16) + n % 16;
                        ar[0] = 0.0;
                        ar[16] = 0.0;
                        const float sgl = vx_silu(y[b][k]);
                        r = fabsf(sgl) < e.thr ? 0.0f : sgl * u[b][k];
                        am_part[j] = fmaxf(am_part[j], fabsf(r));
                    }
                    rows[(size_t)m * ldr + n] = r;
                }
            }
        }
        // every thread's stores of pass 1 complete before the workgroup
        // reads them back (the row statistics end with a barrier)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        vx_epi_row_stats<M>(ss_part, am_part, EPI == VX_EPI_RESID ? e.ss : nullptr, e.pan_rs,
                            e.pan_rs_ld, sg, lds, scl);
        const int n0 = c0 + 8 * g;
        if (n0 >= c1) return;
        float w8[8];
#pragma unroll
        for (int k = 0; k < 8; k++) w8[k] = 1.0f;
        if (EPI == VX_EPI_RESID && e.w) {
            const float4 w0 = *(const float4 *)(e.w + n0), w1 = *(const float4 *)(e.w + n0 + 4);
            w8[0] = w0.x; w8[1] = w0.y; w8[2] = w0.z; w8[3] = w0.w;
            w8[4] = w1.x; w8[5] = w1.y; w8[6] = w1.z; w8[7] = w1.w;
        }
#pragma unroll
        for (int jb = 0; jb < J; jb += JB) {
            float r[JB][8];
#pragma unroll
            for (int b = 0; b < JB; b++) {
                const int m = rh + 2 * (jb + b);
                if (jb + b >= J || m >= M) continue;
                const float *rr = rows + (size_t)m * ldr + n0;
                const float4 r0 = *(const float4 *)rr, r1 = *(const float4 *)(rr + 4);
                r[b][0] = r0.x; r[b][1] = r0.y; r[b][2] = r0.z; r[b][3] = r0.w;
                r[b][4] = r1.x; r[b][5] = r1.y; r[b][6] = r1.z; r[b][7] = r1.w;
            }
#pragma unroll
            for (int b = 0; b < JB; b++) {
                const int m = rh + 2 * (jb + b);
                if (jb + b >= J || m >= M) continue;
                const float sc = scl[m];
                float pv[8];
#pragma unroll
                for (int k = 0; k < 8; k++) pv[k] = w8[k] * r[b][k] * sc;
                vx_panel_store(e.pan, M, n0 / 8, m, pv);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// rows -> panel with chunk scales (first layer's input, tests)
// ---------------------------------------------------------------------------
// Workgroup = (chunk of VX_CHUNK columns, row m), 128 threads x 8 columns.
__global__ __launch_bounds__(128) void vx_rows_xpanel_kernel(const float *__restrict__ x, int ldx, int M,
                                                             int K, const float *__restrict__ w,
                                                             double *ss, uint4 *pan, float *rs, int rs_ld)
{
    __shared__ double r_ss[2];
    __shared__ float r_am[2];
    __shared__ float s_in;
    const int chunk = blockIdx.x, m = blockIdx.y;
    const int c = chunk * VX_CHUNK + 8 * threadIdx.x;
    const bool ok = c < K;
    float v[8];
    double sq = 0.0;
    float am = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = 0.0f;
    if (ok) {
        const float *xr = x + (size_t)m * ldx + c;
        const float4 x0 = *(const float4 *)xr, x1 = *(const float4 *)(xr + 4);
        const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int k = 0; k < 8; k++) {
            sq += (double)xv[k] * (double)xv[k];
            v[k] = w ? w[c + k] * xv[k] : xv[k];
            am = fmaxf(am, fabsf(v[k]));
        }
    }
    sq = vx_wave_sum_f64(sq);
    am = vx_wave_max(am);
    if ((threadIdx.x & 63) == 0) {
        r_ss[threadIdx.x >> 6] = sq;
        r_am[threadIdx.x >> 6] = am;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        if (ss) atomicAdd(&ss[m], r_ss[0] + r_ss[1]);
        float si, so;
        vx_chunk_scale(fmaxf(r_am[0], r_am[1]), &si, &so);
        rs[m * rs_ld + chunk] = so;
        s_in = si;
    }
    __syncthreads();
    if (!ok) return;
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] *= s_in;
    vx_panel_store(pan, M, c / 8, m, v);
}

extern "C" int vxh_xpanel_alloc(vxh_xpanel *p, int max_M, int K)
{
    memset(p, 0, sizeof(*p));
    p->K = K;
    if (max_M < 1 || max_M > 16 || K % 32 || K > VXH_MAX_K)
        return vxh_fail(VXH_ERR_PARAM, "xpanel_alloc: M %d K %d", max_M, K);
    int rc = vxh_malloc(&p->data, vxh_panel_bytes(max_M, K));
    if (rc) return rc;
    p->rs_ld = (K + VXH_CHUNK - 1) / VXH_CHUNK;
    rc = vxh_malloc((void **)&p->rs, sizeof(float) * 16 * (size_t)p->rs_ld);
    if (rc) return rc;
    // the padding block (odd block counts) must read as zeros
    VXH_CHECK(hipMemset(p->data, 0, vxh_panel_bytes(max_M, K)));
    VXH_CHECK(hipDeviceSynchronize());
    return VXH_OK;
}

extern "C" int vxh_xpanel_free(vxh_xpanel *p)
{
    vxh_free(p->data);
    vxh_free(p->rs);
    memset(p, 0, sizeof(*p));
    return VXH_OK;
}

extern "C" int vxh_rows_xpanel(const float *x, int ldx, int M, int K, const float *norm_w,
                               vxh_xpanel *p, vxh_stream s)
{
    if (M < 1 || M > 16 || K != p->K || K % 32)
        return vxh_fail(VXH_ERR_PARAM, "rows_xpanel: M %d K %d (panel K %d)", M, K, p->K);
    p->M = M;
    dim3 grid((K + VXH_CHUNK - 1) / VXH_CHUNK, M);
    vx_rows_xpanel_kernel<<<grid, 128, 0, vxh_hs(s)>>>(x, ldx, M, K, norm_w, p->ss, (uint4 *)p->data,
                                                       p->rs, p->rs_ld);
    VXH_LAUNCHED();
    return VXH_OK;
}

// ---------------------------------------------------------------------------
// GEMM with a fused epilogue
// ---------------------------------------------------------------------------
extern "C" int vxh_gemm_fused(const vxh_qmat *W, const vxh_xpanel *X, int M, double *acc, int ld_acc,
                              int n_out, float scale, const vxh_fepi *e, vxh_event start,
                              vxh_event stop, vxh_stream s)
{
    if (M != X->M || M < 1 || M > 16)
        return vxh_fail(VXH_ERR_PARAM, "gemm_fused: M %d (panel M %d)", M, X->M);
    if (W->n_cols != X->K)
        return vxh_fail(VXH_ERR_PARAM, "gemm_fused: W has K %d, panel %d", W->n_cols, X->K);
    // the epilogues read groups of 8 accumulator columns: ld_acc covers n_out
    // rounded up to 32 (a STORE may end mid-group; the others end on a tile)
    if (n_out < 1 || n_out > W->n_rows || (n_out + 31) / 32 * 32 > ld_acc ||
        (e->kind != VXH_FEPI_STORE && n_out % 32))
        return vxh_fail(VXH_ERR_PARAM, "gemm_fused: n_out %d (rows %d, ld %d)", n_out, W->n_rows, ld_acc);
    const int sg_rows = (e->kind == VXH_FEPI_SWIGLU ? 2 : 1) * VXH_CHUNK;
    const int n_sg = (n_out + sg_rows - 1) / sg_rows;
    const int n_groups = (W->n_rows / 32 + 3) / 4;
    if ((size_t)(n_sg + n_groups) * VX_CNT_STRIDE > (size_t)e->n_counters)
        return vxh_fail(VXH_ERR_PARAM, "gemm_fused: %d super-groups + %d tile groups need %d counter words, have %d",
                        n_sg, n_groups, (n_sg + n_groups) * VX_CNT_STRIDE, e->n_counters);
    vx_gemm_args a;
    memset(&a, 0, sizeof(a));
    a.wq = (const uint4 *)W->qs;
    a.wcache = W->cached;
    a.wd = (const uint32_t *)W->d;
    a.panel = (const uint4 *)X->data;
    a.rscale = X->rs;
    a.rs_ld = X->rs_ld;
    a.rs_chunk = X->rs_ld > 1 ? VXH_CHUNK / 64 : 1 << 30;
    a.ss = X->ss;
    a.ss_K = X->K;
    a.acc = acc;
    a.ld_acc = ld_acc;
    a.n_out = n_out;
    a.scale = scale;
    vx_epi_args &p = a.e;
    p.cnt = e->counters;
    p.n_sg = n_sg;
    p.sg_groups = sg_rows / 128;
    hipStream_t st = vxh_hs(s);
    hipEvent_t e0 = (hipEvent_t)start, e1 = (hipEvent_t)stop;
    switch (e->kind) {
    case VXH_FEPI_STORE:
        p.x = e->y;
        p.ldx = e->ldy;
        p.last_only = e->last_row_only;
        return vx_dispatch<VX_EPI_STORE>(W, M, 0, a, st, e0, e1);
    case VXH_FEPI_RESID:
    case VXH_FEPI_SWIGLU: {
        vxh_xpanel *o = e->out_panel;
        const int K_next = e->kind == VXH_FEPI_RESID ? n_out : e->n_h;
        if (!o || o->K != K_next || o->rs_ld != (K_next + VXH_CHUNK - 1) / VXH_CHUNK)
            return vxh_fail(VXH_ERR_PARAM, "gemm_fused: output panel K %d, need %d", o ? o->K : -1, K_next);
        if (e->kind == VXH_FEPI_SWIGLU && (e->n_h % 8 || 2 * ((e->n_h + 15) / 16) * 16 > n_out))
            return vxh_fail(VXH_ERR_PARAM, "gemm_fused: swiglu F %d over %d rows", e->n_h, n_out);
        o->M = M;
        p.pan = (uint4 *)o->data;
        p.pan_rs = o->rs;
        p.pan_rs_ld = o->rs_ld;
        if (e->kind == VXH_FEPI_RESID) {
            p.w = e->norm_w;
            p.ss = o->ss;
            p.x = e->x;
            p.ldx = e->ldx;
            return vx_dispatch<VX_EPI_RESID>(W, M, 0, a, st, e0, e1);
        }
        if (!e->h || e->ldh != e->n_h)
            return vxh_fail(VXH_ERR_PARAM, "gemm_fused: swiglu needs h rows with ldh == F");
        p.h = e->h;
        p.ldh = e->n_h;
        p.thr = e->thr;
        return vx_dispatch<VX_EPI_SWIGLU>(W, M, 0, a, st, e0, e1);
    }
    case VXH_FEPI_ROPE:
        if (e->head_dim % 8 || e->n_past < 0 || e->n_past + M - 1 >= e->n_pos || e->n_ctx < 1 ||
            n_out != (e->n_heads + 2 * e->n_kv_heads) * e->head_dim)
            return vxh_fail(VXH_ERR_PARAM, "gemm_fused: rope over %d rows, heads %d/%d x %d, n_past %d, n_pos %d",
                            n_out, e->n_heads, e->n_kv_heads, e->head_dim, e->n_past, e->n_pos);
        p.n_past = e->n_past;
        p.n_ctx = e->n_ctx;
        p.n_heads = e->n_heads;
        p.n_kv = e->n_kv_heads;
        p.hd = e->head_dim;
        p.bq = e->bq;
        p.bk = e->bk;
        p.bv = e->bv;
        p.cs = e->cos_tab;
        p.sn = e->sin_tab;
        p.q_out = e->q_out;
        p.kc = e->k_cache;
        p.vc = e->v_cache;
        return vx_dispatch<VX_EPI_ROPE>(W, M, 0, a, st, e0, e1);
    default:
        return vxh_fail(VXH_ERR_PARAM, "gemm_fused: epilogue kind %d", e->kind);
    }
}
