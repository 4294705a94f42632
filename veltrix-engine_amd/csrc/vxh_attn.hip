// Attention block of the verify step: RoPE + KV-cache write, and causal
// attention of M query rows against the resident fp32 KV cache.
#include "vxh_internal.h"

// ---------------------------------------------------------------------------
// RoPE + KV write.  One thread per (row, pair) of q and k; v is copied.
// ---------------------------------------------------------------------------
__global__ void vx_rope_kv_kernel(const float *__restrict__ qkv, int ld_qkv, int M, int n_past,
                                  int n_ctx, int n_heads, int n_kv_heads, int hd,
                                  const float *__restrict__ bq, const float *__restrict__ bk,
                                  const float *__restrict__ bv, const float *__restrict__ cs,
                                  const float *__restrict__ sn, float *__restrict__ q_out,
                                  float *__restrict__ kc, float *__restrict__ vc)
{
    const int qd = n_heads * hd, kvd = n_kv_heads * hd;
    const int half = hd / 2;
    const int per_row = (qd + kvd) / 2 + kvd;   // q pairs, k pairs, v elements
    int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= M * per_row) return;
    int m = idx / per_row, r = idx % per_row;
    int rope_pos = n_past + m;
    int pos = rope_pos < n_ctx ? rope_pos : n_ctx - 1;
    const float *row = qkv + (size_t)m * ld_qkv;
    if (r < (qd + kvd) / 2) {
        int e = 2 * r;                       // element index within [q | k]
        bool isq = e < qd;
        int el = isq ? e : e - qd;
        int i = (el % hd) / 2;               // pair index within the head
        float a = row[e], b = row[e + 1];
        const float *bias = isq ? bq : bk;
        if (bias) { a += bias[el]; b += bias[el + 1]; }
        float c = cs[(size_t)rope_pos * half + i], s = sn[(size_t)rope_pos * half + i];
        float o0 = a * c - b * s;
        float o1 = a * s + b * c;
        if (isq) {
            q_out[(size_t)m * qd + el] = o0;
            q_out[(size_t)m * qd + el + 1] = o1;
        } else {
            kc[(size_t)pos * kvd + el] = o0;
            kc[(size_t)pos * kvd + el + 1] = o1;
        }
    } else {
        int el = r - (qd + kvd) / 2;
        float v = row[qd + kvd + el];
        if (bv) v += bv[el];
        vc[(size_t)pos * kvd + el] = v;
    }
}

extern "C" int vxh_rope_kv(const float *qkv, int ld_qkv, int M, int n_past, int n_ctx, int n_heads,
                           int n_kv_heads, int head_dim, const float *bq, const float *bk,
                           const float *bv, const float *cos_tab, const float *sin_tab, int n_pos,
                           float *q_out, float *k_cache_layer, float *v_cache_layer, vxh_stream s)
{
    if (M < 1 || head_dim % 2 || n_past < 0 || n_past + M - 1 >= n_pos)
        return vxh_fail(VXH_ERR_PARAM, "rope_kv: M %d n_past %d n_pos %d", M, n_past, n_pos);
    int qd = n_heads * head_dim, kvd = n_kv_heads * head_dim;
    int n = M * ((qd + kvd) / 2 + kvd);
    vx_rope_kv_kernel<<<(n + 255) / 256, 256, 0, vxh_hs(s)>>>(
        qkv, ld_qkv, M, n_past, n_ctx, n_heads, n_kv_heads, head_dim, bq, bk, bv, cos_tab, sin_tab,
        q_out, k_cache_layer, v_cache_layer);
    VXH_LAUNCHED();
    return VXH_OK;
}

// ---------------------------------------------------------------------------
// Verify attention.  Workgroup = (kv head g, chunk of ACH positions).  The
// G = n_heads/n_kv query heads of the group times the M rows form QM query
// vectors; K/V rows of the chunk are staged in LDS once and used by all of
// them.  Each workgroup writes (max, sum, acc[hd]) per query; the last
// workgroup of the kv head combines the chunks (online-softmax rescale).
// ---------------------------------------------------------------------------
#define ACH 32

__global__ __launch_bounds__(256) void vx_attention_kernel(
    const float *__restrict__ q, int M, int n_past, int n_ctx, int n_heads, int n_kv, int hd,
    int cap, const float *__restrict__ kc, const float *__restrict__ vc, float *__restrict__ out,
    int ld_out, int n_chunks, int qpg, int n_qg, float *__restrict__ part,
    unsigned *__restrict__ counters)
{
    extern __shared__ float sm[];
    __shared__ int s_last;
    const int per_g = n_chunks * n_qg;
    const int g = blockIdx.x / per_g;
    const int ch = (blockIdx.x % per_g) / n_qg, qg = blockIdx.x % n_qg;
    const int G = n_heads / n_kv;
    const int QM = G * M;
    const int q0 = qg * qpg;
    const int nq = min(qpg, QM - q0);       // queries of this workgroup: [q0, q0 + nq)
    const int kvd = n_kv * hd;
    const int t0 = ch * ACH;
    const int hdp = hd + 1;
    float *sq = sm;                       // [nq][hd]
    float *sk = sq + nq * hd;             // [ACH][hd+1]
    float *sv = sk + ACH * hdp;           // [ACH][hd]
    float *ss = sv + ACH * hd;            // [nq][ACH]
    const float scale = 1.0f / sqrtf((float)hd);

    for (int i = threadIdx.x; i < nq * hd; i += blockDim.x) {
        int qi = q0 + i / hd, d = i % hd;
        int hl = qi / M, m = qi % M;
        sq[i] = q[(size_t)m * n_heads * hd + (size_t)(g * G + hl) * hd + d];
    }
    for (int i = threadIdx.x; i < ACH * hd; i += blockDim.x) {
        int t = i / hd, d = i % hd;
        int ta = t0 + t;
        bool ok = ta < n_ctx;
        sk[t * hdp + d] = ok ? kc[(size_t)ta * kvd + (size_t)g * hd + d] : 0.0f;
        sv[t * hd + d] = ok ? vc[(size_t)ta * kvd + (size_t)g * hd + d] : 0.0f;
    }
    __syncthreads();

    for (int i = threadIdx.x; i < nq * ACH; i += blockDim.x) {
        int ql = i / ACH, t = i % ACH;
        int m = (q0 + ql) % M;
        int pos = n_past + m < n_ctx ? n_past + m : n_ctx - 1;
        int cs = pos + 1;
        if (cap > 0 && cs > cap) cs = cap;
        float sc = -INFINITY;
        if (t0 + t < cs) {
            float a = 0.0f;
            const float *qv = sq + ql * hd;
            const float *kv = sk + t * hdp;
            for (int d = 0; d < hd; d++) a = fmaf(qv[d], kv[d], a);
            sc = a * scale;
        }
        ss[i] = sc;
    }
    __syncthreads();

    float *pstat = part + ((size_t)g * n_chunks + ch) * QM * (hd + 2);
    for (int ql = threadIdx.x; ql < nq; ql += blockDim.x) {
        float mx = -INFINITY;
        for (int t = 0; t < ACH; t++) mx = fmaxf(mx, ss[ql * ACH + t]);
        float l = 0.0f;
        for (int t = 0; t < ACH; t++) {
            float e = mx == -INFINITY ? 0.0f : expf(ss[ql * ACH + t] - mx);
            ss[ql * ACH + t] = e;
            l += e;
        }
        pstat[(size_t)(q0 + ql) * (hd + 2) + 0] = mx;
        pstat[(size_t)(q0 + ql) * (hd + 2) + 1] = l;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nq * hd; i += blockDim.x) {
        int ql = i / hd, d = i % hd;
        float a = 0.0f;
        for (int t = 0; t < ACH; t++) a = fmaf(ss[ql * ACH + t], sv[t * hd + d], a);
        pstat[(size_t)(q0 + ql) * (hd + 2) + 2 + d] = a;
    }

    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned prev = __hip_atomic_fetch_add(&counters[g], 1u, __ATOMIC_ACQ_REL,
                                               __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == (unsigned)(per_g - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const float *pg = part + (size_t)g * n_chunks * QM * (hd + 2);
    for (int i = threadIdx.x; i < QM * hd; i += blockDim.x) {
        int qi = i / hd, d = i % hd;
        int hl = qi / M, m = qi % M;
        float gm = -INFINITY;
        for (int c2 = 0; c2 < n_chunks; c2++) gm = fmaxf(gm, pg[((size_t)c2 * QM + qi) * (hd + 2)]);
        float l = 0.0f, a = 0.0f;
        for (int c2 = 0; c2 < n_chunks; c2++) {
            const float *pc = pg + ((size_t)c2 * QM + qi) * (hd + 2);
            float cm = pc[0];
            if (cm == -INFINITY) continue;
            float f = expf(cm - gm);
            l = fmaf(f, pc[1], l);
            a = fmaf(f, pc[2 + d], a);
        }
        out[(size_t)m * ld_out + (size_t)(g * G + hl) * hd + d] = a * (1.0f / (l + 1e-10f));
    }
    if (threadIdx.x == 0) counters[g] = 0u;
}

// LDS of a workgroup holding nq queries; the query split keeps it <= 64 KiB.
static size_t vx_attn_lds(int nq, int hd)
{
    return sizeof(float) * ((size_t)nq * hd + (size_t)ACH * (hd + 1) + (size_t)ACH * hd + (size_t)nq * ACH);
}

static int vx_attn_qpg(int hd)
{
    long room = 65536 / 4 - (long)ACH * (2 * hd + 1);
    return room > 0 ? (int)(room / (hd + ACH)) : 0;
}

extern "C" size_t vxh_attention_workspace_floats(int M, int n_ctx, int cap, int n_heads,
                                                 int n_kv_heads, int head_dim)
{
    int ctx = n_ctx;
    if (cap > 0 && ctx > cap) ctx = cap;
    int n_chunks = (ctx + ACH - 1) / ACH;
    return (size_t)n_kv_heads * n_chunks * (n_heads / n_kv_heads) * M * (head_dim + 2);
}

extern "C" int vxh_attention(const float *q, int M, int n_past, int n_ctx, int n_heads,
                             int n_kv_heads, int head_dim, int cap, const float *kc,
                             const float *vc, float *out, int ld_out, vxh_workspace *ws,
                             vxh_stream s)
{
    if (M < 1 || n_kv_heads < 1 || n_heads % n_kv_heads)
        return vxh_fail(VXH_ERR_PARAM, "attention: M %d heads %d kv %d", M, n_heads, n_kv_heads);
    int last = n_past + M - 1 < n_ctx ? n_past + M - 1 : n_ctx - 1;
    int ctx = last + 1;
    if (cap > 0 && ctx > cap) ctx = cap;
    int n_chunks = (ctx + ACH - 1) / ACH;
    int G = n_heads / n_kv_heads;
    int QM = G * M;
    int qpg = vx_attn_qpg(head_dim);
    if (qpg < 1) return vxh_fail(VXH_ERR_UNSUPPORTED, "attention: head_dim %d too large", head_dim);
    if (qpg > QM) qpg = QM;
    int n_qg = (QM + qpg - 1) / qpg;
    size_t need = (size_t)n_kv_heads * n_chunks * QM * (head_dim + 2);
    if (need > ws->part_floats || n_kv_heads > ws->n_counters)
        return vxh_fail(VXH_ERR_PARAM, "attention workspace too small (%zu floats needed)", need);
    size_t lds = vx_attn_lds(qpg, head_dim);
    vx_attention_kernel<<<n_kv_heads * n_chunks * n_qg, 256, lds, vxh_hs(s)>>>(
        q, M, n_past, n_ctx, n_heads, n_kv_heads, head_dim, cap, kc, vc, out, ld_out, n_chunks, qpg,
        n_qg, ws->part, ws->counters);
    VXH_LAUNCHED();
    return VXH_OK;
}

__global__ void vx_add_rows_kernel(float *__restrict__ y, int ldy, const float *__restrict__ x,
                                   int ldx, int n)
{
    int m = blockIdx.y;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        y[(size_t)m * ldy + i] += x[(size_t)m * ldx + i];
}

extern "C" int vxh_add_rows(float *y, int ldy, const float *x, int ldx, int M, int n, vxh_stream s)
{
    if (M <= 0 || n <= 0) return VXH_OK;
    int gx = (n + 255) / 256;
    if (gx > 64) gx = 64;
    vx_add_rows_kernel<<<dim3(gx, M), 256, 0, vxh_hs(s)>>>(y, ldy, x, ldx, n);
    VXH_LAUNCHED();
    return VXH_OK;
}

__global__ void vx_copy_rows_kernel(float *__restrict__ d, int ldd, const float *__restrict__ x,
                                    int ldx, int n)
{
    int m = blockIdx.y;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        d[(size_t)m * ldd + i] = x[(size_t)m * ldx + i];
}

extern "C" int vxh_copy_rows(float *dst, int ld_dst, const float *src, int ld_src, int M, int n,
                             vxh_stream s)
{
    if (M <= 0 || n <= 0) return VXH_OK;
    int gx = (n + 255) / 256;
    if (gx > 64) gx = 64;
    vx_copy_rows_kernel<<<dim3(gx, M), 256, 0, vxh_hs(s)>>>(dst, ld_dst, src, ld_src, n);
    VXH_LAUNCHED();
    return VXH_OK;
}

__global__ void vx_fill_rows_kernel(float *__restrict__ y, int ld, int M, int col0, int n, float v)
{
    int m = blockIdx.y;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        y[(size_t)m * ld + col0 + i] = v;
}

extern "C" int vxh_fill_rows(float *y, int ld, int M, int col0, int n, float value, vxh_stream s)
{
    if (M <= 0 || n <= 0) return VXH_OK;
    int gx = (n + 255) / 256;
    if (gx > 128) gx = 128;
    vx_fill_rows_kernel<<<dim3(gx, M), 256, 0, vxh_hs(s)>>>(y, ld, M, col0, n, value);
    VXH_LAUNCHED();
    return VXH_OK;
}
