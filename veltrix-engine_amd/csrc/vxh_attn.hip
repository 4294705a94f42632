// Attention block of the verify step: RoPE + KV-cache write, and causal
// attention of M query rows against the resident fp32 KV cache.
#include <string.h>

#include "vxh_internal.h"

// ---------------------------------------------------------------------------
// RoPE + KV write.  One thread per (row, pair) of q and k; v is copied.  The
// q/k/v rows are read from the fp64 GEMM accumulator, rounded to fp32 (the
// reference's GEMV output) and cleared.
// ---------------------------------------------------------------------------
__global__ void vx_rope_kv_kernel(double *__restrict__ qkv, int ld_qkv, int M, int n_past,
                                  int n_ctx, int n_heads, int n_kv_heads, int hd,
                                  const float *__restrict__ bq, const float *__restrict__ bk,
                                  const float *__restrict__ bv, const float *__restrict__ cs,
                                  const float *__restrict__ sn, const double *__restrict__ ss,
                                  int ss_K, float *__restrict__ q_out, float *__restrict__ kc,
                                  float *__restrict__ vc)
{
    const int qd = n_heads * hd, kvd = n_kv_heads * hd;
    const int half = hd / 2;
    const int per_row = (qd + kvd) / 2 + kvd;   // q pairs, k pairs, v elements
    int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= M * per_row) return;
    int m = idx / per_row, r = idx % per_row;
    int rope_pos = n_past + m;
    int pos = rope_pos < n_ctx ? rope_pos : n_ctx - 1;
    double *row = qkv + (size_t)m * ld_qkv;
    const float rin = ss ? vx_rms_inv((float)ss[m], ss_K) : 1.0f;   // deferred RMSNorm
    if (r < (qd + kvd) / 2) {
        int e = 2 * r;                       // element index within [q | k]
        bool isq = e < qd;
        int el = isq ? e : e - qd;
        int i = (el % hd) / 2;               // pair index within the head
        double2 ab = *(const double2 *)(row + e);
        *(double2 *)(row + e) = make_double2(0.0, 0.0);
        const float *bias = isq ? bq : bk;
        const float a = vx_norm_bias(ab.x, rin, bias, el), b = vx_norm_bias(ab.y, rin, bias, el + 1);
        float c = cs[(size_t)rope_pos * half + i], s = sn[(size_t)rope_pos * half + i];
        const float2 o = vx_rope_rot(a, b, c, s);
        if (isq) {
            *(float2 *)(q_out + (size_t)m * qd + el) = o;
        } else {
            *(float2 *)(kc + (size_t)pos * kvd + el) = o;
        }
    } else {
        int el = r - (qd + kvd) / 2;
        const float v = vx_norm_bias(row[qd + kvd + el], rin, bv, el);
        row[qd + kvd + el] = 0.0;
        vc[(size_t)pos * kvd + el] = v;
    }
}

extern "C" int vxh_rope_kv_norm(double *qkv, int ld_qkv, int M, int n_past, int n_ctx, int n_heads,
                                int n_kv_heads, int head_dim, const float *bq, const float *bk,
                                const float *bv, const float *cos_tab, const float *sin_tab, int n_pos,
                                const double *ss, int ss_K, float *q_out, float *k_cache_layer,
                                float *v_cache_layer, vxh_stream s)
{
    if (M < 1 || head_dim % 2 || ld_qkv % 2 || n_past < 0 || n_past + M - 1 >= n_pos)
        return vxh_fail(VXH_ERR_PARAM, "rope_kv: M %d n_past %d n_pos %d", M, n_past, n_pos);
    if (ss && ss_K < 1) return vxh_fail(VXH_ERR_PARAM, "rope_kv: norm length %d", ss_K);
    int qd = n_heads * head_dim, kvd = n_kv_heads * head_dim;
    int n = M * ((qd + kvd) / 2 + kvd);
    vx_rope_kv_kernel<<<(n + 255) / 256, 256, 0, vxh_hs(s)>>>(
        qkv, ld_qkv, M, n_past, n_ctx, n_heads, n_kv_heads, head_dim, bq, bk, bv, cos_tab, sin_tab,
        ss, ss_K, q_out, k_cache_layer, v_cache_layer);
    VXH_LAUNCHED();
    return VXH_OK;
}

extern "C" int vxh_rope_kv(double *qkv, int ld_qkv, int M, int n_past, int n_ctx, int n_heads,
                           int n_kv_heads, int head_dim, const float *bq, const float *bk,
                           const float *bv, const float *cos_tab, const float *sin_tab, int n_pos,
                           float *q_out, float *k_cache_layer, float *v_cache_layer, vxh_stream s)
{
    return vxh_rope_kv_norm(qkv, ld_qkv, M, n_past, n_ctx, n_heads, n_kv_heads, head_dim, bq, bk, bv,
                            cos_tab, sin_tab, n_pos, nullptr, 0, q_out, k_cache_layer, v_cache_layer, s);
}

// ---------------------------------------------------------------------------
// Verify attention, split over the context.  Workgroup = (kv head g, chunk
// of ACH positions, query group).  The G = n_heads/n_kv query heads of the
// kv head times the M rows form QM query vectors; the chunk's K and V rows
// are loaded once (all loads issued before the first use) into LDS and used
// by all of them.  Scores: one thread per (query, position), float4 LDS
// reads; softmax of a query across its 32 lanes with shuffles; P.V: one
// thread per (query, 4 channels).  Each workgroup writes (max, sum, acc[hd])
// per query at a stride of hd + 4 floats (acc 16-byte aligned at offset 4);
// a second kernel combines the chunks with the online-softmax rescale.
// ---------------------------------------------------------------------------
#define ACH 32
#define ATT_THREADS 256
#define ATT_MAX_HD 128
#define PART_STRIDE(hd) ((hd) + 4)

// QKV variant: q and this forward's own k/v rows come straight from the fp64
// q|k|v GEMM sums (deferred RMSNorm, biases and RoPE applied on the way, as
// vx_rope_kv_kernel does), and the workgroups of query group 0 store the new
// k/v rows into the cache.
struct vx_qkv_args {
    const double *qkv;
    int ld;
    const double *ss;       // NULL: no deferred RMSNorm
    int ss_K;
    const float *bq, *bk, *bv;
    const float *cs, *sn;   // RoPE tables [n_pos][hd/2]
};

// Elements col..col+3 of row m of the sums, times rin plus bias[el..el+3],
// rotated as the pairs i, i+1 of a head at rope position rp (rot = false: v).
__device__ __forceinline__ float4 vx_qkv4(const vx_qkv_args &a, int m, int col, int el, int i, int rp,
                                          int half, const float *bias, bool rot)
{
    const float rin = a.ss ? vx_rms_inv((float)a.ss[m], a.ss_K) : 1.0f;
    const double *r = a.qkv + (size_t)m * a.ld + col;
    const double2 p0 = *(const double2 *)r, p1 = *(const double2 *)(r + 2);
    const float x0 = vx_norm_bias(p0.x, rin, bias, el), x1 = vx_norm_bias(p0.y, rin, bias, el + 1);
    const float x2 = vx_norm_bias(p1.x, rin, bias, el + 2), x3 = vx_norm_bias(p1.y, rin, bias, el + 3);
    if (!rot) return make_float4(x0, x1, x2, x3);
    const float c0 = a.cs[(size_t)rp * half + i], s0 = a.sn[(size_t)rp * half + i];
    const float c1 = a.cs[(size_t)rp * half + i + 1], s1 = a.sn[(size_t)rp * half + i + 1];
    const float2 o0 = vx_rope_rot(x0, x1, c0, s0), o1 = vx_rope_rot(x2, x3, c1, s1);
    return make_float4(o0.x, o0.y, o1.x, o1.y);
}

template <bool QKV>
__global__ __launch_bounds__(ATT_THREADS) void vx_attention_kernel(
    const float *__restrict__ q, int M, int n_past, int n_ctx, int n_heads, int n_kv, int hd,
    int cap, float *__restrict__ kc, float *__restrict__ vc, int n_chunks, int n_chunks_w, int qpg,
    int n_qg, float *__restrict__ part, vx_qkv_args qa)
{
    // chunks [n_chunks, n_chunks_w) (QKV, attention cap below the new rows)
    // only store the new k/v rows
    extern __shared__ float4 sm4[];
    const int per_g = n_chunks_w * n_qg;
    const int g = blockIdx.x / per_g;
    const int ch = (blockIdx.x % per_g) / n_qg, qg = blockIdx.x % n_qg;
    if (ch >= n_chunks && qg != 0) return;
    const int G = n_heads / n_kv;
    const int QM = G * M;
    const int q0 = qg * qpg;
    const int nq = min(qpg, QM - q0);       // queries of this workgroup: [q0, q0 + nq)
    const int kvd = n_kv * hd;
    const int t0 = ch * ACH;
    const int hd4 = hd / 4, kp4 = hd4 + 1;  // K rows padded by one float4
    float4 *sq4 = sm4;                      // [nq][hd4]
    float4 *sk4 = sq4 + nq * hd4;           // [ACH][kp4]
    float4 *sv4 = sk4 + ACH * kp4;          // [ACH][hd4]
    float *sp = (float *)(sv4 + ACH * hd4); // [nq][ACH]
    const float scale = 1.0f / sqrtf((float)hd);

    // K/V chunk: ACH*hd/4 float4 each, at most 4 per thread; rows past the
    // cache end read as zeros (their scores are masked below)
    constexpr int KV4 = ACH * ATT_MAX_HD / 4 / ATT_THREADS;
    float4 kr[KV4], vr[KV4];
    const int qd = n_heads * hd, half = hd / 2;
#pragma unroll
    for (int j = 0; j < KV4; j++) {
        const int i = j * ATT_THREADS + threadIdx.x;
        const int t = i / hd4, d4 = i % hd4;
        const int pos = t0 + t;
        const bool ok = t < ACH && pos < n_ctx;
        const size_t off = (size_t)pos * kvd + (size_t)g * hd + 4 * d4;
        // QKV: the row of this forward whose k/v land at pos (rows sit at
        // min(n_past + m, n_ctx - 1); only a one-row forward is clamped)
        int mn = -1;
        if (QKV && ok) {
            mn = pos - n_past;
            if (mn >= M) mn = -1;
            if (mn < 0 && n_past >= n_ctx && pos == n_ctx - 1) mn = 0;
        }
        if (mn >= 0) {
            const int el = g * hd + 4 * d4;
            kr[j] = vx_qkv4(qa, mn, qd + el, el, 2 * d4, n_past + mn, half, qa.bk, true);
            vr[j] = vx_qkv4(qa, mn, qd + kvd + el, el, 0, 0, half, qa.bv, false);
            if (qg == 0) {
                *(float4 *)(kc + off) = kr[j];
                *(float4 *)(vc + off) = vr[j];
            }
        } else {
            kr[j] = ok ? *(const float4 *)(kc + off) : make_float4(0.f, 0.f, 0.f, 0.f);
            vr[j] = ok ? *(const float4 *)(vc + off) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    if (ch >= n_chunks) return;
    for (int i = threadIdx.x; i < nq * hd4; i += ATT_THREADS) {
        const int ql = i / hd4, d4 = i % hd4;
        const int qi = q0 + ql, hl = qi / M, m = qi % M;
        const int el = (g * G + hl) * hd + 4 * d4;
        if constexpr (QKV)
            sq4[ql * hd4 + d4] = vx_qkv4(qa, m, el, el, 2 * d4, n_past + m, half, qa.bq, true);
        else
            sq4[ql * hd4 + d4] = *(const float4 *)(q + (size_t)m * qd + el);
    }
#pragma unroll
    for (int j = 0; j < KV4; j++) {
        const int i = j * ATT_THREADS + threadIdx.x;
        const int t = i / hd4, d4 = i % hd4;
        if (t < ACH) {
            sk4[t * kp4 + d4] = kr[j];
            sv4[t * hd4 + d4] = vr[j];
        }
    }
    __syncthreads();

    // scores and the chunk's softmax statistics; a query's 32 positions are
    // the 32 lanes of one half-wave (ATT_THREADS and ACH are multiples of 32)
    const size_t ps = PART_STRIDE(hd);
    float *pstat = part + ((size_t)g * n_chunks + ch) * QM * ps;
    for (int i = threadIdx.x; i < nq * ACH; i += ATT_THREADS) {
        const int ql = i / ACH, t = i % ACH;
        const int m = (q0 + ql) % M;
        const int pos = n_past + m < n_ctx ? n_past + m : n_ctx - 1;
        int cs = pos + 1;
        if (cap > 0 && cs > cap) cs = cap;
        float sc = -INFINITY;
        if (t0 + t < cs) {
            const float4 *qv = sq4 + ql * hd4;
            const float4 *kv = sk4 + t * kp4;
            float a0 = 0.0f, a1 = 0.0f;
            for (int d4 = 0; d4 < hd4; d4++) {
                const float4 x = qv[d4], y = kv[d4];
                a0 = fmaf(x.x, y.x, a0);
                a1 = fmaf(x.y, y.y, a1);
                a0 = fmaf(x.z, y.z, a0);
                a1 = fmaf(x.w, y.w, a1);
            }
            sc = (a0 + a1) * scale;
        }
        float mx = sc;
        for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 32));
        const float e = mx == -INFINITY ? 0.0f : expf(sc - mx);
        float l = e;
        for (int o = 16; o > 0; o >>= 1) l += __shfl_xor(l, o, 32);
        sp[ql * ACH + t] = e;
        if (t == 0) {
            pstat[(size_t)(q0 + ql) * ps + 0] = mx;
            pstat[(size_t)(q0 + ql) * ps + 1] = l;
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nq * hd4; i += ATT_THREADS) {
        const int ql = i / hd4, d4 = i % hd4;
        const float *pr = sp + ql * ACH;
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
        for (int t = 0; t < ACH; t++) {
            const float p = pr[t];
            const float4 v = sv4[t * hd4 + d4];
            a.x = fmaf(p, v.x, a.x);
            a.y = fmaf(p, v.y, a.y);
            a.z = fmaf(p, v.z, a.z);
            a.w = fmaf(p, v.w, a.w);
        }
        *(float4 *)(pstat + (size_t)(q0 + ql) * ps + 4 + 4 * d4) = a;
    }
}

// fp32-MFMA variant for head_dim 64 and 128: one wavefront per (kv head,
// group of <= 16 query vectors, chunk of ACH positions), no LDS.  Scores and
// P.V run on v_mfma_f32_16x16x4_f32 (fp32 products and sums).  Lane l = n +
// 16 r (n = l % 16, r = l / 16):
//  * QK^T, per 16 positions and per (j, i): A = K[position n][16 j + 4 r + i],
//    B = q[query n][16 j + 4 r + i] (scaled by 1/sqrt(hd)); the result holds
//    score(position 4 r + i, query n) in item i of lane (n, r).
//  * P.V, per step s and chain c = 4 u + e: A = V[position 4 r + s][64 u +
//    4 n + e], B = the probability in item s of lane (n, r); chain c
//    accumulates output dim 64 u + 4 (4 r + i) + e of query n in item i.
// So every lane loads whole float4s: K rows 4 dims at a time (16 rows x 64 B
// per load), V rows as 4 rows x 256 contiguous bytes per load.
// The chunk's (max, sum, acc[hd]) per query go to the same partials as
// vx_attention_kernel writes (the combine kernels read either).
typedef float vx_f32x4 __attribute__((ext_vector_type(4)));

// Items of the q|k|v sums as the attention reads them: 4 consecutive
// elements of a row per item, RoPE'd as two adjacent pairs (rot) at the
// item's position, with the deferred RMSNorm of its row and its bias
// applied.  All loads of a batch are issued before the first use and every
// address is valid (callers clamp), so a wavefront pays one round trip.
template <int NB>
__device__ __forceinline__ void vx_qkv4_items(const vx_qkv_args &a, const int row[NB], const int col[NB],
                                              const int el[NB], const int pr[NB], const int rp[NB],
                                              const float *const bias[NB], const bool rot[NB], int half,
                                              float4 out[NB])
{
    double2 p0[NB], p1[NB];
    float4 b4[NB];
    float c0[NB], c1[NB], s0[NB], s1[NB];
    double ssv[NB];
#pragma unroll
    for (int u = 0; u < NB; u++) {
        const double *rs = a.qkv + (size_t)row[u] * a.ld;
        ssv[u] = *(a.ss ? a.ss + row[u] : rs);       // any valid address when there is no norm
        p0[u] = *(const double2 *)(rs + col[u]);
        p1[u] = *(const double2 *)(rs + col[u] + 2);
        b4[u] = *(const float4 *)(bias[u] ? bias[u] + el[u] : a.cs);
        const float *ct = a.cs + (size_t)rp[u] * half + pr[u], *st = a.sn + (size_t)rp[u] * half + pr[u];
        c0[u] = ct[0];
        c1[u] = ct[1];
        s0[u] = st[0];
        s1[u] = st[1];
    }
#pragma unroll
    for (int u = 0; u < NB; u++) {
        const float rin = a.ss ? vx_rms_inv((float)ssv[u], a.ss_K) : 1.0f;
        const bool bb = bias[u] != nullptr;
        const float x0 = bb ? fmaf((float)p0[u].x, rin, b4[u].x) : (float)p0[u].x * rin;
        const float x1 = bb ? fmaf((float)p0[u].y, rin, b4[u].y) : (float)p0[u].y * rin;
        const float x2 = bb ? fmaf((float)p1[u].x, rin, b4[u].z) : (float)p1[u].x * rin;
        const float x3 = bb ? fmaf((float)p1[u].y, rin, b4[u].w) : (float)p1[u].y * rin;
        if (rot[u]) {
            const float2 o0 = vx_rope_rot(x0, x1, c0[u], s0[u]), o1 = vx_rope_rot(x2, x3, c1[u], s1[u]);
            out[u] = make_float4(o0.x, o0.y, o1.x, o1.y);
        } else {
            out[u] = make_float4(x0, x1, x2, x3);
        }
    }
}

#define VX_ATT_MFMA_MAX_M VXH_ATTN_QKV_FAST_ROWS   // rows of a forward the QKV variant takes

// v where ok, else zeros (per component: a select of whole float4 array
// elements becomes a select of their addresses and puts the array in scratch)
__device__ __forceinline__ float4 vx_keep4(bool ok, float4 v)
{
    return make_float4(ok ? v.x : 0.0f, ok ? v.y : 0.0f, ok ? v.z : 0.0f, ok ? v.w : 0.0f);
}

// KV cache rows in fp32 (KH = false, the reference's cache) or IEEE fp16
// (KH = true, a flagged mode: round to nearest even on store, exact widening
// on load).  i is an element index, a multiple of 4.
// nt: a non-temporal load (a cache too large to stay in the caches between
// forwards should not evict what does).
template <bool KH, bool NT>
__device__ __forceinline__ float4 vx_kv_load4(const float *base, uint32_t i)
{
    // a 32-bit byte offset from the (uniform) base: the load takes the
    // scalar-base form, no 64-bit address arithmetic per lane
    const char *p = (const char *)base + (uint32_t)(i * (KH ? 2u : 4u));
    if constexpr (KH) {
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
        u32x2 h;
        if constexpr (NT) h = __builtin_nontemporal_load((const u32x2 *)p);
        else h = *(const u32x2 *)p;
        return make_float4(vx_half_bits_to_float(h.x & 0xFFFFu), vx_half_bits_to_float(h.x >> 16),
                           vx_half_bits_to_float(h.y & 0xFFFFu), vx_half_bits_to_float(h.y >> 16));
    } else {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        f32x4 v;
        if constexpr (NT) v = __builtin_nontemporal_load((const f32x4 *)p);
        else v = *(const f32x4 *)p;
        return make_float4(v.x, v.y, v.z, v.w);
    }
}
__device__ __forceinline__ uint32_t vx_half_bits(float x)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);   // round to nearest even
}
// the value a KV row element holds after a store and a load
template <bool KH>
__device__ __forceinline__ float4 vx_kv_round4(float4 v)
{
    if constexpr (KH)
        return make_float4(vx_half_bits_to_float(vx_half_bits(v.x)), vx_half_bits_to_float(vx_half_bits(v.y)),
                           vx_half_bits_to_float(vx_half_bits(v.z)), vx_half_bits_to_float(vx_half_bits(v.w)));
    else
        return v;
}
template <bool KH>
__device__ __forceinline__ void vx_kv_store4(float *base, size_t i, float4 v)
{
    if constexpr (KH)
        *(uint2 *)((uint16_t *)base + i) = make_uint2(vx_half_bits(v.x) | (vx_half_bits(v.y) << 16),
                                                      vx_half_bits(v.z) | (vx_half_bits(v.w) << 16));
    else
        *(float4 *)(base + i) = v;
}

// In the VGPR form, an MFMA whose destination overlaps one of its own A/B
// source registers computes wrong values; the compiler gives a chain's MFMA a
// destination of its own and may place it on a source that dies at that
// MFMA.  These empty asms keep every source of the chains live until all of
// their MFMAs have issued (they also read and write the accumulators, so they
// cannot move above them); no instruction is emitted.
template <int NJ>
__device__ __forceinline__ void vx_keep_past_o(vx_f32x4 (&O)[NJ], float4 v4)
{
    static_assert(NJ == 4 || NJ == 8, "P.V chains of head_dim 64 or 128");
    const vx_f32x4 v = __builtin_bit_cast(vx_f32x4, v4);
    if constexpr (NJ == 8)
        asm volatile("" : "+v"(O[0]), "+v"(O[1]), "+v"(O[2]), "+v"(O[3]), "+v"(O[4]), "+v"(O[5]), "+v"(O[6]),
                     "+v"(O[7]) : "v"(v));
    else
        asm volatile("" : "+v"(O[0]), "+v"(O[1]), "+v"(O[2]), "+v"(O[3]) : "v"(v));
}

template <int NJ>
__device__ __forceinline__ void vx_keep_past_o(vx_f32x4 (&O)[NJ], float v)
{
    if constexpr (NJ == 8)
        asm volatile("" : "+v"(O[0]), "+v"(O[1]), "+v"(O[2]), "+v"(O[3]), "+v"(O[4]), "+v"(O[5]), "+v"(O[6]),
                     "+v"(O[7]) : "v"(v));
    else
        asm volatile("" : "+v"(O[0]), "+v"(O[1]), "+v"(O[2]), "+v"(O[3]) : "v"(v));
}

template <bool QKV, int HD, bool KH = false, int NCW = 1, int NPG = 2, bool MERGE = false, bool NT = false>
__device__ __forceinline__ void vx_attention_mfma_body(
    const float *__restrict__ q, int M, int n_past, int n_ctx, int n_heads, int n_kv, int cap,
    float *__restrict__ kc, float *__restrict__ vc, int n_chunks, int n_chunks_w, int n_qg,
    float *__restrict__ part, vx_qkv_args qa)
{
    constexpr int NJ = HD / 16;      // K float4 per lane per 16 positions; also P.V chains
    constexpr int NV = HD / 16;      // V floats per lane per step
    constexpr int NV4 = NV / 4;
    constexpr int CH = NPG * 16;     // positions of one chunk (NPG groups of 16)
    constexpr int WCH = NCW * CH;    // positions of one wavefront (NCW chunks, walked in order)
    // V of the first chunk with its K (the wavefront holds both): at head_dim
    // 64, where the draft decode has too few wavefronts to hide a second round
    // trip, and whenever a wavefront walks several chunks (its V then streams
    // while the scores of the chunk run).  A one-chunk wavefront at head_dim
    // 128 loads V after issuing the score MFMAs, so K and V need not be live
    // together and 3 wavefronts fit a SIMD.
    constexpr bool V_EARLY = HD == 64 || NCW > 1;
    static_assert(HD == 64 || HD == 128, "head_dim 64 or 128");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, r = lane >> 4;
    // n_chunks / n_chunks_w count ACH-position chunks (attended / holding
    // rows to store); this kernel's wavefronts take WCH positions each
    const int nw_w = (n_chunks_w * ACH + WCH - 1) / WCH;   // wavefronts holding positions to store
    const int nw = (n_chunks * ACH + WCH - 1) / WCH;       // wavefronts with positions to attend
    const int ncg = (nw_w + 3) / 4;
    const int g = blockIdx.x / (n_qg * ncg);
    const int qg = (blockIdx.x / ncg) % n_qg;
    const int wg = blockIdx.x % ncg;
    const int ch = wg * 4 + wave;
    // QKV, MERGE: every wavefront reaches the workgroup barriers below
    if (!QKV && !MERGE && ch >= nw_w) return;
    const bool attend = ch < nw;
    const int G = n_heads / n_kv, QM = G * M;
    const int kvd = n_kv * HD, qd = n_heads * HD, half = HD / 2;
    const int t0 = ch * WCH;

    // K rows of positions tc + 16 pg + n (dims 16 j + 4 r .. + 3) and V rows
    // of positions tc + 16 pg + 4 r + s (dims 64 u + 4 n .. + 3) of chunk tc
    // from the cache; positions past the cache end read as zeros (with one
    // chunk per wavefront only a chunk that reaches past it -- wavefront-
    // uniform -- runs the selects; a branch between a multi-chunk wavefront's
    // loads would wait for the next chunk's K before this chunk's P.V).
    // Offsets are 32-bit element indices from the layer's cache base.
    float4 kr[NPG][NJ], vr[NPG][4][NV4];
    const uint32_t head0 = (uint32_t)(g * HD), ukvd = (uint32_t)kvd;
    auto load_k = [&](int tc) {
#pragma unroll
        for (int pg = 0; pg < NPG; pg++) {
            const int pos = tc + 16 * pg + n;
            const uint32_t off = (uint32_t)min(pos, n_ctx - 1) * ukvd + head0 + 4 * r;
#pragma unroll
            for (int j = 0; j < NJ; j++) kr[pg][j] = vx_kv_load4<KH, NT>(kc, off + 16 * j);
        }
        if (NCW > 1 || tc + 16 * NPG > n_ctx) {
#pragma unroll
            for (int pg = 0; pg < NPG; pg++) {
                const bool ok = tc + 16 * pg + n < n_ctx;
#pragma unroll
                for (int j = 0; j < NJ; j++) kr[pg][j] = vx_keep4(ok, kr[pg][j]);
            }
        }
    };
    auto load_v = [&](int tc) {
#pragma unroll
        for (int pg = 0; pg < NPG; pg++)
#pragma unroll
            for (int st = 0; st < 4; st++) {
                const int pv = tc + 16 * pg + 4 * r + st;
                const uint32_t ov = (uint32_t)min(pv, n_ctx - 1) * ukvd + head0 + 4 * n;
#pragma unroll
                for (int u = 0; u < NV4; u++) vr[pg][st][u] = vx_kv_load4<KH, NT>(vc, ov + 64 * u);
            }
        if (NCW > 1 || tc + 16 * NPG > n_ctx) {
#pragma unroll
            for (int pg = 0; pg < NPG; pg++)
#pragma unroll
                for (int st = 0; st < 4; st++) {
                    const bool okv = tc + 16 * pg + 4 * r + st < n_ctx;
#pragma unroll
                    for (int u = 0; u < NV4; u++) vr[pg][st][u] = vx_keep4(okv, vr[pg][st][u]);
                }
        }
    };
    load_k(t0);
    if constexpr (V_EARLY) load_v(t0);

    // query n of this group: q vector (hl, m), its causal length cs
    const int qi = qg * 16 + n;
    const bool qok = qi < QM;
    const int hl = qok ? qi / M : 0, m = qok ? qi % M : 0;
    const int head = g * G + hl;
    const int qpos = n_past + m < n_ctx ? n_past + m : n_ctx - 1;
    int cs = qpos + 1;
    if (cap > 0 && cs > cap) cs = cap;
    if (!qok) cs = 0;
    const float scale = 1.0f / sqrtf((float)HD);
    float4 qv[NJ];
    if constexpr (!QKV) {
        const float *qr = q + (size_t)m * qd + head * HD + 4 * r;
#pragma unroll
        for (int j = 0; j < NJ; j++) qv[j] = *(const float4 *)(qr + 16 * j);
#pragma unroll
        for (int j = 0; j < NJ; j++)
            qv[j] = vx_keep4(qok, make_float4(qv[j].x * scale, qv[j].y * scale, qv[j].z * scale, qv[j].w * scale));
    }

    // QKV: the workgroup derives its 16 q vectors (deferred RMSNorm, bias,
    // RoPE, 1/sqrt(hd)) once into LDS, and -- when one of its chunks holds a
    // row of this forward (at min(n_past + m, n_ctx - 1); only a one-row
    // forward is clamped) -- head g's new k/v rows too (query group 0 also
    // stores them into the cache); the wavefronts take them from LDS.
    bool has_new_wg = false;   // QKV: this workgroup's chunks hold rows of this forward
    // LDS (float4 units): the new k/v rows [row][k, v][d4] and the q vectors
    // (QKV), then the accumulators the workgroup merges (MERGE).  At head_dim
    // 128 the three would take 58 KB (2 workgroups per CU), so the merge
    // reuses the first two once every wavefront is past its chunks (one more
    // barrier); at 64 they fit side by side in 25 KB.
    constexpr int N_NEW = QKV ? VX_ATT_MFMA_MAX_M * 2 * (HD / 4) : 0, N_Q = QKV ? 16 * (HD / 4 + 1) : 0;
    constexpr int N_MRG = MERGE ? 3 * NJ * 64 : 0;
    constexpr bool ALIAS = QKV && MERGE && (N_NEW + N_Q + N_MRG) * 16 > 32768;
    constexpr int N_BUF0 = ALIAS ? (N_NEW + N_Q > N_MRG ? N_NEW + N_Q : N_MRG) : N_NEW + N_Q + N_MRG;
    constexpr int N_BUF = N_BUF0 > 0 ? N_BUF0 : 1;
    __shared__ float4 s_buf[N_BUF];
    float4 *const s_new = s_buf;
    // new row of this forward at cache position pos, or -1 (rows sit at
    // min(n_past + m, n_ctx - 1); only a one-row forward is clamped)
    auto new_row = [&](int pos) -> int {
        int mn = pos - n_past;
        if (mn >= M || pos >= n_ctx) mn = -1;
        if (mn < 0 && n_past >= n_ctx && pos == n_ctx - 1) mn = 0;
        return mn;
    };
    if constexpr (QKV) {
        constexpr int Q4 = HD / 4, QS = Q4 + 1;                      // float4 per row, padded stride
        float4 *const s_q = s_buf + N_NEW;
        constexpr int QI = 16 * Q4 / ATT_THREADS;                  // q items per thread (1 or 2)
        const int lo = n_past < n_ctx ? n_past : n_ctx - 1;
        const int hi = min(n_past + M - 1, n_ctx - 1);
        const int c0 = wg * 4 * WCH;
        const bool has_new = hi >= c0 && lo < c0 + 4 * WCH;          // uniform over the workgroup
        const int n_new = M * 2 * Q4;                                // new k/v items (row, k|v, float4)
        // new k/v item `it` of this forward: its q|k|v column, cache element,
        // RoPE pair and position
        auto new_item = [&](int it, int &row, int &col, int &el, int &pr, int &rp, const float *&bias, bool &rot) {
            const int d4 = it % Q4, kind = (it / Q4) % 2, mr = it / (2 * Q4);
            row = mr;
            el = g * HD + 4 * d4;
            col = (kind ? qd + kvd : qd) + el;
            pr = 2 * d4;
            rp = n_past + mr;
            bias = kind ? qa.bv : qa.bk;
            rot = kind == 0;
        };
        // the q items and the first new item of each thread load in one batch
        // (a workgroup holding new rows pays one round trip for both, not one
        // after the other); a thread without a first new item loads item 0,
        // whose addresses are those of a q item of row 0
        {
            constexpr int B = QI + 1;
            int row[B], col[B], el[B], pr[B], rp[B];
            bool ok[QI];
            const float *bias[B];
            bool rot[B];
#pragma unroll
            for (int u = 0; u < QI; u++) {
                const int it = threadIdx.x + u * ATT_THREADS, qn = it / Q4, d4 = it % Q4;
                const int qj = qg * 16 + qn;
                ok[u] = qj < QM;
                const int mj = ok[u] ? qj % M : 0, hj = ok[u] ? qj / M : 0;
                row[u] = mj;
                col[u] = (g * G + hj) * HD + 4 * d4;
                el[u] = col[u];
                pr[u] = 2 * d4;
                rp[u] = n_past + mj;
                bias[u] = qa.bq;
                rot[u] = true;
            }
            const bool first_new = has_new && (int)threadIdx.x < n_new;
            new_item(first_new ? (int)threadIdx.x : 0, row[QI], col[QI], el[QI], pr[QI], rp[QI], bias[QI], rot[QI]);
            float4 o[B];
            vx_qkv4_items<B>(qa, row, col, el, pr, rp, bias, rot, half, o);
#pragma unroll
            for (int u = 0; u < QI; u++) {
                const int it = threadIdx.x + u * ATT_THREADS;
                s_q[(it / Q4) * QS + it % Q4] =
                    vx_keep4(ok[u], make_float4(o[u].x * scale, o[u].y * scale, o[u].z * scale, o[u].w * scale));
            }
            if (first_new) {
                const int it = threadIdx.x;
                // the new row as the cache holds it (fp16 mode: rounded)
                s_new[it] = vx_kv_round4<KH>(o[QI]);
                if (qg == 0) {
                    const int kind = (it / Q4) % 2, pos = min(n_past + row[QI], n_ctx - 1);
                    vx_kv_store4<KH>(kind ? vc : kc, (size_t)pos * kvd + el[QI], o[QI]);
                }
            }
        }
        if (has_new) {
            for (int it0 = ATT_THREADS + threadIdx.x; it0 < n_new; it0 += 2 * ATT_THREADS) {
                int row[2], col[2], el[2], pr[2], rp[2];
                const float *bias[2];
                bool rot[2];
#pragma unroll
                for (int u = 0; u < 2; u++)
                    new_item(min(it0 + u * ATT_THREADS, n_new - 1), row[u], col[u], el[u], pr[u], rp[u], bias[u],
                             rot[u]);
                float4 o[2];
                vx_qkv4_items<2>(qa, row, col, el, pr, rp, bias, rot, half, o);
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int it = it0 + u * ATT_THREADS;
                    if (it >= n_new) continue;
                    s_new[it] = vx_kv_round4<KH>(o[u]);
                    if (qg == 0) {
                        const int kind = (it / Q4) % 2, pos = min(n_past + row[u], n_ctx - 1);
                        vx_kv_store4<KH>(kind ? vc : kc, (size_t)pos * kvd + el[u], o[u]);
                    }
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NJ; j++) qv[j] = s_q[n * QS + 4 * j + r];
        has_new_wg = has_new;
    }
    if (!MERGE && (ch >= nw_w || !attend)) return;

    // The wavefront's chunks in order, with the online-softmax rescale
    // (src/tensor.c:156-171 over the chunks): running max rm and sum rl of
    // query n, output accumulators O rescaled when the max grows.
    float rm = -INFINITY, rl = 0.0f;
    vx_f32x4 O[NJ];
#pragma unroll
    for (int c = 0; c < NJ; c++) O[c] = vx_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < NCW; cc++) {
        if (MERGE && !attend) break;
        const int tc = t0 + cc * CH;
        if (cc > 0) load_v(tc);        // this chunk's V streams while its scores run
        // this forward's own k rows from LDS (the cache rows may not be written yet)
        if (QKV && has_new_wg) {
#pragma unroll
            for (int pg = 0; pg < NPG; pg++) {
                const int mn = new_row(tc + 16 * pg + n);
                if (mn >= 0)
#pragma unroll
                    for (int j = 0; j < NJ; j++) kr[pg][j] = s_new[(mn * 2) * (HD / 4) + 4 * j + r];
            }
        }
        // scores of the chunk's positions: S[pg] item i = position 16 pg + 4 r + i
        vx_f32x4 S[NPG];
#pragma unroll
        for (int pg = 0; pg < NPG; pg++) {
            S[pg] = vx_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                S[pg] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[pg][j].x, qv[j].x, S[pg], 0, 0, 0);
                S[pg] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[pg][j].y, qv[j].y, S[pg], 0, 0, 0);
                S[pg] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[pg][j].z, qv[j].z, S[pg], 0, 0, 0);
                S[pg] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[pg][j].w, qv[j].w, S[pg], 0, 0, 0);
            }
#pragma unroll
            for (int j = 0; j < NJ; j++)
                asm volatile("" : "+v"(S[pg]) : "v"(__builtin_bit_cast(vx_f32x4, kr[pg][j])),
                             "v"(__builtin_bit_cast(vx_f32x4, qv[j])));
        }
        if (cc + 1 < NCW) load_k(tc + CH);        // the next chunk's K behind this chunk's V
        if constexpr (!V_EARLY) load_v(tc);
        if (QKV && has_new_wg) {
#pragma unroll
            for (int pg = 0; pg < NPG; pg++)
#pragma unroll
                for (int st = 0; st < 4; st++) {
                    const int mv = new_row(tc + 16 * pg + 4 * r + st);
                    if (mv >= 0)
#pragma unroll
                        for (int u = 0; u < NV4; u++) vr[pg][st][u] = s_new[(mv * 2 + 1) * (HD / 4) + n + 16 * u];
                }
        }
        // chunk statistics of query n against the running ones
        float sc[NPG][4];
        float cm = -INFINITY;
#pragma unroll
        for (int pg = 0; pg < NPG; pg++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = tc + 16 * pg + 4 * r + i;
                sc[pg][i] = t < cs ? S[pg][i] : -INFINITY;
                cm = fmaxf(cm, sc[pg][i]);
            }
        cm = vx_max_x32(vx_max_x16(cm));
        const float nm = fmaxf(rm, cm);
        float p[NPG][4], l = 0.0f;
#pragma unroll
        for (int pg = 0; pg < NPG; pg++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                p[pg][i] = nm == -INFINITY || sc[pg][i] == -INFINITY ? 0.0f : expf(sc[pg][i] - nm);
                l += p[pg][i];
            }
        l = vx_sum_x32(vx_sum_x16(l));
        if (cc == 0) {
            rl = l;
        } else {
            const float fo = rm == -INFINITY ? 0.0f : expf(rm - nm);
            rl = rl * fo + l;
#pragma unroll
            for (int c = 0; c < NJ; c++) O[c] *= fo;
        }
        rm = nm;

        // P.V; each step's sources stay live past its MFMAs (vx_keep_past_o)
#pragma unroll
        for (int pg = 0; pg < NPG; pg++)
#pragma unroll
            for (int st = 0; st < 4; st++) {
#pragma unroll
                for (int c = 0; c < NJ; c++) {
                    const float4 v4 = vr[pg][st][c / 4];
                    const float a = (c % 4) == 0 ? v4.x : (c % 4) == 1 ? v4.y : (c % 4) == 2 ? v4.z : v4.w;
                    O[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, p[pg][st], O[c], 0, 0, 0);
                }
#pragma unroll
                for (int u = 0; u < NV4; u++) vx_keep_past_o<NJ>(O, vr[pg][st][u]);
                vx_keep_past_o<NJ>(O, p[pg][st]);
            }
    }
    int pidx = ch, np = nw;    // this partial's index, partials per query
    if constexpr (MERGE) {
        // the workgroup's four wavefronts merged in LDS into one partial
        // (online-softmax rescale), written by wavefront 0
        __shared__ float s_ml[4][2][16];                                    // [wavefront][max, sum][query]
        vx_f32x4 *const s_o = (vx_f32x4 *)(s_buf + (ALIAS ? 0 : N_NEW + N_Q));   // [wavefront - 1][chain][lane]
        if (r == 0) {
            s_ml[wave][0][n] = rm;
            s_ml[wave][1][n] = rl;
        }
        if (ALIAS) __syncthreads();   // no wavefront reads the q vectors or new rows any more
        if (wave > 0)
#pragma unroll
            for (int c = 0; c < NJ; c++) s_o[((wave - 1) * NJ + c) * 64 + lane] = O[c];
        __syncthreads();
        if (wave != 0) return;
        float gm = rm;
#pragma unroll
        for (int w = 1; w < 4; w++) gm = fmaxf(gm, s_ml[w][0][n]);
        if (gm != -INFINITY) {
            const float f0 = rm == -INFINITY ? 0.0f : expf(rm - gm);
            rl *= f0;
#pragma unroll
            for (int c = 0; c < NJ; c++) O[c] *= f0;
#pragma unroll
            for (int w = 1; w < 4; w++) {
                const float mw = s_ml[w][0][n];
                const float f = mw == -INFINITY ? 0.0f : expf(mw - gm);
                rl = fmaf(f, s_ml[w][1][n], rl);
#pragma unroll
                for (int c = 0; c < NJ; c++) {
                    const vx_f32x4 v = s_o[((w - 1) * NJ + c) * 64 + lane];
                    O[c][0] = fmaf(f, v[0], O[c][0]);
                    O[c][1] = fmaf(f, v[1], O[c][1]);
                    O[c][2] = fmaf(f, v[2], O[c][2]);
                    O[c][3] = fmaf(f, v[3], O[c][3]);
                }
            }
        }
        rm = gm;
        pidx = wg;
        np = (nw + 3) / 4;
        if (wg >= np) return;
    }
    if (!qok) return;
    const size_t ps = PART_STRIDE(HD);
    float *pq = part + (((size_t)g * np + pidx) * QM + qi) * ps;
    if (r == 0) {
        pq[0] = rm;
        pq[1] = rl;
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int u = 0; u < NV4; u++)
            *(float4 *)(pq + 4 + 64 * u + 16 * r + 4 * i) =
                make_float4(O[4 * u][i], O[4 * u + 1][i], O[4 * u + 2][i], O[4 * u + 3][i]);
}

// Work per wavefront of the fp32-MFMA kernels.
// * NCW chunks per wavefront: the q-rows kernel at head_dim 128 (prompt
//   prefill: many query groups per head, so half the wavefronts still fill the
//   chip) walks two, V streaming behind K, and writes half the partials
//   (rocprofv3, 2048-token prefill: 205 -> 188 us per launch).  At head_dim
//   128 with q|k|v sums (the verify, nine rows) two chunks made the attention
//   24 -> 27.6 us per layer: half as many wavefronts, each with a longer K -> V
//   chain.
// * NPG groups of 16 positions per chunk, MERGE: the draft decode (head_dim
//   64, q|k|v sums, one row) has few wavefronts and each spends most of its
//   time on its own instructions, so its wavefronts take 16 positions and the
//   four of a workgroup merge their partials in LDS (one partial per 64
//   positions for the output projection to combine).
template <int HD, bool QKV>
struct vx_att_cfg {
    static constexpr int NCW = 1;
    static constexpr int NPG = QKV ? 1 : 2;
    static constexpr bool MERGE = QKV;
    static constexpr int WCH = NCW * NPG * 16;
};
// positions per wavefront and whether a workgroup merges its partials
static void vx_att_geom(int head_dim, bool qkv, int *wch, bool *merge)
{
    if (head_dim == 128) {
        *wch = qkv ? vx_att_cfg<128, true>::WCH : vx_att_cfg<128, false>::WCH;
        *merge = qkv ? vx_att_cfg<128, true>::MERGE : vx_att_cfg<128, false>::MERGE;
    } else {
        *wch = qkv ? vx_att_cfg<64, true>::WCH : vx_att_cfg<64, false>::WCH;
        *merge = qkv ? vx_att_cfg<64, true>::MERGE : vx_att_cfg<64, false>::MERGE;
    }
}

template <int HD, bool NT = false>
__global__ __launch_bounds__(ATT_THREADS) __attribute__((amdgpu_waves_per_eu(3))) void vx_attention_mfma_kernel(
    const float *__restrict__ q, int M, int n_past, int n_ctx, int n_heads, int n_kv, int cap,
    float *__restrict__ kc, float *__restrict__ vc, int n_chunks, int n_chunks_w, int n_qg,
    float *__restrict__ part, vx_qkv_args qa)
{
    using C = vx_att_cfg<HD, false>;
    vx_attention_mfma_body<false, HD, false, C::NCW, C::NPG, C::MERGE, NT>(
        q, M, n_past, n_ctx, n_heads, n_kv, cap, kc, vc, n_chunks, n_chunks_w, n_qg, part, qa);
}

template <int HD, bool KH = false, bool NT = false>
__global__ __launch_bounds__(ATT_THREADS) __attribute__((amdgpu_waves_per_eu(3))) void vx_attention_mfma_qkv_kernel(
    const float *__restrict__ q, int M, int n_past, int n_ctx, int n_heads, int n_kv, int cap,
    float *__restrict__ kc, float *__restrict__ vc, int n_chunks, int n_chunks_w, int n_qg,
    float *__restrict__ part, vx_qkv_args qa)
{
    using C = vx_att_cfg<HD, true>;
    vx_attention_mfma_body<true, HD, KH, C::NCW, C::NPG, C::MERGE, NT>(
        q, M, n_past, n_ctx, n_heads, n_kv, cap, kc, vc, n_chunks, n_chunks_w, n_qg, part, qa);
}

// One workgroup per (row m, head): merge the chunks' partial results with
// the online-softmax rescale and normalise by 1/(sum + 1e-10)
// (src/tensor.c:156-171).  Thread t owns float4 lane d4 = t % (hd/4) of the
// head and every S-th chunk starting at t / (hd/4) (S = 256/(hd/4) slices);
// its running (max, sum, acc) is merged across the slices in LDS, so the
// chunk walk is spread over the workgroup instead of serialised per thread.
#define CMB_THREADS 256
// NB: chunks whose loads a thread issues together (one round trip per
// batch); the launch picks the smallest of 4, 6, 8, 12 that covers a
// thread's chunks, so no loads or exponentials go to clamped duplicates
// (the visiting order, and so the result, does not depend on NB)
template <int NB>
__global__ __launch_bounds__(CMB_THREADS) void vx_attention_combine_kernel(
    const float *__restrict__ part, int M, int n_heads, int n_kv, int hd, int n_chunks,
    float *__restrict__ out, int ld_out, double *clr, long n_clr)
{
    __shared__ float4 s_acc[CMB_THREADS];
    if (clr) {
        // the q|k|v sums the first launch consumed
        const long per = (n_clr + gridDim.x - 1) / gridDim.x;
        const long b = (long)blockIdx.x * per, e = min(b + per, n_clr);
        for (long i = b + threadIdx.x; i < e; i += CMB_THREADS) clr[i] = 0.0;
    }
    __shared__ float s_m[CMB_THREADS], s_l[CMB_THREADS];
    const int m = blockIdx.x % M, head = blockIdx.x / M;
    const int G = n_heads / n_kv, QM = G * M;
    const int g = head / G, hl = head % G;
    const int qi = hl * M + m;
    const int L4 = hd / 4, S = CMB_THREADS / L4;
    const int d4 = threadIdx.x % L4, sl = threadIdx.x / L4;
    const size_t cstride = (size_t)QM * PART_STRIDE(hd);
    const float *pq = part + (size_t)g * n_chunks * cstride + (size_t)qi * PART_STRIDE(hd);

    float mx = -INFINITY, l = 0.0f;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    if (sl < S) {
        for (int c0 = sl; c0 < n_chunks; c0 += NB * S) {
            float cm[NB], cl[NB];
            float4 ca[NB];
#pragma unroll
            for (int u = 0; u < NB; u++) {
                const int c = c0 + u * S;
                const float *pc = pq + (size_t)min(c, n_chunks - 1) * cstride;
                cm[u] = c < n_chunks ? pc[0] : -INFINITY;
                cl[u] = pc[1];
                ca[u] = *(const float4 *)(pc + 4 + 4 * d4);
            }
#pragma unroll
            for (int u = 0; u < NB; u++) {
                if (cm[u] == -INFINITY) continue;
                const float nm = fmaxf(mx, cm[u]);
                const float fo = mx == -INFINITY ? 0.0f : expf(mx - nm);
                const float fn = expf(cm[u] - nm);
                l = l * fo + cl[u] * fn;
                a.x = a.x * fo + ca[u].x * fn;
                a.y = a.y * fo + ca[u].y * fn;
                a.z = a.z * fo + ca[u].z * fn;
                a.w = a.w * fo + ca[u].w * fn;
                mx = nm;
            }
        }
    }
    s_m[threadIdx.x] = mx;
    s_l[threadIdx.x] = l;
    s_acc[threadIdx.x] = a;
    __syncthreads();
    if (sl == 0) {
        float gm = -INFINITY;
        for (int j = 0; j < S; j++) gm = fmaxf(gm, s_m[j * L4 + d4]);
        float lt = 0.0f;
        float4 at = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int j = 0; j < S; j++) {
            const float cm = s_m[j * L4 + d4];
            if (cm == -INFINITY) continue;
            const float f = expf(cm - gm);
            const float4 v = s_acc[j * L4 + d4];
            lt = fmaf(f, s_l[j * L4 + d4], lt);
            at.x = fmaf(f, v.x, at.x);
            at.y = fmaf(f, v.y, at.y);
            at.z = fmaf(f, v.z, at.z);
            at.w = fmaf(f, v.w, at.w);
        }
        const float inv = 1.0f / (lt + 1e-10f);
        float *o = out + (size_t)m * ld_out + (size_t)head * hd + 4 * d4;
        *(float4 *)o = make_float4(at.x * inv, at.y * inv, at.z * inv, at.w * inv);
    }
}

// LDS of a workgroup holding nq queries; the query split keeps it <= 64 KiB.
static size_t vx_attn_lds(int nq, int hd)
{
    return sizeof(float) * ((size_t)nq * hd + (size_t)ACH * (hd + 4) + (size_t)ACH * hd + (size_t)nq * ACH);
}

static int vx_attn_qpg(int hd)
{
    long room = 65536 / 4 - (long)ACH * (2 * hd + 4);
    return room > 0 ? (int)(room / (hd + ACH)) : 0;
}

extern "C" size_t vxh_attention_workspace_floats(int M, int n_ctx, int cap, int n_heads,
                                                 int n_kv_heads, int head_dim)
{
    int ctx = n_ctx;
    if (cap > 0 && ctx > cap) ctx = cap;
    int n_chunks = (ctx + ACH - 1) / ACH;
    return (size_t)n_kv_heads * n_chunks * (n_heads / n_kv_heads) * M * PART_STRIDE(head_dim);
}

// a layer's attended cache rows beyond this many bytes are read with
// non-temporal loads
#define VX_KV_STREAM_BYTES (16.0 * 1024 * 1024)

// The fp32-MFMA kernels for a head size, cache precision and q source (q
// rows, or the q|k|v sums of A when qkv is set).
template <bool NT>
static void vx_attention_mfma_launch(const float *q, bool qkv, const vx_qkv_args &A, int M, int n_past, int n_ctx,
                                     int n_heads, int n_kv_heads, int head_dim, int cap, float *kc, float *vc,
                                     int n_chunks, int n_chunks_w, int nqg, int grid, float *part, int kv_half,
                                     vxh_stream s)
{
    if (kv_half && head_dim == 64)
        vx_attention_mfma_qkv_kernel<64, true, NT><<<grid, ATT_THREADS, 0, vxh_hs(s)>>>(
            nullptr, M, n_past, n_ctx, n_heads, n_kv_heads, cap, kc, vc, n_chunks, n_chunks_w, nqg, part, A);
    else if (kv_half)
        vx_attention_mfma_qkv_kernel<128, true, NT><<<grid, ATT_THREADS, 0, vxh_hs(s)>>>(
            nullptr, M, n_past, n_ctx, n_heads, n_kv_heads, cap, kc, vc, n_chunks, n_chunks_w, nqg, part, A);
    else if (head_dim == 64 && qkv)
        vx_attention_mfma_qkv_kernel<64, false, NT><<<grid, ATT_THREADS, 0, vxh_hs(s)>>>(
            nullptr, M, n_past, n_ctx, n_heads, n_kv_heads, cap, kc, vc, n_chunks, n_chunks_w, nqg, part, A);
    else if (head_dim == 64)
        vx_attention_mfma_kernel<64, NT><<<grid, ATT_THREADS, 0, vxh_hs(s)>>>(
            q, M, n_past, n_ctx, n_heads, n_kv_heads, cap, kc, vc, n_chunks, n_chunks_w, nqg, part, A);
    else if (qkv)
        vx_attention_mfma_qkv_kernel<128, false, NT><<<grid, ATT_THREADS, 0, vxh_hs(s)>>>(
            nullptr, M, n_past, n_ctx, n_heads, n_kv_heads, cap, kc, vc, n_chunks, n_chunks_w, nqg, part, A);
    else
        vx_attention_mfma_kernel<128, NT><<<grid, ATT_THREADS, 0, vxh_hs(s)>>>(
            q, M, n_past, n_ctx, n_heads, n_kv_heads, cap, kc, vc, n_chunks, n_chunks_w, nqg, part, A);
}

// parts_only: the first launch alone; the partials stay in ws->part for a
// consumer that combines them itself (*n_chunks_out chunks per query).
static int vx_attention_run(const float *q, const vx_qkv_args *qa, long n_clr, int M, int n_past,
                            int n_ctx, int n_heads, int n_kv_heads, int head_dim, int cap, float *kc,
                            float *vc, float *out, int ld_out, vxh_workspace *ws,
                            int parts_only, int *n_chunks_out,
                            vxh_stream s, int kv_half = 0)
{
    if (kv_half && (!qa || (head_dim != 64 && head_dim != 128) || M > VX_ATT_MFMA_MAX_M))
        return vxh_fail(VXH_ERR_UNSUPPORTED, "attention: an fp16 KV cache needs the q|k|v kernel, head_dim "
                        "64 or 128 and at most %d rows (head_dim %d, %d rows)", VX_ATT_MFMA_MAX_M, head_dim, M);
    if (M < 1 || n_kv_heads < 1 || n_heads % n_kv_heads)
        return vxh_fail(VXH_ERR_PARAM, "attention: M %d heads %d kv %d", M, n_heads, n_kv_heads);
    if (head_dim % 4 || head_dim > ATT_MAX_HD)
        return vxh_fail(VXH_ERR_UNSUPPORTED, "attention: head_dim %d (multiple of 4, <= %d)",
                        head_dim, ATT_MAX_HD);
    // the kernels address a layer's cache rows with 32-bit byte offsets
    if ((uint64_t)n_ctx * n_kv_heads * head_dim * (kv_half ? 2u : 4u) > 0xFFFFFFFFull)
        return vxh_fail(VXH_ERR_UNSUPPORTED, "attention: a layer's cache (%d rows of %d) exceeds 4 GiB", n_ctx,
                        n_kv_heads * head_dim);
    int last = n_past + M - 1 < n_ctx ? n_past + M - 1 : n_ctx - 1;
    int ctx = last + 1;
    if (cap > 0 && ctx > cap) ctx = cap;
    int n_chunks = (ctx + ACH - 1) / ACH;
    int n_chunks_w = n_chunks;      // QKV: chunks holding new rows, cap or not
    if (qa && (last + 1 + ACH - 1) / ACH > n_chunks_w) n_chunks_w = (last + 1 + ACH - 1) / ACH;
    int G = n_heads / n_kv_heads;
    int QM = G * M;
    int qpg = vx_attn_qpg(head_dim);
    if (qpg > QM) qpg = QM;
    int n_qg = (QM + qpg - 1) / qpg;
    size_t need = (size_t)n_kv_heads * n_chunks * QM * PART_STRIDE(head_dim);
    if (need > ws->part_floats)
        return vxh_fail(VXH_ERR_PARAM, "attention workspace too small (%zu floats needed)", need);
    size_t lds = vx_attn_lds(qpg, head_dim);
    vx_qkv_args none;
    memset(&none, 0, sizeof(none));
    const bool mfma = (head_dim == 64 || head_dim == 128) && (!qa || M <= VX_ATT_MFMA_MAX_M);
    if (mfma) {
        // fp32-MFMA kernel: 4 wavefronts per workgroup, wch positions each
        int wch;
        bool merge;
        vx_att_geom(head_dim, qa != nullptr, &wch, &merge);
        const int nw_w = (n_chunks_w * ACH + wch - 1) / wch;
        const int nqg = (QM + 15) / 16, ncg = (nw_w + 3) / 4;
        const int grid = n_kv_heads * nqg * ncg;
        const vx_qkv_args &A = qa ? *qa : none;
        // a layer's attended cache beyond VX_KV_STREAM_BYTES streams with
        // non-temporal loads (a 7B target's 2048-position rows: 64 MB; a 1B
        // draft's: 4 MB)
        const bool nt = 2.0 * ctx * n_kv_heads * head_dim * (kv_half ? 2 : 4) > VX_KV_STREAM_BYTES;
        if (nt)
            vx_attention_mfma_launch<true>(q, qa != nullptr, A, M, n_past, n_ctx, n_heads, n_kv_heads, head_dim, cap, kc, vc,
                                           n_chunks, n_chunks_w, nqg, grid, ws->part, kv_half, s);
        else
            vx_attention_mfma_launch<false>(q, qa != nullptr, A, M, n_past, n_ctx, n_heads, n_kv_heads, head_dim, cap, kc, vc,
                                            n_chunks, n_chunks_w, nqg, grid, ws->part, kv_half, s);
    } else if (qa)
        vx_attention_kernel<true><<<n_kv_heads * n_chunks_w * n_qg, ATT_THREADS, lds, vxh_hs(s)>>>(
            nullptr, M, n_past, n_ctx, n_heads, n_kv_heads, head_dim, cap, kc, vc, n_chunks, n_chunks_w,
            qpg, n_qg, ws->part, *qa);
    else
        vx_attention_kernel<false><<<n_kv_heads * n_chunks * n_qg, ATT_THREADS, lds, vxh_hs(s)>>>(
            q, M, n_past, n_ctx, n_heads, n_kv_heads, head_dim, cap, kc, vc, n_chunks, n_chunks, qpg,
            n_qg, ws->part, none);
    VXH_LAUNCHED();
    // partials per query: one per wavefront chunk of the MFMA kernels
    if (mfma) {
        int wch;
        bool merge;
        vx_att_geom(head_dim, qa != nullptr, &wch, &merge);
        const int nw = (n_chunks * ACH + wch - 1) / wch;
        n_chunks = merge ? (nw + 3) / 4 : nw;
    }
    if (n_chunks_out) *n_chunks_out = n_chunks;
    if (parts_only) return VXH_OK;
    double *clr = (qa && n_clr > 0) ? (double *)qa->qkv : nullptr;
    const int per = (n_chunks + CMB_THREADS / (head_dim / 4) - 1) / (CMB_THREADS / (head_dim / 4));
#define VX_CMB_LAUNCH(NB_)                                                                                      \
    vx_attention_combine_kernel<NB_><<<M * n_heads, CMB_THREADS, 0, vxh_hs(s)>>>(                               \
        ws->part, M, n_heads, n_kv_heads, head_dim, n_chunks, out, ld_out, clr, n_clr)
    if (per <= 4) VX_CMB_LAUNCH(4);
    else if (per <= 6) VX_CMB_LAUNCH(6);
    else if (per <= 8) VX_CMB_LAUNCH(8);
    else VX_CMB_LAUNCH(12);
#undef VX_CMB_LAUNCH
    VXH_LAUNCHED();
    return VXH_OK;
}

extern "C" int vxh_attention(const float *q, int M, int n_past, int n_ctx, int n_heads,
                             int n_kv_heads, int head_dim, int cap, const float *kc,
                             const float *vc, float *out, int ld_out, vxh_workspace *ws,
                             vxh_stream s)
{
    return vx_attention_run(q, nullptr, 0, M, n_past, n_ctx, n_heads, n_kv_heads, head_dim, cap,
                            (float *)kc, (float *)vc, out, ld_out, ws, 0, nullptr, s);
}

static int vx_attention_qkv(double *qkv, int ld_qkv, const double *ss, int ss_K, const float *bq,
                            const float *bk, const float *bv, const float *cos_tab, const float *sin_tab,
                            int n_pos, int M, int n_past, int n_ctx, int n_heads, int n_kv_heads,
                            int head_dim, int cap, float *kc, float *vc, float *out, int ld_out,
                            vxh_workspace *ws, int *n_chunks_out, vxh_stream s, int kv_half = 0,
                            bool keep = false)
{
    if (!qkv || ((uintptr_t)qkv & 15) || ld_qkv % 2 || M < 1 || n_kv_heads < 1 ||
        ld_qkv < (n_heads + 2 * n_kv_heads) * head_dim)
        return vxh_fail(VXH_ERR_PARAM, "attention_qkv: ld %d for %d+2x%d heads of %d", ld_qkv, n_heads,
                        n_kv_heads, head_dim);
    if (n_past < 0 || n_past + M - 1 >= n_pos || (n_past + M - 1 >= n_ctx && M > 1))
        return vxh_fail(VXH_ERR_PARAM, "attention_qkv: M %d n_past %d n_ctx %d n_pos %d", M, n_past,
                        n_ctx, n_pos);
    if (ss && ss_K < 1) return vxh_fail(VXH_ERR_PARAM, "attention_qkv: norm length %d", ss_K);
    vx_qkv_args qa;
    qa.qkv = qkv;
    qa.ld = ld_qkv;
    qa.ss = ss;
    qa.ss_K = ss_K;
    qa.bq = bq;
    qa.bk = bk;
    qa.bv = bv;
    qa.cs = cos_tab;
    qa.sn = sin_tab;
    return vx_attention_run(nullptr, &qa, keep ? 0L : (long)M * ld_qkv, M, n_past, n_ctx, n_heads, n_kv_heads,
                            head_dim, cap, kc, vc, out, ld_out, ws, n_chunks_out != nullptr,
                            n_chunks_out, s, kv_half);
}

extern "C" int vxh_attention_qkv(double *qkv, int ld_qkv, const double *ss, int ss_K, const float *bq,
                                 const float *bk, const float *bv, const float *cos_tab,
                                 const float *sin_tab, int n_pos, int M, int n_past, int n_ctx,
                                 int n_heads, int n_kv_heads, int head_dim, int cap, float *kc,
                                 float *vc, float *out, int ld_out, vxh_workspace *ws, vxh_stream s)
{
    return vx_attention_qkv(qkv, ld_qkv, ss, ss_K, bq, bk, bv, cos_tab, sin_tab, n_pos, M, n_past, n_ctx,
                            n_heads, n_kv_heads, head_dim, cap, kc, vc, out, ld_out, ws, nullptr, s);
}

extern "C" int vxh_attention_qkv_keep(double *qkv, int ld_qkv, const double *ss, int ss_K, const float *bq,
                                      const float *bk, const float *bv, const float *cos_tab,
                                      const float *sin_tab, int n_pos, int M, int n_past, int n_ctx,
                                      int n_heads, int n_kv_heads, int head_dim, int cap, float *kc,
                                      float *vc, float *out, int ld_out, vxh_workspace *ws, vxh_stream s)
{
    return vx_attention_qkv(qkv, ld_qkv, ss, ss_K, bq, bk, bv, cos_tab, sin_tab, n_pos, M, n_past, n_ctx,
                            n_heads, n_kv_heads, head_dim, cap, kc, vc, out, ld_out, ws, nullptr, s, 0, true);
}

extern "C" int vxh_attention_parts_qkv(double *qkv, int ld_qkv, const double *ss, int ss_K,
                                       const float *bq, const float *bk, const float *bv,
                                       const float *cos_tab, const float *sin_tab, int n_pos, int M,
                                       int n_past, int n_ctx, int n_heads, int n_kv_heads, int head_dim,
                                       int cap, float *kc, float *vc, vxh_workspace *ws, int *n_chunks,
                                       vxh_stream s)
{
    if (!n_chunks) return vxh_fail(VXH_ERR_PARAM, "attention_parts_qkv: n_chunks output missing");
    return vx_attention_qkv(qkv, ld_qkv, ss, ss_K, bq, bk, bv, cos_tab, sin_tab, n_pos, M, n_past, n_ctx,
                            n_heads, n_kv_heads, head_dim, cap, kc, vc, nullptr, 0, ws, n_chunks, s);
}

extern "C" int vxh_attention_qkv_f16(double *qkv, int ld_qkv, const double *ss, int ss_K, const float *bq,
                                     const float *bk, const float *bv, const float *cos_tab,
                                     const float *sin_tab, int n_pos, int M, int n_past, int n_ctx,
                                     int n_heads, int n_kv_heads, int head_dim, int cap, uint16_t *kc,
                                     uint16_t *vc, float *out, int ld_out, vxh_workspace *ws, vxh_stream s)
{
    if (((uintptr_t)kc | (uintptr_t)vc) & 7) return vxh_fail(VXH_ERR_PARAM, "attention_qkv_f16: cache alignment");
    return vx_attention_qkv(qkv, ld_qkv, ss, ss_K, bq, bk, bv, cos_tab, sin_tab, n_pos, M, n_past, n_ctx,
                            n_heads, n_kv_heads, head_dim, cap, (float *)kc, (float *)vc, out, ld_out, ws,
                            nullptr, s, 1);
}

extern "C" int vxh_attention_parts_qkv_f16(double *qkv, int ld_qkv, const double *ss, int ss_K,
                                           const float *bq, const float *bk, const float *bv,
                                           const float *cos_tab, const float *sin_tab, int n_pos, int M,
                                           int n_past, int n_ctx, int n_heads, int n_kv_heads, int head_dim,
                                           int cap, uint16_t *kc, uint16_t *vc, vxh_workspace *ws,
                                           int *n_chunks, vxh_stream s)
{
    if (!n_chunks) return vxh_fail(VXH_ERR_PARAM, "attention_parts_qkv_f16: n_chunks output missing");
    if (((uintptr_t)kc | (uintptr_t)vc) & 7) return vxh_fail(VXH_ERR_PARAM, "attention_parts_qkv_f16: cache alignment");
    return vx_attention_qkv(qkv, ld_qkv, ss, ss_K, bq, bk, bv, cos_tab, sin_tab, n_pos, M, n_past, n_ctx,
                            n_heads, n_kv_heads, head_dim, cap, (float *)kc, (float *)vc, nullptr, 0, ws,
                            n_chunks, s, 1);
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
