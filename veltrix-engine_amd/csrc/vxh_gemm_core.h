// Shared device code of the skinny-M dequant GEMM: operand unpacking, the
// MFMA kernel templates and their launchers, and the row helpers the panel
// producers use.  Included by vxh_gemm.hip (plain GEMM) and vxh_pro*.hip
// (GEMM that builds its own panel slice).
#pragma once

#include <string.h>

#include <hip/hip_ext.h>

#include "vxh_internal.h"

__device__ __forceinline__ float vx_silu(float g) { return g / (1.0f + expf(-g)); }

// Panel unit of group g (elements 8g..8g+7): block b = g/4, lane half h =
// (g/2)%2, MFMA half s = g%2; hi at slot m, lo at slot M+m.
__device__ __forceinline__ void vx_panel_store(uint4 *__restrict__ panel, int M, int g, int m,
                                               const float v[8])
{
    vx_half8 hi, lo;
#pragma unroll
    for (int kk = 0; kk < 8; kk++) {
        _Float16 a = (_Float16)v[kk];
        hi[kk] = a;
        lo[kk] = (_Float16)(v[kk] - (float)a);
    }
    const int b = g >> 2, h = (g >> 1) & 1, s = g & 1;
    const size_t base = ((size_t)(b * 2 + s) * 2 + h) * (2 * M);
    panel[base + m] = __builtin_bit_cast(uint4, hi);
    panel[base + M + m] = __builtin_bit_cast(uint4, lo);
}


// ---------------------------------------------------------------------------
// MFMA GEMM
// ---------------------------------------------------------------------------
// (q & mask) | magic in one v_and_or_b32.  The compiler splits it into a
// v_and / v_or pair (gfx9 VOP3 encodings take no literal), so it is written
// out; the mask travels in an SGPR and the magic word in a VGPR.
__device__ __forceinline__ uint32_t vx_and_or(uint32_t q, uint32_t mask, uint32_t magic)
{
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(q), "s"(mask), "v"(magic));
    return r;
}

// Q4_0 dword (8 nibbles in the repacked slot order) -> 8 fp16 values s - 8:
// 1024 + s (low nibble) and 1024 + 16 s (high nibble) by exponent magic,
// then one packed add / fma per pair.
__device__ __forceinline__ vx_half8 vx_unpack_q4(uint32_t q, uint32_t magic)
{
    const uint32_t q8 = q >> 8;
    vx_half2 a = __builtin_bit_cast(vx_half2, vx_and_or(q, 0x000F000Fu, magic));
    vx_half2 b = __builtin_bit_cast(vx_half2, vx_and_or(q, 0x00F000F0u, magic));
    vx_half2 c = __builtin_bit_cast(vx_half2, vx_and_or(q8, 0x000F000Fu, magic));
    vx_half2 d = __builtin_bit_cast(vx_half2, vx_and_or(q8, 0x00F000F0u, magic));
    const vx_half2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const vx_half2 sc = {(_Float16)0.0625f, (_Float16)0.0625f};
    const vx_half2 off16 = {(_Float16)-72.0f, (_Float16)-72.0f};
    a = a + off;
    b = b * sc + off16;
    c = c + off;
    d = d * sc + off16;
    vx_half8 r = {a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
    return r;
}

// Two Q8_0 dwords (4 int8 each, bytes in the repacked order) -> 8 fp16:
// (q ^ 0x80) = q + 128 as an unsigned byte, 1024 + that by exponent magic.
__device__ __forceinline__ vx_half8 vx_unpack_q8(uint32_t qa, uint32_t qb, uint32_t magic)
{
    const uint32_t m = 0x00FF00FFu;
    const uint32_t ua = qa ^ 0x80808080u, ub = qb ^ 0x80808080u;
    vx_half2 a0 = __builtin_bit_cast(vx_half2, vx_and_or(ua, m, magic));
    vx_half2 a1 = __builtin_bit_cast(vx_half2, vx_and_or(ua >> 8, m, magic));
    vx_half2 b0 = __builtin_bit_cast(vx_half2, vx_and_or(ub, m, magic));
    vx_half2 b1 = __builtin_bit_cast(vx_half2, vx_and_or(ub >> 8, m, magic));
    const vx_half2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    a0 = a0 + off;
    a1 = a1 + off;
    b0 = b0 + off;
    b1 = b1 + off;
    vx_half8 r = {a0.x, a0.y, a1.x, a1.y, b0.x, b0.y, b1.x, b1.y};
    return r;
}

template <int M>
struct vx_mcfg {
    static constexpr int NS = 2 * M;
    // hi accumulator registers in use: register r < R1 holds column
    // c = 8(r/4) + 4h + r%4 (h = lane/32); lo is register r + 8.
    static constexpr int R1 = M <= 4 ? M : (M <= 8 ? 4 : (4 + (M - 8 < 4 ? M - 8 : 4)));
};

// Block pairs per K slice.  Each M has up to three slice lengths (in
// ascending order); the launcher takes the shortest one whose launch stays
// within `target` workgroups, or the longest.  Short slices suit the small
// draft matrices at M = 1 (in the decode pipeline 2 pairs beat 1 and 4 by
// 5-10% of the draft time), long ones the large verify matrices; M > 12
// stays short for LDS.
template <int QT, int M>
struct vx_ppw_set {
    static constexpr int n = QT == 8 ? (M <= 4 ? 2 : 1) : (M <= 4 ? 3 : 2);
    static constexpr int v0 = QT == 8 ? (M <= 4 ? 2 : 8) : (M <= 4 ? 2 : (M <= 12 ? 8 : 4));
    static constexpr int v1 = QT == 8 ? 8 : (M <= 4 ? 4 : (M <= 12 ? 16 : 8));
    static constexpr int v2 = QT == 8 ? 8 : (M <= 4 ? 8 : (M <= 12 ? 16 : 8));
    static constexpr int target = 1600;
};

#define VX_CHUNK 1024   // panel columns per power-of-two scale chunk (SwiGLU panel)

// Prologue kinds (vxh_pro*.hip): instead of reading a panel that a row kernel
// wrote, the workgroup builds its own K slice of the panel from the rows the
// panel is made of.  Every workgroup sharing a K slice builds the same slice;
// the first tile group also stores the updated residual and adds the row's
// sum of squares, so the consumer of the product can apply the RMSNorm.
enum { VX_PRO_PANEL = 0, VX_PRO_ROWS = 1, VX_PRO_RESID = 2, VX_PRO_SWIGLU = 3, VX_PRO_ATTN = 4 };
#define VX_PRO_ATTN_MAX_M VXH_PRO_ATTN_MAX_ROWS   // ATTN: M * PPW * 16 float4 columns <= 256 threads

struct vx_pro_args {
    const float *x;         // ROWS, RESID: input rows
    int ldx;
    const double *src;      // RESID: pending sums added to x; SWIGLU: gate/up accumulator
    int ld_src;
    const float *w;         // ROWS, RESID: RMSNorm weight folded into the panel (NULL: none)
    float *x_out;           // RESID: x + src, stored by the first tile group (NULL: not stored)
    int ld_xout;
    double *ss;             // ROWS, RESID: sum of squares of the rows, added by the first tile group
    const double *ss_in;    // SWIGLU: gate/up sums are scaled by 1/rms(ss_in[m] / ss_K)
    int ss_K;
    float thr;              // SWIGLU gate threshold
    int K;                  // row length
    double *clr;            // n_clr doubles zeroed by the launch (an accumulator already consumed)
    long n_clr;
    const float *part;      // ATTN: per-chunk attention partials (max, sum, pad 2, acc[hd])
    int n_chunks, G, hd;    // ATTN: chunks per query, query heads per kv head, head_dim
};

struct vx_gemm_args {
    const uint4 *wq;
    const uint32_t *wd;
    const uint4 *panel;
    const float *corr;
    // output scale of row m for a K slice starting at pair p0:
    // rscale[m * rs_ld + p0 / rs_chunk] * (ss ? 1/rms(ss[m] / ss_K) : 1) * scale
    const float *rscale;
    int rs_ld, rs_chunk;
    const double *ss;
    int ss_K;
    int n_tiles, n_pairs, n_splits;
    int wcache;             // weights with plain loads (else non-temporal)
    double *acc;
    int ld_acc;
    int n_out;
    float scale;
    const float *gate;
    int ld_gate;
    float thr;
    vx_pro_args p;
    // verify-batch kernel (vx_vg_kernel): the 64-row tiled copy of the matrix
    const void *tq, *td;
    uint32_t tq_bytes, td_bytes, pan_bytes;
    int n_t64, n_blk;
};

// ---------------------------------------------------------------------------
// prologue kinds: building the panel slice in the GEMM
// ---------------------------------------------------------------------------
// Source values of one 8-column group of a prologue row.
struct vx_pro_raw {
    float4 x0, x1, w0, w1;
    double2 a[4], b[4];
};

template <int PRO>
__device__ __forceinline__ void vx_pro_load(const vx_pro_args &p, int m, int e0, vx_pro_raw &r)
{
    if constexpr (PRO == VX_PRO_SWIGLU) {
        // h column i -> tile i/16: gate at physical column 32(i/16) + i%16, up 16 further
        const double *ar = p.src + (size_t)m * p.ld_src + 32 * (e0 / 16) + e0 % 16;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            r.a[q] = *(const double2 *)(ar + 2 * q);
            r.b[q] = *(const double2 *)(ar + 16 + 2 * q);
        }
    } else {
        const float *xr = p.x + (size_t)m * p.ldx + e0;
        r.x0 = *(const float4 *)xr;
        r.x1 = *(const float4 *)(xr + 4);
        if (PRO == VX_PRO_RESID) {
            const double *ar = p.src + (size_t)m * p.ld_src + e0;
#pragma unroll
            for (int q = 0; q < 4; q++) r.a[q] = *(const double2 *)(ar + 2 * q);
        }
        if (p.w) {
            r.w0 = *(const float4 *)(p.w + e0);
            r.w1 = *(const float4 *)(p.w + e0 + 4);
        }
    }
}

// Panel values of a loaded group.  ROWS, RESID: v = w .* t with t = x (+ src),
// t^2 added to ss, t stored to xo when not NULL.  SWIGLU: v = silu(g) * u,
// zero where |silu(g)| < thr (src/model.c:582-585), g and u the fp32
// roundings of the sums times rin.
template <int PRO>
__device__ __forceinline__ void vx_pro_values(const vx_pro_args &p, const vx_pro_raw &r, float rin,
                                              float *xo, float v[8], float &ss)
{
    if constexpr (PRO == VX_PRO_SWIGLU) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float g0 = vx_silu((float)r.a[q].x * rin), g1 = vx_silu((float)r.a[q].y * rin);
            const float u0 = (float)r.b[q].x * rin, u1 = (float)r.b[q].y * rin;
            v[2 * q] = fabsf(g0) < p.thr ? 0.0f : g0 * u0;
            v[2 * q + 1] = fabsf(g1) < p.thr ? 0.0f : g1 * u1;
        }
    } else {
        float t[8] = {r.x0.x, r.x0.y, r.x0.z, r.x0.w, r.x1.x, r.x1.y, r.x1.z, r.x1.w};
        if (PRO == VX_PRO_RESID) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                t[2 * q] = t[2 * q] + (float)r.a[q].x;
                t[2 * q + 1] = t[2 * q + 1] + (float)r.a[q].y;
            }
            if (xo) {
                *(float4 *)xo = make_float4(t[0], t[1], t[2], t[3]);
                *(float4 *)(xo + 4) = make_float4(t[4], t[5], t[6], t[7]);
            }
        }
#pragma unroll
        for (int kk = 0; kk < 8; kk++) ss += t[kk] * t[kk];
        if (p.w) {
            const float wv[8] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w, r.w1.x, r.w1.y, r.w1.z, r.w1.w};
#pragma unroll
            for (int kk = 0; kk < 8; kk++) v[kk] = wv[kk] * t[kk];
        } else {
#pragma unroll
            for (int kk = 0; kk < 8; kk++) v[kk] = t[kk];
        }
    }
}


// ATTN: the K slice of the attention rows, combined from the per-chunk
// partials of the attention's first launch (online-softmax rescale and
// 1/(sum + 1e-10), src/tensor.c:156-171), then converted to the panel.
// Thread t owns float4 column u = t % U of the slice (U = M * L/4: row m,
// head, lane d4) and every S-th chunk from t / U (S = 256 / U slices); the
// slices merge in LDS.
// chunks of partials whose loads one thread issues together (one round trip
// per batch; with one partial per 64 positions a thread of a one-row slice
// (8 slices) visits every 8th: 6 cover a 3072-position draft context in one
// batch without loading clamped duplicates at the usual ~2000-2400, two rows
// (4 slices) take 12 per batch)
#define VX_CMB_BATCH(M) ((M) == 1 ? 6 : 12)

template <int M, int PPW>
__device__ __forceinline__ void vx_pro_attn(const vx_pro_args &p, int p0, int np, uint4 *lds, float *lrs)
{
    constexpr int NS = 2 * M;
    constexpr int LMAX = PPW * 64;
    __shared__ float s_m[256], s_l[256];
    __shared__ float4 s_a[256];
    __shared__ float s_row[M][LMAX];
    const int L4 = np * 16, k0 = p0 * 64;
    const int U = M * L4, S = 256 / U;
    const int t = threadIdx.x, u = t % U, sl = t / U;
    const int hd = p.hd, QM = p.G * M, PS = hd + 4;
    const size_t cstride = (size_t)QM * PS;
    const int m = u / L4, c4 = u % L4;
    float mx = -INFINITY, l = 0.0f;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    if (sl < S) {
        const int e = k0 + 4 * c4;
        const int head = e / hd, d4 = (e % hd) / 4;
        const int g = head / p.G, qi = (head % p.G) * M + m;
        const float *pq = p.part + (size_t)g * p.n_chunks * cstride + (size_t)qi * PS;
        constexpr int NB = VX_CMB_BATCH(M);
        for (int c0 = sl; c0 < p.n_chunks; c0 += NB * S) {
            float cm[NB], cl[NB];
            float4 ca[NB];
#pragma unroll
            for (int v = 0; v < NB; v++) {
                const int c = c0 + v * S;
                const float *pc = pq + (size_t)min(c, p.n_chunks - 1) * cstride;
                cm[v] = c < p.n_chunks ? pc[0] : -INFINITY;
                cl[v] = pc[1];
                ca[v] = *(const float4 *)(pc + 4 + 4 * d4);
            }
#pragma unroll
            for (int v = 0; v < NB; v++) {
                if (cm[v] == -INFINITY) continue;
                const float nm = fmaxf(mx, cm[v]);
                const float fo = mx == -INFINITY ? 0.0f : expf(mx - nm);
                const float fn = expf(cm[v] - nm);
                l = l * fo + cl[v] * fn;
                a.x = a.x * fo + ca[v].x * fn;
                a.y = a.y * fo + ca[v].y * fn;
                a.z = a.z * fo + ca[v].z * fn;
                a.w = a.w * fo + ca[v].w * fn;
                mx = nm;
            }
        }
    }
    s_m[t] = mx;
    s_l[t] = l;
    s_a[t] = a;
    __syncthreads();
    if (t < U) {
        float gm = -INFINITY;
        for (int j = 0; j < S; j++) gm = fmaxf(gm, s_m[j * U + t]);
        float lt = 0.0f;
        float4 at = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int j = 0; j < S; j++) {
            const float cm = s_m[j * U + t];
            if (cm == -INFINITY) continue;
            const float f = expf(cm - gm);
            const float4 v = s_a[j * U + t];
            lt = fmaf(f, s_l[j * U + t], lt);
            at.x = fmaf(f, v.x, at.x);
            at.y = fmaf(f, v.y, at.y);
            at.z = fmaf(f, v.z, at.z);
            at.w = fmaf(f, v.w, at.w);
        }
        const float inv = 1.0f / (lt + 1e-10f);
        *(float4 *)&s_row[m][4 * c4] = make_float4(at.x * inv, at.y * inv, at.z * inv, at.w * inv);
    }
    __syncthreads();
    // panel of the slice: wavefront w builds rows m = w + 4r, lane l the
    // 8-column groups l + 64j (as the other prologue kinds)
    const int lane = t & 63, wave = t >> 6, ng = np * 8;
    constexpr int GL = (PPW * 8 + 63) / 64;
#pragma unroll
    for (int rr = 0; rr < (M + 3) / 4; rr++) {
        const int mm = wave + 4 * rr;
        if (mm >= M) continue;
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < GL; j++) {
            const int g = lane + 64 * j;
            if (g < ng)
#pragma unroll
                for (int kk = 0; kk < 8; kk++) amax = fmaxf(amax, fabsf(s_row[mm][8 * g + kk]));
        }
        amax = vx_wave_max64(amax);
        float rs;
        const float sc = vx_row_scale(amax, &rs);
        if (lane == 0) lrs[mm] = rs;
#pragma unroll
        for (int j = 0; j < GL; j++) {
            const int g = lane + 64 * j;
            if (g >= ng) continue;
            vx_half8 hi, lo;
#pragma unroll
            for (int kk = 0; kk < 8; kk++) {
                const float xv = s_row[mm][8 * g + kk] * sc;
                const _Float16 h = (_Float16)xv;
                hi[kk] = h;
                lo[kk] = (_Float16)(xv - (float)h);
            }
            const int b = g >> 2, h2 = (g >> 1) & 1, s2 = g & 1;
            const int base = ((b * 2 + s2) * 2 + h2) * NS;
            lds[base + mm] = __builtin_bit_cast(uint4, hi);
            lds[base + M + mm] = __builtin_bit_cast(uint4, lo);
        }
    }
}

#define VX_RING 4

// A weight load: non-temporal unless the matrix is marked to stay cached.
__device__ __forceinline__ uint4 vx_load_w(const uint4 *p, int cached)
{
    if (cached) return *p;
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load((const u32x4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Wavefronts (tiles) per workgroup: 8 for the residual prologue of Q4_0
// verify batches at 8-pair slices (every workgroup rebuilds its K slice of
// the panel from x, the fp64 pending sums and the norm weight; 8 tiles per
// workgroup halve those rebuilds: 22016x4096 at M = 9 20.6 -> 18.6 us,
// 12288x4096 13.2 -> 12.8 us), 4 otherwise (Q8_0 11008x4096 15.2 -> 16.7 us
// and the 16-pair logits GEMM 26.7 -> 27.5 us with 8).
template <int QT, int M, bool AVX2, int PPW, int PRO>
struct vx_nwv {
    static constexpr int v =
        PRO == VX_PRO_RESID && QT == 2 && M >= 5 && PPW == 8 && !AVX2 ? 8 : 4;
};

// QT: 2 = Q4_0, 8 = Q8_0.
template <int QT, int M, bool AVX2, int PPW, int PRO = VX_PRO_PANEL>
__global__ __launch_bounds__((64 * vx_nwv<QT, M, AVX2, PPW, PRO>::v)) void vx_gemm_kernel(vx_gemm_args a)
{
    constexpr int NWV = vx_nwv<QT, M, AVX2, PPW, PRO>::v;   // wavefronts, one tile each
    constexpr int NT = 64 * NWV;                          // threads
    static_assert(NWV == 4 || (!AVX2 && PRO != VX_PRO_ATTN),
                  "AVX2 corrections and the attention prologue assume 4 wavefronts");
    // With 8 wavefronts per workgroup the compiler may give a wavefront at
    // most 256 registers and, seeing no AGPR use, selects the VGPR-destination
    // MFMA form, whose destinations it overlaps with their own A/B sources
    // (results have been wrong with that form here).  An AGPR clobber keeps
    // the AGPR-destination form.
    if constexpr (NWV > 4) asm volatile("" ::: "a0");
    static_assert(!AVX2 || PRO == VX_PRO_PANEL, "AVX2-lane corrections come with panels");
    constexpr bool PANEL = PRO == VX_PRO_PANEL;
    constexpr int NS = vx_mcfg<M>::NS;
    constexpr int R1 = vx_mcfg<M>::R1;
    constexpr int WPP = QT == 2 ? 1 : 2;   // 16-byte weight loads per lane per block pair
    // two accumulator sets per block pair for verify batches read from a
    // panel or plain rows; the residual/SwiGLU prologues keep one (their
    // preloaded rows already cost registers: a second set lowered occupancy
    // and slowed 22016x4096 at M = 9 from 21.1 to 23.8 us)
    constexpr bool DUAL = M >= 5 && (PRO == VX_PRO_PANEL || PRO == VX_PRO_ROWS);
    constexpr int UNITS = PPW * 8 * NS;    // panel units of a full slice
    constexpr int UPT = (UNITS + NT - 1) / NT;
    __shared__ uint4 lds[UPT * NT];
    __shared__ float lcorr[AVX2 ? PPW * 2 * M : 1];
    __shared__ float lrs[PANEL ? 1 : M];   // prologue kinds: output scale of each row's slice

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = blockIdx.x / a.n_splits, split = blockIdx.x % a.n_splits;
    const int T = grp * NWV + wave;
    const bool tile_ok = T < a.n_tiles;
    const int Tc = tile_ok ? T : 0;
    const int p0 = split * PPW;
    const int np = min(PPW, a.n_pairs - p0);
    const int units = np * 8 * NS;
    const int c = lane & 31, h = lane >> 5;
    const uint32_t magic = 0x64006400u;

    // 0. prologue kinds: this workgroup's share of the accumulator to clear
    if constexpr (!PANEL) {
        if (a.p.clr) {
            const long per = (a.p.n_clr + gridDim.x - 1) / gridDim.x;
            const long b = (long)blockIdx.x * per, e = min(b + per, a.p.n_clr);
            for (long i = b + threadIdx.x; i < e; i += NT) a.p.clr[i] = 0.0;
        }
    }

    // 1. the panel slice (issued first so its wait does not cover the weights)
    constexpr int PU = PANEL ? UPT : 1;
    uint4 pv[PU];
    if constexpr (PANEL) {
        const uint4 *psrc = a.panel + (size_t)p0 * 8 * NS;
#pragma unroll
        for (int j = 0; j < UPT; j++) pv[j] = psrc[min(j * NT + (int)threadIdx.x, units - 1)];
    }
    // prologue kinds: the slice's source rows; wavefront w builds rows
    // m = w + 4r, lane l the 8-column groups l + 64j.  Up to 4 groups per lane
    // are loaded here, ahead of the weights, so their round trips overlap
    // (verify at M = 9: 3 groups; 186 -> 192 tok/s); larger slices go row by
    // row after them (8 preloaded groups cost occupancy: logits GEMM 24 -> 30 us).
    constexpr int RW = PANEL ? 1 : (M + NWV - 1) / NWV;
    constexpr int GL = PANEL ? 1 : (PPW * 8 + 63) / 64;
    constexpr bool PRELOAD = !PANEL && PRO != VX_PRO_ATTN && RW * GL <= 4;
    const int ng = np * 8, k0 = p0 * 64;
    vx_pro_raw raw[PRELOAD ? RW : 1][PRELOAD ? GL : 1];
    if constexpr (PRELOAD) {
#pragma unroll
        for (int rr = 0; rr < RW; rr++) {
            const int m = wave + NWV * rr;
            if (m >= M) continue;
#pragma unroll
            for (int j = 0; j < GL; j++) {
                const int g = lane + 64 * j;
                if (g < ng && k0 + 8 * g < a.p.K) vx_pro_load<PRO>(a.p, m, k0 + 8 * g, raw[rr][j]);
            }
        }
    }
    // AVX2 corrections of the slice: at most PPW*2*M <= 512 floats, two per thread
    float cv0 = 0.0f, cv1 = 0.0f;
    if (AVX2) {
        const int cnt = np * 2 * M;
        const float *cs = a.corr + (size_t)p0 * 2 * M;
        cv0 = cs[min((int)threadIdx.x, cnt - 1)];
        cv1 = cs[min((int)threadIdx.x + 256, cnt - 1)];
    }
    // 2. the first RING pairs of this wavefront's weights and scales
    const uint4 *wp = a.wq + ((size_t)Tc * a.n_pairs + p0) * WPP * 64 + lane;
    const uint32_t *sp = a.wd + ((size_t)Tc * a.n_pairs + p0) * 32 + c;
    uint4 w[VX_RING][WPP];
    uint32_t sc[VX_RING];
#pragma unroll
    for (int i = 0; i < VX_RING; i++) {
        const int pi = min(i, np - 1);
#pragma unroll
        for (int q = 0; q < WPP; q++) w[i][q] = vx_load_w(wp + ((size_t)pi * WPP + q) * 64, a.wcache);
        sc[i] = sp[(size_t)pi * 32];
    }
    if constexpr (PANEL) {
#pragma unroll
        for (int j = 0; j < UPT; j++) lds[j * NT + threadIdx.x] = pv[j];
    } else if constexpr (PRO == VX_PRO_ATTN) {
        static_assert(M <= VX_PRO_ATTN_MAX_M && M * PPW * 16 <= 256, "ATTN slice columns exceed the workgroup");
        vx_pro_attn<M, PPW>(a.p, p0, np, lds, lrs);
    } else {
        const bool lead = grp == 0;
#pragma unroll
        for (int rr = 0; rr < RW; rr++) {
            const int m = wave + NWV * rr;
            if (m >= M) continue;
            const float rin = (PRO == VX_PRO_SWIGLU && a.p.ss_in) ? vx_rms_inv((float)a.p.ss_in[m], a.p.ss_K)
                                                                  : 1.0f;
            float v[GL][8];
            float ss = 0.0f, amax = 0.0f;
#pragma unroll
            for (int j = 0; j < GL; j++) {
                const int g = lane + 64 * j, e0 = k0 + 8 * g;
#pragma unroll
                for (int kk = 0; kk < 8; kk++) v[j][kk] = 0.0f;
                if (g < ng && e0 < a.p.K) {
                    vx_pro_raw r;
                    if constexpr (PRELOAD) r = raw[rr][j];
                    else vx_pro_load<PRO>(a.p, m, e0, r);
                    float *xo = (lead && a.p.x_out) ? a.p.x_out + (size_t)m * a.p.ld_xout + e0 : nullptr;
                    vx_pro_values<PRO>(a.p, r, rin, xo, v[j], ss);
                }
#pragma unroll
                for (int kk = 0; kk < 8; kk++) amax = fmaxf(amax, fabsf(v[j][kk]));
            }
            amax = vx_wave_max64(amax);
            float rs;
            const float sc = vx_row_scale(amax, &rs);
            if (lane == 0) lrs[m] = rs;
            if (PRO != VX_PRO_SWIGLU && lead && a.p.ss) {
                ss = vx_wave_sum64(ss);
                if (lane == 0)
                    __hip_atomic_fetch_add(&a.p.ss[m], (double)ss, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int j = 0; j < GL; j++) {
                const int g = lane + 64 * j;
                if (g >= ng) continue;
                vx_half8 hi, lo;
#pragma unroll
                for (int kk = 0; kk < 8; kk++) {
                    const float xv = v[j][kk] * sc;
                    const _Float16 t = (_Float16)xv;
                    hi[kk] = t;
                    lo[kk] = (_Float16)(xv - (float)t);
                }
                const int b = g >> 2, h2 = (g >> 1) & 1, s2 = g & 1;
                const int base = ((b * 2 + s2) * 2 + h2) * NS;
                lds[base + m] = __builtin_bit_cast(uint4, hi);
                lds[base + M + m] = __builtin_bit_cast(uint4, lo);
            }
        }
    }
    if (AVX2) {
        if ((int)threadIdx.x < PPW * 2 * M) lcorr[threadIdx.x] = cv0;
        if ((int)threadIdx.x + 256 < PPW * 2 * M) lcorr[threadIdx.x + 256] = cv1;
    }
    __syncthreads();

    // idle A lanes read a valid slot; their output rows are never used
    const int slot = c < 16 ? min(c, M - 1) : M + min(c - 16, M - 1);
    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    const vx_f32x16 zero16 = {};
#pragma unroll
    for (int i = 0; i < PPW; i++) {
        uint4 wv[WPP];
#pragma unroll
        for (int q = 0; q < WPP; q++) wv[q] = w[i % VX_RING][q];
        const uint32_t sv = sc[i % VX_RING];
        if (i + VX_RING < PPW) {
            const int pi = min(i + VX_RING, np - 1);
#pragma unroll
            for (int q = 0; q < WPP; q++) w[i % VX_RING][q] = vx_load_w(wp + ((size_t)pi * WPP + q) * 64, a.wcache);
            sc[i % VX_RING] = sp[(size_t)pi * 32];
        }
        if (DUAL && i < np) {
            // Both blocks of the pair issue their MFMAs into separate
            // accumulator sets before either result is read, so one block's
            // MFMA latency overlaps the other's reads and FMAs (one shared
            // set serialises MFMA -> wait -> reads per block).
            vx_half8 b[2][2], av[2][2];
#pragma unroll
            for (int blk = 0; blk < 2; blk++) {
                const int bl = 2 * i + blk;
                if (QT == 2) {
                    b[blk][0] = vx_unpack_q4(blk ? wv[0].z : wv[0].x, magic);
                    b[blk][1] = vx_unpack_q4(blk ? wv[0].w : wv[0].y, magic);
                } else {
                    b[blk][0] = vx_unpack_q8(wv[blk].x, wv[blk].y, magic);
                    b[blk][1] = vx_unpack_q8(wv[blk].z, wv[blk].w, magic);
                }
                av[blk][0] = __builtin_bit_cast(vx_half8, lds[((bl * 2 + 0) * 2 + h) * NS + slot]);
                av[blk][1] = __builtin_bit_cast(vx_half8, lds[((bl * 2 + 1) * 2 + h) * NS + slot]);
            }
            vx_f32x16 D0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[0][0], b[0][0], zero16, 0, 0, 0);
            vx_f32x16 D1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[1][0], b[1][0], zero16, 0, 0, 0);
            D0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[0][1], b[0][1], D0, 0, 0, 0);
            D1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[1][1], b[1][1], D1, 0, 0, 0);
#pragma unroll
            for (int blk = 0; blk < 2; blk++) {
                const int bl = 2 * i + blk;
                const vx_f32x16 &D = blk ? D1 : D0;
                const float d = vx_half_bits_to_float((sv >> (16 * blk)) & 0xFFFFu);
#pragma unroll
                for (int r = 0; r < R1; r++) {
                    float dh = D[r];
                    if (AVX2) {
                        const int m = 8 * (r / 4) + 4 * h + (r % 4);
                        dh = fmaf(-8.0f, m < M ? lcorr[bl * M + m] : 0.0f, dh);
                    }
                    acc[r] = fmaf(d, dh, acc[r]);
                    acc[r + 8] = fmaf(d, D[r + 8], acc[r + 8]);
                }
            }
        }
        if (!DUAL && i < np) {
            // one accumulator set, block by block (fewer registers: the M <= 4
            // decode GEMMs run more wavefronts per SIMD with it)
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
                const vx_half8 a0 = __builtin_bit_cast(vx_half8, lds[((bl * 2 + 0) * 2 + h) * NS + slot]);
                const vx_half8 a1 = __builtin_bit_cast(vx_half8, lds[((bl * 2 + 1) * 2 + h) * NS + slot]);
                vx_f32x16 D = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, zero16, 0, 0, 0);
                D = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, D, 0, 0, 0);
                const float d = vx_half_bits_to_float((sv >> (16 * blk)) & 0xFFFFu);
#pragma unroll
                for (int r = 0; r < R1; r++) {
                    float dh = D[r];
                    if (AVX2) {
                        const int m = 8 * (r / 4) + 4 * h + (r % 4);
                        dh = fmaf(-8.0f, m < M ? lcorr[bl * M + m] : 0.0f, dh);
                    }
                    acc[r] = fmaf(d, dh, acc[r]);
                    acc[r + 8] = fmaf(d, D[r + 8], acc[r + 8]);
                }
            }
        }
        // Keep this pair's accumulation here: without it the compiler sinks
        // every result read and FMA below the last MFMA of the unrolled loop
        // and holds all accumulator sets live at once.
        if constexpr (DUAL) {
#pragma unroll
            for (int r = 0; r < R1; r++) asm volatile("" : "+v"(acc[r]), "+v"(acc[r + 8]));
        }
    }

    // 3. this slice's contribution, added in fp64.  Every load of the flush
    // (row scales, sums of squares, gate values) is issued before any of it
    // is used: with the loads inside the per-row branches each row waited
    // for its own round trip (at M = 9 five in a row; measured on MI355X,
    // 4096x4096 8.46 -> 6.56 us, 22016x4096 18.59 -> 16.90 us).
    const int n = T * 32 + c;
    const bool out_ok = tile_ok && n < a.n_out;
    const int chunk = p0 / a.rs_chunk;
    float osc[R1];
#pragma unroll
    for (int r = 0; r < R1; r++) {
        const int m = min(8 * (r / 4) + 4 * h + (r % 4), M - 1);
        osc[r] = (PANEL ? a.rscale[m * a.rs_ld + chunk] : lrs[m]) * a.scale;
    }
    if (a.ss) {
        double ssv[R1];
#pragma unroll
        for (int r = 0; r < R1; r++) ssv[r] = a.ss[min(8 * (r / 4) + 4 * h + (r % 4), M - 1)];
#pragma unroll
        for (int r = 0; r < R1; r++) osc[r] *= vx_rms_inv((float)ssv[r], a.ss_K);
    }
    bool keep[R1];
#pragma unroll
    for (int r = 0; r < R1; r++) keep[r] = 8 * (r / 4) + 4 * h + (r % 4) < M;
    if (a.gate && out_ok) {
        float gv[R1];
#pragma unroll
        for (int r = 0; r < R1; r++)
            gv[r] = a.gate[(size_t)min(8 * (r / 4) + 4 * h + (r % 4), M - 1) * a.ld_gate + n];
#pragma unroll
        for (int r = 0; r < R1; r++) keep[r] = keep[r] && !(fabsf(gv[r]) < a.thr);
    }
    if (out_ok) {
#pragma unroll
        for (int r = 0; r < R1; r++) {
            if (!keep[r]) continue;
            const int m = 8 * (r / 4) + 4 * h + (r % 4);
            const float v = (acc[r] + acc[r + 8]) * osc[r];
            __hip_atomic_fetch_add(&a.acc[(size_t)m * a.ld_acc + n], (double)v, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---------------------------------------------------------------------------
// Verify-batch GEMM (M = 5..16): v_mfma_f32_16x16x32_f16 on 64-row tiles
// ---------------------------------------------------------------------------
// The weights are the B operand: one MFMA multiplies the 16 activation slots
// (the rows' fp16 hi parts; a second MFMA chains the lo parts into the same
// accumulator) by 16 weight rows x one whole Q4_0/Q8_0 block (K = 32), so the
// four results a lane holds (activation rows 4G..4G+3 of one weight row) all
// take the scale of one block: 16 scale FMAs per 64 rows and block, and the
// MFMA results land in VGPRs (no accumulator-register reads).  Weights come
// from the matrix's 64-row tiled copy (vxh_qmat.tq/td) through buffer loads
// whose per-block offset is wave-uniform.
//
// Workgroup = NT tiles x NK consecutive K ranges of KB blocks, one wavefront
// each.  Its panel slice (NK*KB blocks, the vx_gemm_kernel LDS layout) is
// staged in LDS -- copied from a panel or built by a prologue kind -- except
// for a plain panel with one tile per workgroup, whose wavefronts read their
// slice from HBM with the weights.  Each wavefront scales its sums, waves
// along K add theirs in LDS in wave order, and the workgroup adds the total
// into the fp64 accumulator (one atomic per output and workgroup).

// MFMA sources stay live past the MFMAs of a block: a VGPR-destination MFMA
// whose destination overlaps its own A/B registers computes wrong values,
// and the compiler reuses a source that dies at the MFMA as its destination
// unless something reads the source afterwards.  The asm also reads the
// results, so it cannot move above the MFMAs.
#define VX_MFMA_KEEP4(D0, D1, D2, D3, A0, A1, B0, B1, B2, B3)                                   \
    asm volatile("" : "+v"(D0), "+v"(D1), "+v"(D2), "+v"(D3)                                  \
                 : "v"(A0), "v"(A1), "v"(B0), "v"(B1), "v"(B2), "v"(B3))

typedef float vx_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int vx_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int vx_u32x2 __attribute__((ext_vector_type(2)));

// vx_unpack_q4 with the high-nibble offset held in a register (a literal
// operand is re-materialised per block)
__device__ __forceinline__ vx_half8 vx_unpack_q4r(uint32_t q, uint32_t magic, uint32_t off16w)
{
    const uint32_t q8 = q >> 8;
    vx_half2 a = __builtin_bit_cast(vx_half2, vx_and_or(q, 0x000F000Fu, magic));
    vx_half2 b = __builtin_bit_cast(vx_half2, vx_and_or(q, 0x00F000F0u, magic));
    vx_half2 c = __builtin_bit_cast(vx_half2, vx_and_or(q8, 0x000F000Fu, magic));
    vx_half2 d = __builtin_bit_cast(vx_half2, vx_and_or(q8, 0x00F000F0u, magic));
    const vx_half2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const vx_half2 sc = {(_Float16)0.0625f, (_Float16)0.0625f};
    const vx_half2 off16 = __builtin_bit_cast(vx_half2, off16w);
    a = a + off;
    b = b * sc + off16;
    c = c + off;
    d = d * sc + off16;
    vx_half8 r = {a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
    return r;
}

template <int QT, int M, int NT, int NK, int KB, int RING, int PRO>
__global__ __launch_bounds__(64 * NT * NK) __attribute__((amdgpu_waves_per_eu(2))) void vx_vg_kernel(vx_gemm_args a)
{
    static_assert(M >= 2 && M <= 16 && KB % 2 == 0 && RING >= 1 && RING <= KB, "vg: shape");
    static_assert(PRO == VX_PRO_PANEL || PRO == VX_PRO_ROWS || PRO == VX_PRO_RESID || PRO == VX_PRO_SWIGLU,
                  "vg: prologue kind");
    constexpr int NW = NT * NK, NTH = 64 * NW;
    constexpr bool PANEL = PRO == VX_PRO_PANEL;
    constexpr bool ALDS = !(PANEL && NT == 1);   // slice staged in LDS
    constexpr int NS = 2 * M;
    constexpr int PPW = NK * KB / 2;             // block pairs of the workgroup's K range
    constexpr int UNITS = PPW * 8 * NS;
    constexpr int UPT = ALDS ? (UNITS + NTH - 1) / NTH : 1;
    constexpr int WPB = QT == 2 ? 1 : 2;         // 16-byte weight loads per lane and block
    __shared__ uint4 lds[ALDS ? UPT * NTH : 1];
    __shared__ float lrs[PANEL ? 1 : M];
    __shared__ float red[NK > 1 ? (NK - 1) * NT * 16 * 64 : 1];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t = wave % NT, kq = wave / NT;
    const int tg = blockIdx.x / a.n_splits, split = blockIdx.x % a.n_splits;
    const int tile = tg * NT + t;
    const bool tile_ok = tile < a.n_t64;
    const int tc = tile_ok ? tile : a.n_t64 - 1;
    const int p0 = split * PPW;
    const int np = min(PPW, a.n_pairs - p0);
    const int wb0 = 2 * p0 + kq * KB;                  // this wavefront's first block
    const int nbk = max(0, min(KB, a.n_blk - wb0));     // and its block count
    const int bcl = min(wb0, a.n_blk - 1);
    const int nbl = max(nbk, 1);
    const int G = lane >> 4, mrow = min(lane & 15, M - 1);
    uint32_t magic, off16;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
    asm volatile("v_mov_b32 %0, 0xd480d480" : "=v"(off16));   // -72 (fp16) twice

    // 0. prologue kinds: this workgroup's share of the accumulator to clear
    if constexpr (!PANEL) {
        if (a.p.clr) {
            const long per = (a.p.n_clr + gridDim.x - 1) / gridDim.x;
            const long b = (long)blockIdx.x * per, e = min(b + per, a.p.n_clr);
            for (long i = b + threadIdx.x; i < e; i += NTH) a.p.clr[i] = 0.0;
        }
    }
    // 1. the slice's panel units or source rows, ahead of the weights
    const int units = np * 8 * NS;
    uint4 pv[PANEL && ALDS ? UPT : 1];
    if constexpr (PANEL && ALDS) {
        const uint4 *psrc = a.panel + (size_t)p0 * 8 * NS;
#pragma unroll
        for (int j = 0; j < UPT; j++) pv[j] = psrc[min(j * NTH + (int)threadIdx.x, units - 1)];
    }
    constexpr int RW = PANEL ? 1 : (M + NW - 1) / NW;
    constexpr int GL = PANEL ? 1 : (PPW * 8 + 63) / 64;
    constexpr bool PRELOAD = !PANEL && RW * GL <= 4;
    const int ng = np * 8, k0 = p0 * 64;
    vx_pro_raw raw[PRELOAD ? RW : 1][PRELOAD ? GL : 1];
    if constexpr (PRELOAD) {
#pragma unroll
        for (int rr = 0; rr < RW; rr++) {
            const int m = wave + NW * rr;
            if (m >= M) continue;
#pragma unroll
            for (int j = 0; j < GL; j++) {
                const int g = lane + 64 * j;
                if (g < ng && k0 + 8 * g < a.p.K) vx_pro_load<PRO>(a.p, m, k0 + 8 * g, raw[rr][j]);
            }
        }
    }
    // 2. the first RING blocks of weights and scales (and of the slice when
    // it is read from HBM)
    const __amdgpu_buffer_rsrc_t rwq = __builtin_amdgcn_make_buffer_rsrc((void *)a.tq, (short)0, (int)a.tq_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rwd = __builtin_amdgcn_make_buffer_rsrc((void *)a.td, (short)0, (int)a.td_bytes, 0x00020000);
    const uint32_t wbase = ((uint32_t)tc * a.n_blk + bcl) * (1024u * WPB);
    const uint32_t sbase = ((uint32_t)tc * a.n_blk + bcl) * 128u;
    const uint32_t wlo = lane * 16u, slo = (lane & 15) * 8u;
    const int cpol = a.wcache ? 0 : 2;   // nt unless the matrix is marked cached
    uint4 w[RING][WPB];
    uint2 sc[RING];
    uint4 arh[ALDS ? 1 : RING], arl[ALDS ? 1 : RING];
    const __amdgpu_buffer_rsrc_t rpa = __builtin_amdgcn_make_buffer_rsrc((void *)a.panel, (short)0, (int)a.pan_bytes, 0x00020000);
    const uint32_t alo = ((((G & 1) * 2 + (G >> 1)) * NS) + mrow) * 16u;
    const uint32_t abase = (uint32_t)bcl * 4u * NS * 16u;
#define VX_VG_WLD(bi, q)                                                                                   \
    ({                                                                                                     \
        const vx_u32x4 v_ = cpol ? __builtin_amdgcn_raw_buffer_load_b128(rwq, wlo, wbase + (uint32_t)(bi) * (1024u * WPB) + (q) * 1024u, 2) \
                                 : __builtin_amdgcn_raw_buffer_load_b128(rwq, wlo, wbase + (uint32_t)(bi) * (1024u * WPB) + (q) * 1024u, 0); \
        make_uint4(v_.x, v_.y, v_.z, v_.w);                                                                \
    })
#define VX_VG_SLD(bi)                                                                                      \
    ({                                                                                                     \
        const vx_u32x2 v_ = __builtin_amdgcn_raw_buffer_load_b64(rwd, slo, sbase + (uint32_t)(bi) * 128u, 0); \
        make_uint2(v_.x, v_.y);                                                                            \
    })
#define VX_VG_ALD(bi, hl)                                                                                  \
    ({                                                                                                     \
        const vx_u32x4 v_ = __builtin_amdgcn_raw_buffer_load_b128(rpa, alo, abase + (uint32_t)(bi) * 4u * NS * 16u + (hl) * M * 16u, 0); \
        make_uint4(v_.x, v_.y, v_.z, v_.w);                                                                \
    })
#pragma unroll
    for (int i = 0; i < RING; i++) {
        const int bi = min(i, nbl - 1);
#pragma unroll
        for (int q = 0; q < WPB; q++) w[i][q] = VX_VG_WLD(bi, q);
        sc[i] = VX_VG_SLD(bi);
        if constexpr (!ALDS) {
            arh[i] = VX_VG_ALD(bi, 0);
            arl[i] = VX_VG_ALD(bi, 1);
        }
    }
    // 3. the LDS slice
    if constexpr (ALDS) {
        if constexpr (PANEL) {
#pragma unroll
            for (int j = 0; j < UPT; j++) lds[j * NTH + threadIdx.x] = pv[j];
        } else {
            const bool lead = tg == 0;
#pragma unroll
            for (int rr = 0; rr < RW; rr++) {
                const int m = wave + NW * rr;
                if (m >= M) continue;
                const float rin = (PRO == VX_PRO_SWIGLU && a.p.ss_in) ? vx_rms_inv((float)a.p.ss_in[m], a.p.ss_K)
                                                                      : 1.0f;
                float v[GL][8];
                float ss = 0.0f, amax = 0.0f;
#pragma unroll
                for (int j = 0; j < GL; j++) {
                    const int g = lane + 64 * j, e0 = k0 + 8 * g;
#pragma unroll
                    for (int kk = 0; kk < 8; kk++) v[j][kk] = 0.0f;
                    if (g < ng && e0 < a.p.K) {
                        vx_pro_raw r;
                        if constexpr (PRELOAD) r = raw[rr][j];
                        else vx_pro_load<PRO>(a.p, m, e0, r);
                        float *xo = (lead && a.p.x_out) ? a.p.x_out + (size_t)m * a.p.ld_xout + e0 : nullptr;
                        vx_pro_values<PRO>(a.p, r, rin, xo, v[j], ss);
                    }
#pragma unroll
                    for (int kk = 0; kk < 8; kk++) amax = fmaxf(amax, fabsf(v[j][kk]));
                }
                amax = vx_wave_max64(amax);
                float rs;
                const float scl = vx_row_scale(amax, &rs);
                if (lane == 0) lrs[m] = rs;
                if (PRO != VX_PRO_SWIGLU && lead && a.p.ss) {
                    ss = vx_wave_sum64(ss);
                    if (lane == 0)
                        __hip_atomic_fetch_add(&a.p.ss[m], (double)ss, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
                for (int j = 0; j < GL; j++) {
                    const int g = lane + 64 * j;
                    if (g >= ng) continue;
                    vx_half8 hi, lo;
#pragma unroll
                    for (int kk = 0; kk < 8; kk++) {
                        const float xv = v[j][kk] * scl;
                        const _Float16 th = (_Float16)xv;
                        hi[kk] = th;
                        lo[kk] = (_Float16)(xv - (float)th);
                    }
                    const int b = g >> 2, h2 = (g >> 1) & 1, s2 = g & 1;
                    const int base = ((b * 2 + s2) * 2 + h2) * NS;
                    lds[base + m] = __builtin_bit_cast(uint4, hi);
                    lds[base + M + m] = __builtin_bit_cast(uint4, lo);
                }
            }
        }
        __syncthreads();
    }

    // 4. the K range: per block 4 (Q4_0) or 8 (Q8_0) dwords of weights unpack
    // into the four row groups' B operands, eight MFMAs, sixteen scale FMAs
    vx_f32x4 acc[4];
#pragma unroll
    for (int rg = 0; rg < 4; rg++) acc[rg] = vx_f32x4{0.f, 0.f, 0.f, 0.f};
    const vx_f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    const int lsel = ((G & 1) * 2 + (G >> 1)) * NS + mrow;
#pragma unroll
    for (int i = 0; i < KB; i++) {
        uint4 wv[WPB];
#pragma unroll
        for (int q = 0; q < WPB; q++) wv[q] = w[i % RING][q];
        const uint2 sv = sc[i % RING];
        uint4 ahv, alv;
        if constexpr (ALDS) {
            const int u = (kq * KB + i) * 4 * NS + lsel;
            ahv = lds[u];
            alv = lds[u + M];
        } else {
            ahv = arh[i % RING];
            alv = arl[i % RING];
        }
        if (i + RING < KB) {
            const int bi = min(i + RING, nbl - 1);
#pragma unroll
            for (int q = 0; q < WPB; q++) w[i % RING][q] = VX_VG_WLD(bi, q);
            sc[i % RING] = VX_VG_SLD(bi);
            if constexpr (!ALDS) {
                arh[i % RING] = VX_VG_ALD(bi, 0);
                arl[i % RING] = VX_VG_ALD(bi, 1);
            }
        }
        if (i < nbk) {
            const vx_half8 A0 = __builtin_bit_cast(vx_half8, ahv);
            const vx_half8 A1 = __builtin_bit_cast(vx_half8, alv);
            vx_half8 B0, B1, B2, B3;
            if constexpr (QT == 2) {
                B0 = vx_unpack_q4r(wv[0].x, magic, off16);
                B1 = vx_unpack_q4r(wv[0].y, magic, off16);
                B2 = vx_unpack_q4r(wv[0].z, magic, off16);
                B3 = vx_unpack_q4r(wv[0].w, magic, off16);
            } else {
                B0 = vx_unpack_q8(wv[0].x, wv[0].y, magic);
                B1 = vx_unpack_q8(wv[0].z, wv[0].w, magic);
                B2 = vx_unpack_q8(wv[WPB - 1].x, wv[WPB - 1].y, magic);
                B3 = vx_unpack_q8(wv[WPB - 1].z, wv[WPB - 1].w, magic);
            }
            vx_f32x4 D0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, B0, zero4, 0, 0, 0);
            vx_f32x4 D1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, B1, zero4, 0, 0, 0);
            vx_f32x4 D2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, B2, zero4, 0, 0, 0);
            vx_f32x4 D3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, B3, zero4, 0, 0, 0);
            D0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, B0, D0, 0, 0, 0);
            D1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, B1, D1, 0, 0, 0);
            D2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, B2, D2, 0, 0, 0);
            D3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, B3, D3, 0, 0, 0);
            VX_MFMA_KEEP4(D0, D1, D2, D3, A0, A1, B0, B1, B2, B3);
            const float d0 = vx_half_bits_to_float(sv.x & 0xFFFFu);
            const float d1 = vx_half_bits_to_float(sv.x >> 16);
            const float d2 = vx_half_bits_to_float(sv.y & 0xFFFFu);
            const float d3 = vx_half_bits_to_float(sv.y >> 16);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                acc[0][r] = fmaf(d0, D0[r], acc[0][r]);
                acc[1][r] = fmaf(d1, D1[r], acc[1][r]);
                acc[2][r] = fmaf(d2, D2[r], acc[2][r]);
                acc[3][r] = fmaf(d3, D3[r], acc[3][r]);
            }
        }
    }
#undef VX_VG_WLD
#undef VX_VG_SLD
#undef VX_VG_ALD

    // 5. output scale of each row (the slice's power of two, the synthetic
    // scale, the deferred norm), the sum along K, the fp64 add.  A K range
    // lies inside one panel scale chunk (checked by the launcher).
    const int chunk = (bcl / 2) / a.rs_chunk;
    float osc[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int mr = min(4 * G + r, M - 1);
        osc[r] = (PANEL ? a.rscale[mr * a.rs_ld + chunk] : lrs[mr]) * a.scale;
    }
    if (a.ss) {
        double ssv[4];
#pragma unroll
        for (int r = 0; r < 4; r++) ssv[r] = a.ss[min(4 * G + r, M - 1)];
#pragma unroll
        for (int r = 0; r < 4; r++) osc[r] *= vx_rms_inv((float)ssv[r], a.ss_K);
    }
#pragma unroll
    for (int rg = 0; rg < 4; rg++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[rg][r] *= osc[r];
    if constexpr (NK > 1) {
        if (kq > 0) {
#pragma unroll
            for (int rg = 0; rg < 4; rg++)
#pragma unroll
                for (int r = 0; r < 4; r++) red[(((kq - 1) * NT + t) * 16 + rg * 4 + r) * 64 + lane] = acc[rg][r];
        }
        __syncthreads();
        if (kq != 0) return;
#pragma unroll
        for (int q = 1; q < NK; q++)
#pragma unroll
            for (int rg = 0; rg < 4; rg++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[rg][r] += red[(((q - 1) * NT + t) * 16 + rg * 4 + r) * 64 + lane];
    }
    if (!tile_ok) return;
    bool keep[4][4];
#pragma unroll
    for (int rg = 0; rg < 4; rg++)
#pragma unroll
        for (int r = 0; r < 4; r++)
            keep[rg][r] = 4 * G + r < M && tile * 64 + rg * 16 + (lane & 15) < a.n_out;
    if (a.gate) {
        float gv[4][4];
#pragma unroll
        for (int rg = 0; rg < 4; rg++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int n = min(tile * 64 + rg * 16 + (lane & 15), a.n_out - 1);
                gv[rg][r] = a.gate[(size_t)min(4 * G + r, M - 1) * a.ld_gate + n];
            }
#pragma unroll
        for (int rg = 0; rg < 4; rg++)
#pragma unroll
            for (int r = 0; r < 4; r++) keep[rg][r] = keep[rg][r] && !(fabsf(gv[rg][r]) < a.thr);
    }
#pragma unroll
    for (int rg = 0; rg < 4; rg++) {
        const int n = tile * 64 + rg * 16 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            if (!keep[rg][r]) continue;
            __hip_atomic_fetch_add(&a.acc[(size_t)(4 * G + r) * a.ld_acc + n], (double)acc[rg][r], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int QT, int M, int NT, int NK, int KB, int RING, int PRO>
static int vx_launch_vg(const vxh_qmat *W, vx_gemm_args &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1)
{
    constexpr int PPW = NK * KB / 2;
    a.n_pairs = W->n_pairs;
    a.n_blk = W->n_cols / 32;
    a.n_t64 = (W->n_rows + 63) / 64;
    a.n_splits = (W->n_pairs + PPW - 1) / PPW;
    a.tq = W->tq;
    a.td = W->td;
    a.tq_bytes = (uint32_t)((size_t)a.n_t64 * a.n_blk * (QT == 2 ? 1024u : 2048u));
    a.td_bytes = (uint32_t)((size_t)a.n_t64 * a.n_blk * 128u);
    a.pan_bytes = (uint32_t)((size_t)W->n_pairs * 8 * 2 * M * 16);
    if (PRO == VX_PRO_PANEL && a.rs_ld > 1 && a.rs_chunk % PPW)
        return vxh_fail(VXH_ERR_PARAM, "gemm: K range of %d pairs crosses a %d-pair scale chunk", PPW, a.rs_chunk);
    const int groups = (a.n_t64 + NT - 1) / NT;
    if (e0 || e1)   // events recorded by the dispatch itself around the kernel
        hipExtLaunchKernelGGL(vx_vg_kernel<QT, M, NT, NK, KB, RING, PRO>, dim3(groups * a.n_splits),
                              dim3(64 * NT * NK), 0, st, e0, e1, 0, a);
    else
        vx_vg_kernel<QT, M, NT, NK, KB, RING, PRO><<<groups * a.n_splits, 64 * NT * NK, 0, st>>>(a);
    VXH_LAUNCHED();
    return VXH_OK;
}

// Work split of a verify-batch GEMM, measured on MI355X at M = 9 with the
// inputs of the verify forward (kernel durations, weights rotated past the
// Infinity Cache, fp64 atomics included):
//   plain panel (down, 4096x11008): one tile per workgroup, four wavefronts
//     along K of 8 blocks, 8-block ring: 10.5-10.7 us (vx_gemm_kernel 12.4);
//   rows (attention output, 4096x4096): two tiles x four K ranges of 4
//     blocks: 6.5 us (6.8);
//   residual + norm prologue, 32000x4096 (logits): four tiles, 32-block
//     ranges, 6-block ring: 23.0 us (26.8).
// The residual prologue on narrower matrices stays with vx_gemm_kernel
// (returns 1): every workgroup rebuilds its slice from x, the fp64 pending
// sums and the norm weight, and the 8-wavefront 32-row tiles of that kernel
// hide it better (12288x4096 12.7 us against 12.9-20 for every split tried
// here, 22016x4096 18.3 against 18.4-31).
template <int QT, int M, int PRO>
static int vx_launch_verify(const vxh_qmat *W, vx_gemm_args &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1)
{
    const int t64 = (W->n_rows + 63) / 64;
    if constexpr (PRO == VX_PRO_PANEL) return vx_launch_vg<QT, M, 1, 4, 8, 8, PRO>(W, a, st, e0, e1);
    if constexpr (PRO == VX_PRO_ROWS) return vx_launch_vg<QT, M, 2, 4, 4, 2, PRO>(W, a, st, e0, e1);
    if constexpr (PRO == VX_PRO_RESID)
        if (t64 >= 400) return vx_launch_vg<QT, M, 4, 1, 32, 6, PRO>(W, a, st, e0, e1);
    return 1;
}

template <int QT, int M, bool AVX2, int PPW, int PRO>
static int vx_launch_ppw(const vxh_qmat *W, vx_gemm_args &a, hipStream_t st, hipEvent_t e0,
                         hipEvent_t e1)
{
    a.n_tiles = W->n_rows / 32;
    a.n_pairs = W->n_pairs;
    a.n_splits = (W->n_pairs + PPW - 1) / PPW;
    if (PRO == VX_PRO_PANEL && a.rs_ld > 1 && a.rs_chunk % PPW)
        return vxh_fail(VXH_ERR_PARAM, "gemm: K slice of %d pairs crosses a %d-pair scale chunk", PPW,
                        a.rs_chunk);
    constexpr int NWV = vx_nwv<QT, M, AVX2, PPW, PRO>::v;
    const int groups = (a.n_tiles + NWV - 1) / NWV;
    if (e0 || e1)   // events recorded by the dispatch itself around the kernel
        hipExtLaunchKernelGGL(vx_gemm_kernel<QT, M, AVX2, PPW, PRO>, dim3(groups * a.n_splits),
                              dim3(64 * NWV), 0, st, e0, e1, 0, a);
    else
        vx_gemm_kernel<QT, M, AVX2, PPW, PRO><<<groups * a.n_splits, 64 * NWV, 0, st>>>(a);
    VXH_LAUNCHED();
    return VXH_OK;
}

// Verify batches (M >= 5) from a plain panel or rows, and the widest residual
// GEMMs, take vx_vg_kernel on the matrix's 64-row tiled copy; decode rows
// (M <= 4: latency-bound launches, where vx_vg_kernel measured no faster:
// 2560x2048 3.7 -> 3.8 us, 11264x2048 5.3 -> 5.5), the other residual
// prologues and AVX2-lane panels take vx_gemm_kernel.
template <int QT, int M, bool AVX2, int PRO>
static int vx_launch_gemm(const vxh_qmat *W, vx_gemm_args &a, hipStream_t st, hipEvent_t e0,
                          hipEvent_t e1)
{
    if constexpr (M >= 5 && !AVX2 && PRO != VX_PRO_ATTN)
        if (W->tq && W->td) {
            const int rc = vx_launch_verify<QT, M, PRO>(W, a, st, e0, e1);
            if (rc <= 0) return rc;
        }
    typedef vx_ppw_set<QT, M> S;
    const long groups = (W->n_rows / 32 + 3) / 4;
    const int cand[3] = {S::v0, S::v1, S::v2};
    int pick = S::n - 1;
    if (QT == 2 && M >= 5 && M <= 12 && (PRO == VX_PRO_PANEL || PRO == VX_PRO_ROWS)) {
        // verify batches (Q4_0) from a plain panel or rows: the 16-pair slice
        // whenever it still gives every CU more than one workgroup (measured
        // on MI355X at M = 9: 4096x11008 and 32000x4096 4-10% faster than 8
        // pairs; 4096x4096 keeps 8 -- 128 workgroups leave half the CUs
        // idle).  Residual prologues keep 8: twice the slice per workgroup
        // costs them more than the longer stream saves (12288x4096 12.7 ->
        // 15.4 us).
        pick = groups * ((W->n_pairs + 15) / 16) >= 340 ? 1 : 0;
    } else {
        for (int i = 0; i < S::n; i++)
            if (groups * ((W->n_pairs + cand[i] - 1) / cand[i]) <= S::target) { pick = i; break; }
    }
    if (pick == 0) return vx_launch_ppw<QT, M, AVX2, S::v0, PRO>(W, a, st, e0, e1);
    if (pick == 1) return vx_launch_ppw<QT, M, AVX2, S::v1, PRO>(W, a, st, e0, e1);
    return vx_launch_ppw<QT, M, AVX2, S::v2, PRO>(W, a, st, e0, e1);
}

template <int M, int PRO>
static int vx_dispatch_m(const vxh_qmat *W, int avx2, vx_gemm_args &a, hipStream_t st, hipEvent_t e0,
                         hipEvent_t e1)
{
    if (W->type != 2 && W->type != 8)
        return vxh_fail(VXH_ERR_UNSUPPORTED, "matrix type %d: this GEMM takes Q4_0 and Q8_0", W->type);
    if (W->type == 2) {
        if constexpr (PRO == VX_PRO_PANEL)
            if (avx2) return vx_launch_gemm<2, M, true, PRO>(W, a, st, e0, e1);
        return vx_launch_gemm<2, M, false, PRO>(W, a, st, e0, e1);
    }
    if (avx2) return vxh_fail(VXH_ERR_UNSUPPORTED, "AVX2-lane panels apply to Q4_0 only");
    return vx_launch_gemm<8, M, false, PRO>(W, a, st, e0, e1);
}

// M = 1..16 to the templates
template <int PRO = VX_PRO_PANEL>
static int vx_dispatch(const vxh_qmat *W, int M, int avx2, vx_gemm_args &a, hipStream_t st, hipEvent_t e0,
                       hipEvent_t e1)
{
    switch (M) {
    case 1: return vx_dispatch_m<1, PRO>(W, avx2, a, st, e0, e1);
    case 2: return vx_dispatch_m<2, PRO>(W, avx2, a, st, e0, e1);
    case 3: return vx_dispatch_m<3, PRO>(W, avx2, a, st, e0, e1);
    case 4: return vx_dispatch_m<4, PRO>(W, avx2, a, st, e0, e1);
    case 5: return vx_dispatch_m<5, PRO>(W, avx2, a, st, e0, e1);
    case 6: return vx_dispatch_m<6, PRO>(W, avx2, a, st, e0, e1);
    case 7: return vx_dispatch_m<7, PRO>(W, avx2, a, st, e0, e1);
    case 8: return vx_dispatch_m<8, PRO>(W, avx2, a, st, e0, e1);
    case 9: return vx_dispatch_m<9, PRO>(W, avx2, a, st, e0, e1);
    case 10: return vx_dispatch_m<10, PRO>(W, avx2, a, st, e0, e1);
    case 11: return vx_dispatch_m<11, PRO>(W, avx2, a, st, e0, e1);
    case 12: return vx_dispatch_m<12, PRO>(W, avx2, a, st, e0, e1);
    case 13: return vx_dispatch_m<13, PRO>(W, avx2, a, st, e0, e1);
    case 14: return vx_dispatch_m<14, PRO>(W, avx2, a, st, e0, e1);
    case 15: return vx_dispatch_m<15, PRO>(W, avx2, a, st, e0, e1);
    default: return vx_dispatch_m<16, PRO>(W, avx2, a, st, e0, e1);
    }
}
