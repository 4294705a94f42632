// Prompt prefill at large M: the reference runs the prompt one token per
// forward (src/speculative.c:100-107, src/model.c:450-616); here a chunk of
// up to a few hundred prompt rows runs as one batch.
//
//   vx_pf_gemm_kernel    Y = X W^T (+ R) for M rows, compute-bound MFMA tiles
//   vx_pf_rope_kv_kernel RoPE of q|k rows and the k/v cache store (fp32 rows)
//   vx_pf_swiglu_kernel  h = |silu(g)| < thr ? 0 : silu(g) * u
//
// GEMM arithmetic.  Q4_0/Q8_0 weights are d * q with q = s - 8 (resp. the
// int8) exact in fp16 and d an fp16 scale; their product has at most 15
// (resp. 19) significant bits, so w = w_hi + w_lo with w_hi = fp16(d q) and
// w_lo = fp16(d q - w_hi) is exact (v_pk_fma_f16 rounds the exact remainder,
// which fits fp16; its last bit is never below d's, 2^-24).  Activations are
// split the same way into x_hi + x_lo.  The MFMA then accumulates
// x_hi w_hi + x_lo w_hi + x_hi w_lo over the whole K range in fp32 -- no
// per-block rescaling, unlike the skinny verify kernel; the dropped x_lo w_lo
// term is below 2^-22 of each product.
#include "vxh_internal.h"
#include "vxh_gemm_core.h"

#define PF_BM 64                 // activation rows per workgroup
#define PF_MT (PF_BM / 32)       // 32-row MFMA tiles per workgroup
#define PF_STAGE (PF_MT * 2 * 2 * 2 * 64)   // A units (8 fp16) of one block pair: [mt][blk][s][hl][lane]
#define PF_RING 3                // weight pairs in flight per wavefront

struct vx_pf_args {
    const uint4 *wq;
    const uint32_t *wd;
    int n_tiles, n_pairs, K;
    const uint4 *px;   // rows panel (vxh_rows_panel): [row group][pair][PF_STAGE units]
    const float *rs;   // [M] power-of-two row scales of the panel
    int M;
    float *y;
    int ldy, n_out;
    const float *r;
    int ldr;
    float scale;
};

// Workgroup = 4 wavefronts = 4 weight tiles of 32 rows (128 output columns)
// x PF_BM activation rows.  Per block pair (64 of K) the workgroup copies the
// activation slice of the rows panel into LDS -- MFMA A units (lane l: row
// l%32, elements 16(l/32) + 8s .. +7 of block blk, matching the weight
// layout's lane split), hi and lo, converted once per GEMM input by
// vx_pf_panel_kernel instead of by each of the column workgroups (which
// spent more VALU on it than on the weights) -- double-buffered: pair p+1 is
// copied into the other buffer while pair p is multiplied, one barrier per
// pair.  Each wavefront keeps
// PF_RING pairs of its weights in flight, unpacks a pair once and runs 3
// MFMAs per (tile, block, K half).  64-row tiles keep the grid at several
// workgroups per CU for the 4096-column matrices of a 512-row chunk.
template <int QT>
__global__ __launch_bounds__(256) void vx_pf_gemm_kernel(vx_pf_args a)
{
    constexpr int WPP = QT == 2 ? 1 : 2;
    __shared__ uint4 lds[2 * PF_STAGE];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int T = blockIdx.x * 4 + wave;
    const bool tile_ok = T < a.n_tiles;
    const int Tc = tile_ok ? T : a.n_tiles - 1;
    const int m0 = blockIdx.y * PF_BM;
    const int c = lane & 31, h = lane >> 5;
    const uint32_t magic = 0x64006400u;
    const uint4 *wp = a.wq + (size_t)Tc * a.n_pairs * WPP * 64 + lane;
    const uint32_t *sp = a.wd + (size_t)Tc * a.n_pairs * 32 + c;

    // staging: the pair's PF_STAGE units of the rows panel, already in the
    // LDS layout: a contiguous 16 KiB copy, 4 units per thread
    constexpr int XU = PF_STAGE / 256;
    const uint4 *xp = a.px + (size_t)blockIdx.y * a.n_pairs * PF_STAGE + threadIdx.x;
    uint4 xa[XU];
    auto load_x = [&](int p) {
#pragma unroll
        for (int j = 0; j < XU; j++) xa[j] = xp[(size_t)p * PF_STAGE + 256 * j];
    };
    auto store_x = [&](uint4 *buf) {
#pragma unroll
        for (int j = 0; j < XU; j++) buf[threadIdx.x + 256 * j] = xa[j];
    };

    vx_f32x16 D[PF_MT];
#pragma unroll
    for (int mt = 0; mt < PF_MT; mt++) D[mt] = vx_f32x16{};
    uint4 w[PF_RING][WPP];
    uint32_t sc[PF_RING];
#pragma unroll
    for (int i = 0; i < PF_RING; i++) {
        const int pi = min(i, a.n_pairs - 1);
#pragma unroll
        for (int q = 0; q < WPP; q++) w[i][q] = wp[((size_t)pi * WPP + q) * 64];
        sc[i] = sp[(size_t)pi * 32];
    }
    load_x(0);
    store_x(lds);
    if (a.n_pairs > 1) load_x(1);
    __syncthreads();
    for (int p0 = 0; p0 < a.n_pairs; p0 += PF_RING) {
#pragma unroll
        for (int i = 0; i < PF_RING; i++) {
            const int p = p0 + i;
            if (p >= a.n_pairs) break;
            const uint4 *cur = lds + (p & 1) * PF_STAGE;
            // the next pair's activations into the other buffer (free since
            // the barrier that ended pair p-1), then the one after in flight
            if (p + 1 < a.n_pairs) {
                store_x(lds + ((p + 1) & 1) * PF_STAGE);
                if (p + 2 < a.n_pairs) load_x(p + 2);
            }
            uint4 wv[WPP];
#pragma unroll
            for (int q = 0; q < WPP; q++) wv[q] = w[i][q];
            const uint32_t sv = sc[i];
            {
                const int pn = min(p + PF_RING, a.n_pairs - 1);
#pragma unroll
                for (int q = 0; q < WPP; q++) w[i][q] = wp[((size_t)pn * WPP + q) * 64];
                sc[i] = sp[(size_t)pn * 32];
            }
            // weights of the pair as exact hi + lo fp16 terms
            vx_half8 bh[2][2], bl[2][2];
#pragma unroll
            for (int blk = 0; blk < 2; blk++) {
                vx_half8 q0, q1;
                if (QT == 2) {
                    q0 = vx_unpack_q4(blk ? wv[0].z : wv[0].x, magic);
                    q1 = vx_unpack_q4(blk ? wv[0].w : wv[0].y, magic);
                } else {
                    q0 = vx_unpack_q8(wv[blk].x, wv[blk].y, magic);
                    q1 = vx_unpack_q8(wv[blk].z, wv[blk].w, magic);
                }
                const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)((sv >> (16 * blk)) & 0xFFFFu));
                vx_half8 dd;
#pragma unroll
                for (int e = 0; e < 8; e++) dd[e] = d;
                bh[blk][0] = q0 * dd;
                bh[blk][1] = q1 * dd;
                bl[blk][0] = __builtin_elementwise_fma(q0, dd, -bh[blk][0]);
                bl[blk][1] = __builtin_elementwise_fma(q1, dd, -bh[blk][1]);
            }
#pragma unroll
            for (int blk = 0; blk < 2; blk++) {
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    vx_half8 ah[PF_MT], al[PF_MT];
#pragma unroll
                    for (int mt = 0; mt < PF_MT; mt++) {
                        const int rest = (mt * 2 + blk) * 2 + s;
                        ah[mt] = __builtin_bit_cast(vx_half8, cur[(rest * 2 + 0) * 64 + lane]);
                        al[mt] = __builtin_bit_cast(vx_half8, cur[(rest * 2 + 1) * 64 + lane]);
                    }
#pragma unroll
                    for (int mt = 0; mt < PF_MT; mt++)
                        D[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[mt], bh[blk][s], D[mt], 0, 0, 0);
#pragma unroll
                    for (int mt = 0; mt < PF_MT; mt++)
                        D[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[mt], bh[blk][s], D[mt], 0, 0, 0);
#pragma unroll
                    for (int mt = 0; mt < PF_MT; mt++)
                        D[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[mt], bl[blk][s], D[mt], 0, 0, 0);
                }
            }
            __syncthreads();
        }
    }
    const int n = T * 32 + c;
    if (!tile_ok || n >= a.n_out) return;
#pragma unroll
    for (int mt = 0; mt < PF_MT; mt++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = m0 + mt * 32 + 8 * (r / 4) + 4 * h + (r % 4);
            if (row >= a.M) continue;
            float v = (D[mt][r] * a.rs[row]) * a.scale;   // the row scale is a power of two
            if (a.r) v = a.r[(size_t)row * a.ldr + n] + v;
            a.y[(size_t)row * a.ldy + n] = v;
        }
    }
}

// Rows panel: fp32 rows x[M][ldx] as the GEMM's LDS stages.  Unit u of a
// (row group rg, pair p) stage, u = ((mt*2 + blk)*2 + s)*64 + ln, holds row
// 64 rg + 32 mt + ln % 32, elements 64 p + 32 blk + 16 (ln/32) + 8 s .. + 7,
// as hi = fp16(x') and (64 units further) lo = fp16(x' - hi).  One workgroup
// per row: x' = x 2^-e with e from the row's largest magnitude (vx_row_scale:
// |x'| < 1), so no element overflows fp16 and a row of small values keeps
// the low parts' bits; rs[row] = 2^e goes back in in the GEMM epilogue,
// exactly.  Rows past M (up to the 64-row group) and columns past K are
// zeros.
__global__ __launch_bounds__(256) void vx_pf_panel_kernel(const float *__restrict__ x, int ldx, int M, int K,
                                                          int n_pairs, uint4 *__restrict__ px, float *__restrict__ rs)
{
    const int row = blockIdx.x;
    const int rg = row / PF_BM, mt = (row % PF_BM) / 32, l32 = row % 32;
    const bool live = row < M;
    const float *xr = x + (size_t)(live ? row : 0) * ldx;
    __shared__ float red[4];
    float amax = 0.0f;
    if (live)
        for (int k = 8 * threadIdx.x; k < K; k += 8 * 256) {
            const float4 a = *(const float4 *)(xr + k), b = *(const float4 *)(xr + k + 4);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
        }
    amax = vx_wave_max64(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float rsv;
    const float sc = live ? vx_row_scale(amax, &rsv) : 1.0f;
    if (live && threadIdx.x == 0) rs[row] = rsv;
    for (int k = 8 * threadIdx.x; k < n_pairs * 64; k += 8 * 256) {
        float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (live && k < K) {   // K % 32 == 0: a block is wholly in range or out
            const float4 a = *(const float4 *)(xr + k), b = *(const float4 *)(xr + k + 4);
            v[0] = a.x * sc; v[1] = a.y * sc; v[2] = a.z * sc; v[3] = a.w * sc;
            v[4] = b.x * sc; v[5] = b.y * sc; v[6] = b.z * sc; v[7] = b.w * sc;
        }
        vx_half8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const _Float16 t = (_Float16)v[e];
            hi[e] = t;
            lo[e] = (_Float16)(v[e] - (float)t);
        }
        const int p = k / 64, blk = (k / 32) & 1, half = (k / 16) & 1, s = (k / 8) & 1;
        uint4 *o = px + ((size_t)rg * n_pairs + p) * PF_STAGE + ((mt * 2 + blk) * 2 + s) * 128 + l32 + 32 * half;
        o[0] = __builtin_bit_cast(uint4, hi);
        o[64] = __builtin_bit_cast(uint4, lo);
    }
}

// the row scales follow the stages (16-byte aligned)
static size_t vx_pf_stage_bytes(int M, int K)
{
    return (size_t)((M + PF_BM - 1) / PF_BM) * ((K + 63) / 64) * PF_STAGE * sizeof(uint4);
}

extern "C" size_t vxh_rows_panel_bytes(int M, int K)
{
    if (M < 1 || K < 1) return 0;
    return vx_pf_stage_bytes(M, K) + ((size_t)M * sizeof(float) + 15) / 16 * 16;
}

extern "C" int vxh_rows_panel(const float *X, int ldx, int M, int K, void *px, vxh_stream s)
{
    if (!X || !px || M < 1 || K < 32 || K % 32 || ldx < K || ldx % 4 || ((uintptr_t)X & 15) || ((uintptr_t)px & 15))
        return vxh_fail(VXH_ERR_PARAM, "rows_panel: M %d K %d ldx %d", M, K, ldx);
    const int n_pairs = (K + 63) / 64;
    const unsigned rows = (unsigned)((M + PF_BM - 1) / PF_BM * PF_BM);
    vx_pf_panel_kernel<<<rows, 256, 0, vxh_hs(s)>>>(X, ldx, M, K, n_pairs, (uint4 *)px,
                                                     (float *)((char *)px + vx_pf_stage_bytes(M, K)));
    VXH_LAUNCHED();
    return VXH_OK;
}

extern "C" int vxh_gemm_rows(const vxh_qmat *W, const void *px, int M, float *Y, int ldy, int n_out,
                             const float *R, int ldr, float scale, vxh_stream s)
{
    if (!W || !px || !Y || M < 1 || n_out < 1 || n_out > W->n_rows || ldy < n_out || (R && ldr < n_out) ||
        ((uintptr_t)px & 15))
        return vxh_fail(VXH_ERR_PARAM, "gemm_rows: M %d n_out %d (rows %d, K %d, ldy %d)", M, n_out, W->n_rows,
                        W->n_cols, ldy);
    if (W->type != 2 && W->type != 8) return vxh_fail(VXH_ERR_UNSUPPORTED, "gemm_rows: type %d", W->type);
    vx_pf_args a;
    a.wq = (const uint4 *)W->qs;
    a.wd = (const uint32_t *)W->d;
    a.n_tiles = W->n_rows / 32;
    a.n_pairs = W->n_pairs;
    a.K = W->n_cols;
    a.px = (const uint4 *)px;
    a.rs = (const float *)((const char *)px + vx_pf_stage_bytes(M, W->n_cols));
    a.M = M;
    a.y = Y;
    a.ldy = ldy;
    a.n_out = n_out;
    a.r = R;
    a.ldr = ldr;
    a.scale = scale;
    const dim3 grid((unsigned)((a.n_tiles + 3) / 4), (unsigned)((M + PF_BM - 1) / PF_BM));
    if (W->type == 2)
        vx_pf_gemm_kernel<2><<<grid, 256, 0, vxh_hs(s)>>>(a);
    else
        vx_pf_gemm_kernel<8><<<grid, 256, 0, vxh_hs(s)>>>(a);
    VXH_LAUNCHED();
    return VXH_OK;
}

// ---------------------------------------------------------------------------
// RoPE + KV store for fp32 q|k|v rows (the same per-pair arithmetic as the
// verify path's vx_rope_kv_kernel, src/tensor.c:249-270): one thread per
// (row, pair) of q and k, v copied.
// ---------------------------------------------------------------------------
__global__ void vx_pf_rope_kv_kernel(const float *__restrict__ qkv, int ld_qkv, int M, int n_past, int n_ctx,
                                     int n_heads, int n_kv_heads, int hd, const float *__restrict__ bq,
                                     const float *__restrict__ bk, const float *__restrict__ bv,
                                     const float *__restrict__ cs, const float *__restrict__ sn,
                                     float *__restrict__ q_out, int ldq, float *__restrict__ kc,
                                     float *__restrict__ vc)
{
    const int qd = n_heads * hd, kvd = n_kv_heads * hd;
    const int half = hd / 2;
    const int per_row = (qd + kvd) / 2 + kvd;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)M * per_row) return;
    const int m = (int)(idx / per_row), r = (int)(idx % per_row);
    const int rope_pos = n_past + m;
    const int pos = rope_pos < n_ctx ? rope_pos : n_ctx - 1;
    const float *row = qkv + (size_t)m * ld_qkv;
    if (r < (qd + kvd) / 2) {
        const int e = 2 * r;
        const bool isq = e < qd;
        const int el = isq ? e : e - qd;
        const int i = (el % hd) / 2;
        const float *bias = isq ? bq : bk;
        const float a = vx_norm_bias((double)row[e], 1.0f, bias, el);
        const float b = vx_norm_bias((double)row[e + 1], 1.0f, bias, el + 1);
        const float2 o = vx_rope_rot(a, b, cs[(size_t)rope_pos * half + i], sn[(size_t)rope_pos * half + i]);
        if (isq) *(float2 *)(q_out + (size_t)m * ldq + el) = o;
        else *(float2 *)(kc + (size_t)pos * kvd + el) = o;
    } else {
        const int el = r - (qd + kvd) / 2;
        vc[(size_t)pos * kvd + el] = vx_norm_bias((double)row[qd + kvd + el], 1.0f, bv, el);
    }
}

extern "C" int vxh_rope_kv_rows(const float *qkv, int ld_qkv, int M, int n_past, int n_ctx, int n_heads,
                                int n_kv_heads, int head_dim, const float *bq, const float *bk, const float *bv,
                                const float *cos_tab, const float *sin_tab, int n_pos, float *q_out, int ldq,
                                float *k_cache_layer, float *v_cache_layer, vxh_stream s)
{
    if (M < 1 || head_dim % 2 || ld_qkv % 2 || ldq % 2 || n_past < 0 || n_past + M - 1 >= n_pos ||
        ld_qkv < (n_heads + 2 * n_kv_heads) * head_dim || ldq < n_heads * head_dim)
        return vxh_fail(VXH_ERR_PARAM, "rope_kv_rows: M %d n_past %d n_pos %d", M, n_past, n_pos);
    const int qd = n_heads * head_dim, kvd = n_kv_heads * head_dim;
    const long n = (long)M * ((qd + kvd) / 2 + kvd);
    vx_pf_rope_kv_kernel<<<(unsigned)((n + 255) / 256), 256, 0, vxh_hs(s)>>>(
        qkv, ld_qkv, M, n_past, n_ctx, n_heads, n_kv_heads, head_dim, bq, bk, bv, cos_tab, sin_tab, q_out, ldq,
        k_cache_layer, v_cache_layer);
    VXH_LAUNCHED();
    return VXH_OK;
}

// ---------------------------------------------------------------------------
// SwiGLU with the FFN gate-skip (src/model.c:582-585) from the interleaved
// gate/up product (16 gate then 16 up columns per tile of 32): row m, column
// i reads gate at 32(i/16) + i%16 and up 16 further.
// ---------------------------------------------------------------------------
__global__ void vx_pf_swiglu_kernel(const float *__restrict__ gu, int ld_gu, int M, int F, float thr,
                                    float *__restrict__ h, int ldh)
{
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)M * F) return;
    const int m = (int)(idx / F), i = (int)(idx % F);
    const float *pg = gu + (size_t)m * ld_gu + 32 * (i / 16) + i % 16;
    const float g = vx_silu(pg[0]), u = pg[16];
    h[(size_t)m * ldh + i] = fabsf(g) < thr ? 0.0f : g * u;
}

extern "C" int vxh_swiglu_rows(const float *gu, int ld_gu, int M, int F, float thr, float *h, int ldh,
                               vxh_stream s)
{
    if (M < 1 || F < 1 || ldh < F || ld_gu < (F + 15) / 16 * 32)
        return vxh_fail(VXH_ERR_PARAM, "swiglu_rows: M %d F %d", M, F);
    const long n = (long)M * F;
    vx_pf_swiglu_kernel<<<(unsigned)((n + 255) / 256), 256, 0, vxh_hs(s)>>>(gu, ld_gu, M, F, thr, h, ldh);
    VXH_LAUNCHED();
    return VXH_OK;
}
