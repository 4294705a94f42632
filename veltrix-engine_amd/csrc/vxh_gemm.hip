// Skinny-M dequant GEMM for GGUF Q4_0 / Q8_0 weights on gfx950.
//
//   Y[m][n] = sum_k X[m][k] * W[n][k],  1 <= M <= 16
//
// MFMA path: v_mfma_f32_32x32x16_f16 with the activations as the A operand
// (32 columns: rows m as fp16 hi parts in columns 0..15, lo parts in 16..31)
// and 32 weight rows as the B operand.  Weights are exact small integers in
// fp16 (s-8 for Q4_0, q for Q8_0) unpacked in registers from the tiled
// nibble/byte plane; one Q4_0/Q8_0 block is exactly K=32 = two MFMAs, after
// which the 32x32 block product is scaled by the block's fp16 scale d and
// accumulated in fp32.  x = hi + lo carries 22 significant bits, so the
// products match fp32 arithmetic to ~1e-7 relative.
//
// Work split: a workgroup is 4 wavefronts = 4 tiles of 32 weight rows, all on
// the same K range (the activation panel slice for that range is staged in
// LDS once per workgroup); the K range is split across workgroups and the
// partial sums are reduced by the last workgroup to arrive (atomic counter),
// which also applies the epilogue.
#include "vxh_internal.h"

// ---------------------------------------------------------------------------
// panel prep
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
    if (max_M < 1 || max_M > 16 || K % 32)
        return vxh_fail(VXH_ERR_PARAM, "panel_alloc: M %d K %d", max_M, K);
    int rc = vxh_malloc(&p->data, vxh_panel_bytes(max_M, K));
    if (rc) return rc;
    int nb = (K / 32 + 1) / 2 * 2;
    rc = vxh_malloc((void **)&p->corr, (size_t)nb * max_M * sizeof(float));
    if (rc) return rc;
    rc = vxh_malloc((void **)&p->rscale, 16 * sizeof(float));
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

// Writes one 16-byte unit pair (hi, lo) of row m for elements
// 32b + 16h + 8s + 0..7, given their fp32 values v[8].
__device__ __forceinline__ void vx_panel_store(uint4 *__restrict__ panel, int M, int b, int s, int h,
                                               int m, const float v[8])
{
    vx_half8 hi, lo;
#pragma unroll
    for (int kk = 0; kk < 8; kk++) {
        _Float16 a = (_Float16)v[kk];
        hi[kk] = a;
        lo[kk] = (_Float16)(v[kk] - (float)a);
    }
    int NS = 2 * M;
    size_t base = ((size_t)(b * 2 + s) * 2 + h) * NS;
    panel[base + m] = __builtin_bit_cast(uint4, hi);
    panel[base + M + m] = __builtin_bit_cast(uint4, lo);
}

__device__ __forceinline__ float vx_block_max(float v, float *red);

// Power-of-two row scale: s = 2^-e with amax = f * 2^e, f in [0.5, 1), so
// that every scaled value has magnitude < 1 (fp16 hi/lo keep 22 bits).
__device__ __forceinline__ float vx_row_scale(float amax, float *rs_out)
{
    if (!(amax > 0.0f) || !isfinite(amax)) { *rs_out = 1.0f; return 1.0f; }
    int e;
    frexpf(amax, &e);
    *rs_out = ldexpf(1.0f, e);
    return ldexpf(1.0f, -e);
}

// One workgroup per row.  AVX2-lane weights: elements with t % 8 >= 4 count
// twice (kk >= 4 within a unit); the per-(block,row) correction is the sum of
// x at offsets 8..11, 16..19, 24..27, 32..35 (offsets >= K read the tail).
__global__ void vx_prep_panel_kernel(const float *__restrict__ x, int ldx, int M, int K, int avx2,
                                     const float *__restrict__ tail, int ld_tail,
                                     uint4 *__restrict__ panel, float *__restrict__ corr,
                                     float *__restrict__ rscale)
{
    __shared__ float red[16];
    const int m = blockIdx.x;
    const int nb = K / 32, nbp = (nb + 1) / 2 * 2;
    const float *xr = x + (size_t)m * ldx;
    float amax = 0.0f;
    for (int i = threadIdx.x; i < K; i += blockDim.x) amax = fmaxf(amax, fabsf(xr[i]));
    amax = vx_block_max(amax, red);
    float rs;
    const float sc = vx_row_scale(avx2 ? 2.0f * amax : amax, &rs);
    if (threadIdx.x == 0) rscale[m] = rs;
    for (int u = threadIdx.x; u < nbp * 4; u += blockDim.x) {
        const int b = u / 4, h = (u / 2) % 2, s = u % 2;
        const int t0 = 32 * b + 16 * h + 8 * s;
        float v[8];
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
            float xv = b < nb ? xr[t0 + kk] * sc : 0.0f;   // the padding block of an odd count is zero
            v[kk] = (avx2 && kk >= 4) ? 2.0f * xv : xv;
        }
        vx_panel_store(panel, M, b, s, h, m, v);
    }
    if (avx2) {
        for (int b = threadIdx.x; b < nbp; b += blockDim.x) {
            float c = 0.0f;
            if (b < nb)
                for (int g = 1; g <= 4; g++)
                    for (int q = 0; q < 4; q++) {
                        int t = 32 * b + 8 * g + q;
                        float xv = t < K ? xr[t] : (tail ? tail[(size_t)m * ld_tail + (t - K)] : 0.0f);
                        c += xv;
                    }
            corr[(size_t)b * M + m] = c * sc;
        }
    }
}

extern "C" int vxh_prep_panel(vxh_panel *p, const float *x, int ldx, int M, int K, int avx2,
                              const float *tail, int ld_tail, vxh_stream s)
{
    if (M < 1 || M > 16 || K != p->K || K % 32)
        return vxh_fail(VXH_ERR_PARAM, "prep_panel: M %d K %d (panel K %d)", M, K, p->K);
    p->M = M;
    p->avx2 = avx2;
    vx_prep_panel_kernel<<<M, 256, 0, vxh_hs(s)>>>(x, ldx, M, K, avx2, tail, ld_tail,
                                                  (uint4 *)p->data, p->corr, p->rscale);
    VXH_LAUNCHED();
    return VXH_OK;
}

// ---------------------------------------------------------------------------
// fused RMSNorm + panel (one workgroup per row)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float vx_block_sum(float v, float *red)
{
    // wave reduction then across the (up to 16) waves of the block
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) red[w] = v;
    __syncthreads();
    int nw = (blockDim.x + 63) >> 6;
    float t = 0.0f;
    if (threadIdx.x < 64) {
        t = threadIdx.x < nw ? red[threadIdx.x] : 0.0f;
        for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off, 64);
        if (threadIdx.x == 0) red[0] = t;
    }
    __syncthreads();
    float r = red[0];
    __syncthreads();
    return r;
}

__device__ __forceinline__ float vx_block_max(float v, float *red)
{
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) red[w] = v;
    __syncthreads();
    int nw = (blockDim.x + 63) >> 6;
    float r = red[0];
    for (int i = 1; i < nw; i++) r = fmaxf(r, red[i]);
    __syncthreads();
    return r;
}

// inv = 1/sqrt(ss/K + 1e-5) as in the reference (src/tensor.c:134-139);
// returns 0 when the rms is below 1e-10 (the reference then writes zeros).
__device__ __forceinline__ float vx_rms_inv(float ss, int K)
{
    float rms = sqrtf(ss / (float)K + 1e-5f);
    return rms < 1e-10f ? 0.0f : 1.0f / rms;
}

__global__ void vx_rmsnorm_panel_kernel(const float *__restrict__ x, int ldx, int M, int K,
                                        const float *__restrict__ w, int avx2,
                                        const float *__restrict__ tail, int ld_tail,
                                        uint4 *__restrict__ panel, float *__restrict__ corr,
                                        float *__restrict__ rscale, float *__restrict__ xn_out,
                                        int ld_xn)
{
    __shared__ float red[16];
    int m = blockIdx.x;
    const float *xr = x + (size_t)m * ldx;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < K; i += blockDim.x) ss += xr[i] * xr[i];
    ss = vx_block_sum(ss, red);
    float inv = vx_rms_inv(ss, K);
    float amax = 0.0f;
    for (int i = threadIdx.x; i < K; i += blockDim.x) amax = fmaxf(amax, fabsf((w ? w[i] : 1.0f) * (xr[i] * inv)));
    amax = vx_block_max(amax, red);
    float rs;
    const float sc = vx_row_scale(avx2 ? 2.0f * amax : amax, &rs);
    if (threadIdx.x == 0) rscale[m] = rs;
    int nb = K / 32, nbp = (nb + 1) / 2 * 2;
    // units (b, h, s): 8 elements each; the padding block of an odd count is zero
    for (int u = threadIdx.x; u < nbp * 4; u += blockDim.x) {
        int b = u / 4, h = (u / 2) % 2, s = u % 2;
        int t0 = 32 * b + 16 * h + 8 * s;
        float v[8];
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
            float xv = 0.0f;
            if (b < nb) {
                float wv = w ? w[t0 + kk] : 1.0f;
                xv = wv * (xr[t0 + kk] * inv);
                if (xn_out) xn_out[(size_t)m * ld_xn + t0 + kk] = xv;
                xv *= sc;
            }
            v[kk] = (avx2 && kk >= 4) ? 2.0f * xv : xv;
        }
        vx_panel_store(panel, M, b, s, h, m, v);
    }
    if (avx2) {
        // corrections need normalised values of the next block and, for the
        // last block, the caller's tail values (src/model.c:425-435)
        for (int b = threadIdx.x; b < nbp; b += blockDim.x) {
            float c = 0.0f;
            if (b < nb)
            for (int g = 1; g <= 4; g++)
                for (int q = 0; q < 4; q++) {
                    int t = 32 * b + 8 * g + q;
                    float xv = t < K ? (w ? w[t] : 1.0f) * (xr[t] * inv)
                                     : (tail ? tail[(size_t)m * ld_tail + (t - K)] : 0.0f);
                    c += xv;
                }
            corr[(size_t)b * M + m] = c * sc;
        }
    }
}

extern "C" int vxh_rmsnorm_panel(const float *x, int ldx, int M, int K, const float *w, int avx2,
                                 const float *tail, int ld_tail, vxh_panel *p, float *xn_out,
                                 int ld_xn, vxh_stream s)
{
    if (M < 1 || M > 16 || K != p->K || K % 32)
        return vxh_fail(VXH_ERR_PARAM, "rmsnorm_panel: M %d K %d (panel K %d)", M, K, p->K);
    p->M = M;
    p->avx2 = avx2;
    vx_rmsnorm_panel_kernel<<<M, 256, 0, vxh_hs(s)>>>(x, ldx, M, K, w, avx2, tail, ld_tail,
                                                     (uint4 *)p->data, p->corr, p->rscale, xn_out,
                                                     ld_xn);
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
// MFMA GEMM
// ---------------------------------------------------------------------------
struct vx_epi {
    const float *rscale;
    int kind;
    float *y;
    int ldy;
    const float *r;
    int ldr;
    float thr;
    float scale;
    int n_out;
};

// Q4_0 dword (8 nibbles in the repacked slot order) -> 8 fp16 values s - 8.
__device__ __forceinline__ vx_half8 vx_unpack_q4(uint32_t q)
{
    const uint32_t lo = 0x000F000Fu, hi = 0x00F000F0u, magic = 0x64006400u;
    uint32_t q8 = q >> 8;
    vx_half2 a = __builtin_bit_cast(vx_half2, (q & lo) | magic);
    vx_half2 b = __builtin_bit_cast(vx_half2, (q & hi) | magic);
    vx_half2 c = __builtin_bit_cast(vx_half2, (q8 & lo) | magic);
    vx_half2 d = __builtin_bit_cast(vx_half2, (q8 & hi) | magic);
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

// Two Q8_0 dwords (4 int8 each, bytes in the repacked order) -> 8 fp16.
__device__ __forceinline__ vx_half8 vx_unpack_q8(uint32_t qa, uint32_t qb)
{
    const uint32_t m = 0x00FF00FFu, magic = 0x64006400u;
    uint32_t ua = qa ^ 0x80808080u, ub = qb ^ 0x80808080u;
    vx_half2 a0 = __builtin_bit_cast(vx_half2, (ua & m) | magic);
    vx_half2 a1 = __builtin_bit_cast(vx_half2, ((ua >> 8) & m) | magic);
    vx_half2 b0 = __builtin_bit_cast(vx_half2, (ub & m) | magic);
    vx_half2 b1 = __builtin_bit_cast(vx_half2, ((ub >> 8) & m) | magic);
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

__device__ __forceinline__ float vx_silu(float g) { return g / (1.0f + expf(-g)); }

__device__ __forceinline__ void vx_store_epi(const vx_epi &ep, int m, int n, float v)
{
    if (n >= ep.n_out) return;
    float y = v * ep.rscale[m] * ep.scale;
    if (ep.kind == VXH_EPI_RESID) y = ep.r[(size_t)m * ep.ldr + n] + y;
    else if (ep.kind == VXH_EPI_GATE) y = fabsf(ep.r[(size_t)m * ep.ldr + n]) < ep.thr ? 0.0f : y;
    ep.y[(size_t)m * ep.ldy + n] = y;
}

// QT: 2 = Q4_0, 8 = Q8_0.  PF: weight loads kept in flight per wave.
template <int QT, int M, bool AVX2, int PF>
__global__ __launch_bounds__(256) void vx_gemm_mfma_kernel(
    const uint4 *__restrict__ wq, const uint32_t *__restrict__ wd, const uint4 *__restrict__ panel,
    const float *__restrict__ corr, int n_tiles, int n_pairs, int pps, int n_splits,
    float *__restrict__ part, unsigned *__restrict__ counters, vx_epi ep)
{
    constexpr int NS = vx_mcfg<M>::NS;
    constexpr int R1 = vx_mcfg<M>::R1;
    constexpr int WPP = QT == 2 ? 1 : 2;   // 16-byte weight loads per lane per block pair
    extern __shared__ uint4 lds[];
    __shared__ int s_last;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = blockIdx.x / n_splits, split = blockIdx.x % n_splits;
    const int T = grp * 4 + wave;
    const bool tile_ok = T < n_tiles;
    const int p0 = split * pps;
    const int p1 = min(p0 + pps, n_pairs);
    const int np = p1 - p0;
    const int c = lane & 31, h = lane >> 5;

    // ---- weight stream prefetch (issued before the LDS staging) ----
    const uint4 *wp = wq + ((size_t)(tile_ok ? T : 0) * n_pairs * WPP + (size_t)p0 * WPP) * 64 + lane;
    const uint32_t *sp = wd + ((size_t)(tile_ok ? T : 0) * n_pairs + p0) * 32 + c;
    uint4 wbuf[PF][WPP];
    uint32_t sbuf[PF];
#pragma unroll
    for (int i = 0; i < PF; i++) {
        if (tile_ok && i < np) {
#pragma unroll
            for (int q = 0; q < WPP; q++) wbuf[i][q] = wp[((size_t)i * WPP + q) * 64];
            sbuf[i] = sp[(size_t)i * 32];
        }
    }

    // ---- stage the panel slice (and corrections) for blocks [2p0, 2p1) ----
    const int units = np * 2 * 4 * NS;
    const uint4 *psrc = panel + (size_t)p0 * 2 * 4 * NS;
    for (int i = threadIdx.x; i < units; i += 256) lds[i] = psrc[i];
    float *lcorr = (float *)(lds + units);
    if (AVX2) {
        const float *csrc = corr + (size_t)p0 * 2 * M;
        for (int i = threadIdx.x; i < np * 2 * M; i += 256) lcorr[i] = csrc[i];
    }
    __syncthreads();

    const bool a_ok = c < 16 ? (c < M) : (c - 16 < M);
    const int slot = c < 16 ? c : M + (c - 16);
    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    const vx_f32x16 zero16 = {};
    const vx_half8 zero8 = {};

    if (tile_ok) {
        for (int pb = 0; pb < np; pb += PF) {
#pragma unroll
            for (int i = 0; i < PF; i++) {
                const int pl = pb + i;
                if (pl < np) {
                    uint4 w[WPP];
#pragma unroll
                    for (int q = 0; q < WPP; q++) w[q] = wbuf[i][q];
                    const uint32_t sc = sbuf[i];
                    if (pl + PF < np) {
#pragma unroll
                        for (int q = 0; q < WPP; q++) wbuf[i][q] = wp[((size_t)(pl + PF) * WPP + q) * 64];
                        sbuf[i] = sp[(size_t)(pl + PF) * 32];
                    }
#pragma unroll
                    for (int blk = 0; blk < 2; blk++) {
                        const int bl = 2 * pl + blk;
                        vx_half8 b0, b1;
                        if (QT == 2) {
                            b0 = vx_unpack_q4(blk ? w[0].z : w[0].x);
                            b1 = vx_unpack_q4(blk ? w[0].w : w[0].y);
                        } else {
                            b0 = vx_unpack_q8(w[blk].x, w[blk].y);
                            b1 = vx_unpack_q8(w[blk].z, w[blk].w);
                        }
                        vx_half8 a0 = zero8, a1 = zero8;
                        if (a_ok) {
                            a0 = __builtin_bit_cast(vx_half8, lds[((bl * 2 + 0) * 2 + h) * NS + slot]);
                            a1 = __builtin_bit_cast(vx_half8, lds[((bl * 2 + 1) * 2 + h) * NS + slot]);
                        }
                        vx_f32x16 D = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, zero16, 0, 0, 0);
                        D = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, D, 0, 0, 0);
                        const float d = vx_half_bits_to_float((sc >> (16 * blk)) & 0xFFFFu);
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
            }
        }
    }

    // ---- partial sums: hi + lo per (m, n) ----
    const int n_phys = n_tiles * 32;
    if (tile_ok) {
#pragma unroll
        for (int r = 0; r < R1; r++) {
            const int m = 8 * (r / 4) + 4 * h + (r % 4);
            if (m < M) part[((size_t)split * M + m) * n_phys + T * 32 + c] = acc[r] + acc[r + 8];
        }
    }

    // ---- last workgroup of this tile group reduces and applies the epilogue ----
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned prev = __hip_atomic_fetch_add(&counters[grp], 1u, __ATOMIC_ACQ_REL,
                                               __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == (unsigned)(n_splits - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const int n0 = grp * 128;
    if (ep.kind == VXH_EPI_SWIGLU) {
        // tile t holds gate rows 16t..16t+15 (j < 16) and up rows (j >= 16)
        for (int i = threadIdx.x; i < M * 64; i += 256) {
            const int m = i / 64, jj = i % 64, tl = jj / 16, j = jj % 16;
            const int tg = grp * 4 + tl;
            if (tg >= n_tiles) continue;
            float g = 0.0f, u = 0.0f;
            for (int sp2 = 0; sp2 < n_splits; sp2++) {
                const float *pr = part + ((size_t)sp2 * M + m) * n_phys + tg * 32;
                g += pr[j];
                u += pr[16 + j];
            }
            g *= ep.rscale[m] * ep.scale;
            u *= ep.rscale[m] * ep.scale;
            const int n = tg * 16 + j;
            if (n < ep.n_out) {
                const float sg = vx_silu(g);
                ep.y[(size_t)m * ep.ldy + n] = fabsf(sg) < ep.thr ? 0.0f : sg * u;
            }
        }
    } else {
        for (int i = threadIdx.x; i < M * 128; i += 256) {
            const int m = i / 128, n = n0 + i % 128;
            if (n >= n_phys) continue;
            float v = 0.0f;
            for (int sp2 = 0; sp2 < n_splits; sp2++) v += part[((size_t)sp2 * M + m) * n_phys + n];
            vx_store_epi(ep, m, n, v);
        }
    }
    if (threadIdx.x == 0) counters[grp] = 0u;
}

// Splits the K range so that the launch has enough workgroups to cover the
// 256 CUs while the LDS slice stays <= 40 KiB.
static void vx_gemm_plan(int n_tiles, int n_pairs, int M, int *pps, int *n_splits)
{
    int groups = (n_tiles + 3) / 4;
    int per_pair_lds = 128 * 2 * M + 8 * M;          // panel units + corrections
    int max_pps = 40960 / per_pair_lds;
    if (max_pps < 1) max_pps = 1;
    int want_splits = (1024 + groups - 1) / groups;
    int p = (n_pairs + want_splits - 1) / want_splits;
    if (p < 4) p = 4;
    if (p > max_pps) p = max_pps;
    if (p > n_pairs) p = n_pairs;
    *pps = p;
    *n_splits = (n_pairs + p - 1) / p;
}

extern "C" size_t vxh_gemm_workspace_floats(int n_rows, int n_cols, int M)
{
    int n_tiles = (n_rows + 31) / 32, n_pairs = (n_cols / 32 + 1) / 2, pps, ns;
    vx_gemm_plan(n_tiles, n_pairs, M, &pps, &ns);
    return (size_t)ns * M * n_tiles * 32;
}

extern "C" int vxh_gemm_workspace_counters(int n_rows) { return ((n_rows + 31) / 32 + 3) / 4; }

template <int QT, int M, bool AVX2>
static int vx_launch_mfma(const vxh_qmat *W, const vxh_panel *X, const vx_epi &ep,
                          vxh_workspace *ws, hipStream_t st)
{
    int n_tiles = W->n_rows / 32;
    int pps, n_splits;
    vx_gemm_plan(n_tiles, W->n_pairs, M, &pps, &n_splits);
    int groups = (n_tiles + 3) / 4;
    size_t need = (size_t)n_splits * M * W->n_rows;
    if (need > ws->part_floats || groups > ws->n_counters)
        return vxh_fail(VXH_ERR_PARAM, "gemm workspace too small: need %zu floats / %d counters",
                        need, groups);
    size_t lds = (size_t)pps * 2 * 4 * 2 * M * 16 + (AVX2 ? (size_t)pps * 2 * M * 4 : 0);
    vx_gemm_mfma_kernel<QT, M, AVX2, 4><<<groups * n_splits, 256, lds, st>>>(
        (const uint4 *)W->qs, (const uint32_t *)W->d, (const uint4 *)X->data, X->corr, n_tiles,
        W->n_pairs, pps, n_splits, ws->part, ws->counters, ep);
    VXH_LAUNCHED();
    return VXH_OK;
}

template <int M>
static int vx_dispatch_m(const vxh_qmat *W, const vxh_panel *X, const vx_epi &ep,
                         vxh_workspace *ws, hipStream_t st)
{
    if (W->type == 2) {
        if (X->avx2) return vx_launch_mfma<2, M, true>(W, X, ep, ws, st);
        return vx_launch_mfma<2, M, false>(W, X, ep, ws, st);
    }
    if (X->avx2) return vxh_fail(VXH_ERR_UNSUPPORTED, "AVX2-lane panels apply to Q4_0 only");
    return vx_launch_mfma<8, M, false>(W, X, ep, ws, st);
}

extern "C" int vxh_gemm(const vxh_qmat *W, const vxh_panel *X, int M, const vxh_epilogue *e,
                        vxh_workspace *ws, int path, vxh_stream s)
{
    if (M != X->M || M < 1 || M > 16)
        return vxh_fail(VXH_ERR_PARAM, "gemm: M %d (panel M %d)", M, X->M);
    if (W->n_cols != X->K)
        return vxh_fail(VXH_ERR_PARAM, "gemm: W has K %d, panel %d", W->n_cols, X->K);
    if (path == VXH_PATH_DOT)
        return vxh_fail(VXH_ERR_UNSUPPORTED, "dot-product path not built for this shape");
    vx_epi ep{X->rscale, e->kind, e->y, e->ldy, e->r, e->ldr, e->thr, e->scale, e->n_out};
    hipStream_t st = vxh_hs(s);
    switch (M) {
    case 1: return vx_dispatch_m<1>(W, X, ep, ws, st);
    case 2: return vx_dispatch_m<2>(W, X, ep, ws, st);
    case 3: return vx_dispatch_m<3>(W, X, ep, ws, st);
    case 4: return vx_dispatch_m<4>(W, X, ep, ws, st);
    case 5: return vx_dispatch_m<5>(W, X, ep, ws, st);
    case 6: return vx_dispatch_m<6>(W, X, ep, ws, st);
    case 7: return vx_dispatch_m<7>(W, X, ep, ws, st);
    case 8: return vx_dispatch_m<8>(W, X, ep, ws, st);
    case 9: return vx_dispatch_m<9>(W, X, ep, ws, st);
    case 10: return vx_dispatch_m<10>(W, X, ep, ws, st);
    case 11: return vx_dispatch_m<11>(W, X, ep, ws, st);
    case 12: return vx_dispatch_m<12>(W, X, ep, ws, st);
    case 13: return vx_dispatch_m<13>(W, X, ep, ws, st);
    case 14: return vx_dispatch_m<14>(W, X, ep, ws, st);
    case 15: return vx_dispatch_m<15>(W, X, ep, ws, st);
    default: return vx_dispatch_m<16>(W, X, ep, ws, st);
    }
}
