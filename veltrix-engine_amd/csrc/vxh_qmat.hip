// Quantised matrices in HBM: allocation, GGUF <-> tiled repack, seeded
// synthetic weights and row gathers (include/vxh.h, "quantised matrices").
#include "vxh_internal.h"

#include <string.h>

// Q4_0: element e (0..7) of a dword is stored in nibble slot kSlot4[e], so that
// the unpack in the GEMM ((q & 0x000F000F), (q & 0x00F000F0), and the same of
// q >> 8) produces fp16 pairs (e0,e1), (e2,e3), (e4,e5), (e6,e7).
__constant__ int kSlot4[8] = {0, 4, 1, 5, 2, 6, 3, 7};
// Q8_0: element e (0..3) of a dword sits in byte kPos8[e]; the unpack
// ((u & 0x00FF00FF), (u >> 8) & 0x00FF00FF) then yields (e0,e1), (e2,e3).
__constant__ int kPos8[4] = {0, 2, 1, 3};

__host__ __device__ static inline int vx_block_bytes(int type) { return type == 2 ? 18 : 34; }

extern "C" int vxh_qmat_alloc(vxh_qmat *m, int type, int n_rows, int n_cols)
{
    memset(m, 0, sizeof(*m));
    if ((type != 0 && type != 2 && type != 8) || n_rows <= 0 || n_cols <= 0 || n_cols % 32)
        return vxh_fail(VXH_ERR_PARAM, "qmat_alloc: type %d rows %d cols %d", type, n_rows, n_cols);
    m->type = type;
    m->n_rows = (n_rows + 31) / 32 * 32;
    m->n_cols = n_cols;
    m->n_pairs = (n_cols / 32 + 1) / 2;
    if (type == 0) {
        // F32: plain rows of n_pairs * 64 floats, zero past n_cols and past
        // the logical rows
        size_t bytes = (size_t)m->n_rows * m->n_pairs * 64 * sizeof(float);
        int rc = vxh_malloc(&m->qs, bytes);
        if (rc) return rc;
        VXH_CHECK(hipMemset(m->qs, 0, bytes));
        VXH_CHECK(hipDeviceSynchronize());
        return VXH_OK;
    }
    size_t tiles = (size_t)m->n_rows / 32;
    size_t qs_bytes = tiles * m->n_pairs * (type == 2 ? 1024u : 2048u);
    size_t d_bytes = tiles * m->n_pairs * 32u * 4u;
    // the 64-row tiled copy (GEMMs of 5..16 rows); its buffer loads take
    // 32-bit offsets
    const size_t t64 = ((size_t)m->n_rows + 63) / 64, nb = (size_t)n_cols / 32;
    size_t tq_bytes = t64 * nb * (type == 2 ? 1024u : 2048u);
    size_t td_bytes = t64 * nb * 128u;
    if (tq_bytes > 0xFFFFFFFFull)
        return vxh_fail(VXH_ERR_UNSUPPORTED, "qmat_alloc: %d x %d matrix exceeds 4 GiB", n_rows, n_cols);
    int rc = vxh_malloc(&m->qs, qs_bytes);
    if (rc == VXH_OK) rc = vxh_malloc(&m->d, d_bytes);
    if (rc == VXH_OK) rc = vxh_malloc(&m->tq, tq_bytes);
    if (rc == VXH_OK) rc = vxh_malloc(&m->td, td_bytes);
    if (rc) {
        vxh_free(m->qs); vxh_free(m->d); vxh_free(m->tq); vxh_free(m->td);
        memset(m, 0, sizeof(*m));
        return rc;
    }
    // padding rows/blocks must read as d = 0
    VXH_CHECK(hipMemset(m->d, 0, d_bytes));
    VXH_CHECK(hipMemset(m->qs, 0, qs_bytes));
    VXH_CHECK(hipMemset(m->td, 0, td_bytes));
    VXH_CHECK(hipMemset(m->tq, 0, tq_bytes));
    VXH_CHECK(hipDeviceSynchronize());
    return VXH_OK;
}

extern "C" int vxh_qmat_free(vxh_qmat *m)
{
    vxh_free(m->qs);
    vxh_free(m->d);
    vxh_free(m->tq);
    vxh_free(m->td);
    memset(m, 0, sizeof(*m));
    return VXH_OK;
}

__device__ __forceinline__ int vx_phys_row(int r, int group, int group_stride, int row_offset)
{
    return (r / group) * group_stride + row_offset + r % group;
}

__device__ __forceinline__ uint32_t vx_permute_q4_dword(uint32_t q)
{
    uint32_t o = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) o |= ((q >> (4 * e)) & 15u) << (4 * kSlot4[e]);
    return o;
}

__device__ __forceinline__ uint32_t vx_unpermute_q4_dword(uint32_t o)
{
    uint32_t q = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) q |= ((o >> (4 * kSlot4[e])) & 15u) << (4 * e);
    return q;
}

__device__ __forceinline__ uint32_t vx_permute_q8_dword(uint32_t q)
{
    uint32_t o = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) o |= ((q >> (8 * e)) & 255u) << (8 * kPos8[e]);
    return o;
}

__device__ __forceinline__ uint32_t vx_unpermute_q8_dword(uint32_t o)
{
    uint32_t q = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) q |= ((o >> (8 * kPos8[e])) & 255u) << (8 * e);
    return q;
}

// Reads 4 bytes at an address that is only 2-byte aligned.
__device__ __forceinline__ uint32_t vx_ld32_a2(const uint8_t *p)
{
    const uint16_t *h = (const uint16_t *)p;
    return (uint32_t)h[0] | ((uint32_t)h[1] << 16);
}

__device__ __forceinline__ void vx_st32_a2(uint8_t *p, uint32_t v)
{
    uint16_t *h = (uint16_t *)p;
    h[0] = (uint16_t)v;
    h[1] = (uint16_t)(v >> 16);
}

// One thread per (logical row, block pair).
__global__ void vx_repack_kernel(const uint8_t *__restrict__ src, int type, int n_rows, int nb,
                                 int n_pairs, int group, int group_stride, int row_offset,
                                 uint32_t *__restrict__ qs, uint32_t *__restrict__ dpl)
{
    long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)n_rows * n_pairs) return;
    int r = (int)(idx / n_pairs), p = (int)(idx % n_pairs);
    int pr = vx_phys_row(r, group, group_stride, row_offset);
    int T = pr / 32, j = pr % 32;
    int bb = vx_block_bytes(type);
    uint32_t dd = 0;
    for (int blk = 0; blk < 2; blk++) {
        int b = 2 * p + blk;
        const uint8_t *blkp = b < nb ? src + ((size_t)r * nb + b) * bb : nullptr;
        uint32_t dh = blkp ? ((const uint16_t *)blkp)[0] : 0u;
        dd |= dh << (16 * blk);
        for (int h = 0; h < 2; h++) {
            if (type == 2) {
                // lane chunk (T, p, j + 32h): [blk0 dw 2h, 2h+1][blk1 dw 2h, 2h+1]
                uint32_t *dst = qs + (((size_t)T * n_pairs + p) * 64 + j + 32 * h) * 4 + blk * 2;
                for (int w = 0; w < 2; w++) {
                    uint32_t q = blkp ? vx_ld32_a2(blkp + 2 + 4 * (2 * h + w)) : 0x88888888u;
                    dst[w] = vx_permute_q4_dword(q);
                }
            } else {
                // lane chunk (T, b, j + 32h): bytes 16h..16h+15 of block b
                uint32_t *dst = qs + (((size_t)T * n_pairs * 2 + b) * 64 + j + 32 * h) * 4;
                for (int w = 0; w < 4; w++) {
                    uint32_t q = blkp ? vx_ld32_a2(blkp + 2 + 16 * h + 4 * w) : 0u;
                    dst[w] = vx_permute_q8_dword(q);
                }
            }
        }
    }
    dpl[((size_t)T * n_pairs + p) * 32 + j] = dd;
}

// The 64-row tiled copy: one thread per (logical row, block).
__global__ void vx_repack_t64_kernel(const uint8_t *__restrict__ src, int type, int n_rows, int nb, int group,
                                     int group_stride, int row_offset, uint32_t *__restrict__ tq,
                                     uint16_t *__restrict__ td)
{
    long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)n_rows * nb) return;
    const int r = (int)(idx / nb), b = (int)(idx % nb);
    const int pr = vx_phys_row(r, group, group_stride, row_offset);
    const int T = pr / 64, g = (pr % 64) / 16, n = pr % 16;
    const uint8_t *blkp = src + ((size_t)r * nb + b) * vx_block_bytes(type);
    const size_t tb = (size_t)T * nb + b;
    td[(tb * 16 + n) * 4 + g] = ((const uint16_t *)blkp)[0];
    for (int G = 0; G < 4; G++) {
        if (type == 2) {
            tq[(tb * 64 + G * 16 + n) * 4 + g] = vx_permute_q4_dword(vx_ld32_a2(blkp + 2 + 4 * G));
        } else {
            uint32_t *dst = tq + ((tb * 2 + (g >> 1)) * 64 + G * 16 + n) * 4 + (g & 1) * 2;
            dst[0] = vx_permute_q8_dword(vx_ld32_a2(blkp + 2 + 8 * G));
            dst[1] = vx_permute_q8_dword(vx_ld32_a2(blkp + 2 + 8 * G + 4));
        }
    }
}

__global__ void vx_unrepack_kernel(uint8_t *__restrict__ dstb, int type, int n_rows, int nb,
                                   int n_pairs, int group, int group_stride, int row_offset,
                                   const uint32_t *__restrict__ qs,
                                   const uint32_t *__restrict__ dpl)
{
    long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)n_rows * n_pairs) return;
    int r = (int)(idx / n_pairs), p = (int)(idx % n_pairs);
    int pr = vx_phys_row(r, group, group_stride, row_offset);
    int T = pr / 32, j = pr % 32;
    int bb = vx_block_bytes(type);
    uint32_t dd = dpl[((size_t)T * n_pairs + p) * 32 + j];
    for (int blk = 0; blk < 2; blk++) {
        int b = 2 * p + blk;
        if (b >= nb) break;
        uint8_t *blkp = dstb + ((size_t)r * nb + b) * bb;
        ((uint16_t *)blkp)[0] = (uint16_t)(dd >> (16 * blk));
        for (int h = 0; h < 2; h++) {
            if (type == 2) {
                const uint32_t *s = qs + (((size_t)T * n_pairs + p) * 64 + j + 32 * h) * 4 + blk * 2;
                for (int w = 0; w < 2; w++) vx_st32_a2(blkp + 2 + 4 * (2 * h + w), vx_unpermute_q4_dword(s[w]));
            } else {
                const uint32_t *s = qs + (((size_t)T * n_pairs * 2 + b) * 64 + j + 32 * h) * 4;
                for (int w = 0; w < 4; w++) vx_st32_a2(blkp + 2 + 16 * h + 4 * w, vx_unpermute_q8_dword(s[w]));
            }
        }
    }
}

// F32 rows: src[r][0..n_cols) <-> the matrix's physical row of r (row stride
// ld floats).  One thread per float4.
__global__ void vx_f32_rows_kernel(const float *__restrict__ src, float *__restrict__ dst, int n_rows,
                                   int n_cols, int ld, int group, int group_stride, int row_offset, int to_matrix)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int c4 = n_cols / 4;
    if (i >= (long)n_rows * c4) return;
    const int r = (int)(i / c4), k = (int)(i % c4) * 4;
    const size_t pm = (size_t)vx_phys_row(r, group, group_stride, row_offset) * ld + k;
    const size_t pr = (size_t)r * n_cols + k;
    if (to_matrix) *(float4 *)(dst + pm) = *(const float4 *)(src + pr);
    else *(float4 *)(dst + pr) = *(const float4 *)(src + pm);
}

static int check_map(const vxh_qmat *m, int n_rows, int group, int group_stride, int row_offset)
{
    if (n_rows <= 0 || group <= 0) return vxh_fail(VXH_ERR_PARAM, "qmat rows: n_rows %d group %d", n_rows, group);
    long last = (long)((n_rows - 1) / group) * group_stride + row_offset + (n_rows - 1 < group ? n_rows - 1 : group - 1);
    if (row_offset < 0 || last >= m->n_rows)
        return vxh_fail(VXH_ERR_PARAM, "qmat rows map past the matrix (%ld >= %d)", last, m->n_rows);
    return VXH_OK;
}

extern "C" int vxh_qmat_set_rows(vxh_qmat *m, const void *src, int src_on_device, int n_rows,
                                 int group, int group_stride, int row_offset, vxh_stream s)
{
    int rc = check_map(m, n_rows, group, group_stride, row_offset);
    if (rc) return rc;
    int nb = m->n_cols / 32;
    size_t bytes = m->type == 0 ? (size_t)n_rows * m->n_cols * sizeof(float)
                                : (size_t)n_rows * nb * vx_block_bytes(m->type);
    const void *dsrc = src;
    void *stage = nullptr;
    if (!src_on_device) {
        rc = vxh_malloc(&stage, bytes);
        if (rc) return rc;
        VXH_CHECK(hipMemcpyAsync(stage, src, bytes, hipMemcpyHostToDevice, vxh_hs(s)));
        dsrc = stage;
    }
    if (m->type == 0) {
        long n = (long)n_rows * (m->n_cols / 4);
        vx_f32_rows_kernel<<<(unsigned)((n + 255) / 256), 256, 0, vxh_hs(s)>>>(
            (const float *)dsrc, (float *)m->qs, n_rows, m->n_cols, m->n_pairs * 64, group, group_stride,
            row_offset, 1);
    } else {
        long n = (long)n_rows * m->n_pairs;
        vx_repack_kernel<<<(unsigned)((n + 255) / 256), 256, 0, vxh_hs(s)>>>(
            (const uint8_t *)dsrc, m->type, n_rows, nb, m->n_pairs, group, group_stride, row_offset,
            (uint32_t *)m->qs, (uint32_t *)m->d);
        VXH_LAUNCHED();
        if (m->tq) {
            const long nt = (long)n_rows * nb;
            vx_repack_t64_kernel<<<(unsigned)((nt + 255) / 256), 256, 0, vxh_hs(s)>>>(
                (const uint8_t *)dsrc, m->type, n_rows, nb, group, group_stride, row_offset, (uint32_t *)m->tq,
                (uint16_t *)m->td);
        }
    }
    VXH_LAUNCHED();
    if (stage) {
        VXH_CHECK(hipStreamSynchronize(vxh_hs(s)));
        vxh_free(stage);
    }
    return VXH_OK;
}

extern "C" int vxh_qmat_get_rows(const vxh_qmat *m, void *host_dst, int n_rows, int group,
                                 int group_stride, int row_offset, vxh_stream s)
{
    int rc = check_map(m, n_rows, group, group_stride, row_offset);
    if (rc) return rc;
    int nb = m->n_cols / 32;
    size_t bytes = m->type == 0 ? (size_t)n_rows * m->n_cols * sizeof(float)
                                : (size_t)n_rows * nb * vx_block_bytes(m->type);
    void *stage = nullptr;
    rc = vxh_malloc(&stage, bytes);
    if (rc) return rc;
    if (m->type == 0) {
        long n = (long)n_rows * (m->n_cols / 4);
        vx_f32_rows_kernel<<<(unsigned)((n + 255) / 256), 256, 0, vxh_hs(s)>>>(
            (const float *)m->qs, (float *)stage, n_rows, m->n_cols, m->n_pairs * 64, group, group_stride,
            row_offset, 0);
    } else {
        long n = (long)n_rows * m->n_pairs;
        vx_unrepack_kernel<<<(unsigned)((n + 255) / 256), 256, 0, vxh_hs(s)>>>(
            (uint8_t *)stage, m->type, n_rows, nb, m->n_pairs, group, group_stride, row_offset,
            (const uint32_t *)m->qs, (const uint32_t *)m->d);
    }
    VXH_LAUNCHED();
    VXH_CHECK(hipMemcpyAsync(host_dst, stage, bytes, hipMemcpyDeviceToHost, vxh_hs(s)));
    VXH_CHECK(hipStreamSynchronize(vxh_hs(s)));
    vxh_free(stage);
    return VXH_OK;
}

// ---------------------------------------------------------------------------
// Synthetic weights
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t vx_splitmix64(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Truncating fp32 -> fp16 bits with flush-to-zero (the Q4_0 writer's
// conversion, src/quantize.c:17-35).
__device__ __forceinline__ uint16_t vx_f32_to_f16_trunc(float f)
{
    uint32_t b = __float_as_uint(f);
    uint32_t sign = (b >> 31) << 15;
    int e = (int)((b >> 23) & 255u);
    uint32_t m = b & 0x7FFFFFu;
    if (e == 0) return (uint16_t)sign;
    if (e == 255) return (uint16_t)(sign | 0x7C00u | (m >> 13));
    int he = e - 112;
    if (he <= 0) return (uint16_t)sign;
    if (he >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)he << 10) | (m >> 13));
}

// One thread per block of 32 weights.
__global__ void vx_synth_kernel(uint8_t *__restrict__ dst, int type, long n_blocks, uint64_t seed,
                                float std)
{
    long bi = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (bi >= n_blocks) return;
    float x[32];
    float amax = 0.0f;
#pragma unroll
    for (int t = 0; t < 32; t++) {
        uint64_t r = vx_splitmix64(seed ^ ((uint64_t)(bi * 32 + t) * 0xD1B54A32D192ED03ull));
        float u1 = ((float)(uint32_t)(r >> 40) + 1.0f) * (1.0f / 16777216.0f);   // (0, 1]
        float u2 = (float)(uint32_t)((r >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
        float z = sqrtf(-2.0f * logf(u1)) * cosf(6.2831853071795864f * u2);
        x[t] = z * std;
        amax = fmaxf(amax, fabsf(x[t]));
    }
    if (type == 2) {
        uint8_t *b = dst + bi * 18;
        float d = amax / 7.0f;
        if (d < 1e-10f) d = 1e-10f;
        ((uint16_t *)b)[0] = vx_f32_to_f16_trunc(d);
        float inv = 1.0f / d;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            int a0 = (int)(x[2 * j] * inv), a1 = (int)(x[2 * j + 1] * inv);
            a0 = a0 < -8 ? -8 : (a0 > 7 ? 7 : a0);
            a1 = a1 < -8 ? -8 : (a1 > 7 ? 7 : a1);
            b[2 + j] = (uint8_t)((a0 + 8) | ((a1 + 8) << 4));
        }
    } else {
        uint8_t *b = dst + bi * 34;
        _Float16 dh = (_Float16)(amax / 127.0f);
        float d = (float)dh;
        ((uint16_t *)b)[0] = __builtin_bit_cast(uint16_t, dh);
        float inv = d > 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
        for (int t = 0; t < 32; t++) {
            float v = x[t] * inv;
            float q = copysignf(floorf(fabsf(v) + 0.5f), v);
            q = fminf(127.0f, fmaxf(-127.0f, q));
            ((int8_t *)b)[2 + t] = (int8_t)(int)q;
        }
    }
}

extern "C" int vxh_synth_blocks(void *dev_blocks, int type, int n_rows, int n_cols, uint64_t seed,
                                float std, vxh_stream s)
{
    if ((type != 2 && type != 8) || n_cols % 32)
        return vxh_fail(VXH_ERR_PARAM, "synth: type %d cols %d", type, n_cols);
    long nbk = (long)n_rows * (n_cols / 32);
    vx_synth_kernel<<<(unsigned)((nbk + 127) / 128), 128, 0, vxh_hs(s)>>>((uint8_t *)dev_blocks, type,
                                                                        nbk, seed, std);
    VXH_LAUNCHED();
    return VXH_OK;
}

// ---------------------------------------------------------------------------
// Row gather (embedding lookup)
// ---------------------------------------------------------------------------
__global__ void vx_gather_kernel(const uint32_t *__restrict__ qs, const uint32_t *__restrict__ dpl,
                                 int type, int n_rows_logical, int n_cols, int n_pairs,
                                 const int *__restrict__ ids, float scale, float *__restrict__ out,
                                 int ld_out, double *__restrict__ clr, long n_clr)
{
    if (clr) {
        // this block's share of the range to clear
        const long nb = (long)gridDim.x * gridDim.y, bi = (long)blockIdx.y * gridDim.x + blockIdx.x;
        const long per = (n_clr + nb - 1) / nb, e = min(bi * per + per, n_clr);
        for (long k = bi * per + threadIdx.x; k < e; k += blockDim.x) clr[k] = 0.0;
    }
    int i = blockIdx.y;
    int id = ids[i];
    float *o = out + (size_t)i * ld_out;
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < n_cols; c += gridDim.x * blockDim.x) {
        if (id < 0 || id >= n_rows_logical) { o[c] = 0.0f; continue; }
        if (type == 0) {   // F32 rows are copied as they are (src/model.c:459-463)
            o[c] = ((const float *)qs)[(size_t)id * n_pairs * 64 + c];
            continue;
        }
        int T = id / 32, j = id % 32;
        int b = c / 32, e = c % 32, p = b / 2, blk = b % 2, h = e / 16;
        uint32_t dd = dpl[((size_t)T * n_pairs + p) * 32 + j];
        float d = vx_half_bits_to_float((dd >> (16 * blk)) & 0xFFFFu) * scale;
        int v;
        if (type == 2) {
            int s = (e % 16) / 8, kk = e % 8;
            uint32_t q = qs[(((size_t)T * n_pairs + p) * 64 + j + 32 * h) * 4 + blk * 2 + s];
            v = (int)((q >> (4 * kSlot4[kk])) & 15u) - 8;
        } else {
            int e2 = e - 16 * h;
            uint32_t q = qs[(((size_t)T * n_pairs * 2 + b) * 64 + j + 32 * h) * 4 + e2 / 4];
            v = (int)(int8_t)((q >> (8 * kPos8[e2 % 4])) & 255u);
        }
        o[c] = (float)v * d;
    }
}

extern "C" int vxh_qmat_gather_rows_clear(const vxh_qmat *m, const int *dev_ids, int n, float scale,
                                          float *out, int ld_out, double *clr, long n_clr, vxh_stream s)
{
    if (n_clr < 0 || (n_clr > 0 && !clr)) return vxh_fail(VXH_ERR_PARAM, "gather: clear %ld doubles at %p", n_clr,
                                                          (void *)clr);
    if (n <= 0) return n_clr > 0 ? vxh_fill_f32((float *)clr, 0.0f, 2 * (size_t)n_clr, s) : VXH_OK;
    int gx = (m->n_cols + 255) / 256;
    if (gx > 64) gx = 64;
    // enough workgroups that each clears at most 4096 doubles (the gather
    // loop has nothing to do in the extra ones)
    const long gc = (n_clr + 4096L * n - 1) / (4096L * n);
    if (gc > gx) gx = (int)(gc < 1024 ? gc : 1024);
    dim3 grid(gx, n);
    vx_gather_kernel<<<grid, 256, 0, vxh_hs(s)>>>((const uint32_t *)m->qs, (const uint32_t *)m->d,
                                                  m->type, m->n_rows, m->n_cols, m->n_pairs, dev_ids,
                                                  scale, out, ld_out, n_clr > 0 ? clr : nullptr, n_clr);
    VXH_LAUNCHED();
    return VXH_OK;
}

extern "C" int vxh_qmat_gather_rows(const vxh_qmat *m, const int *dev_ids, int n, float scale,
                                    float *out, int ld_out, vxh_stream s)
{
    if (n <= 0) return VXH_OK;
    return vxh_qmat_gather_rows_clear(m, dev_ids, n, scale, out, ld_out, nullptr, 0, s);
}
