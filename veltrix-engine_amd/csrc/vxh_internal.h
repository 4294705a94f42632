// Internal helpers shared by the HIP translation units of the engine.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>

#include "vxh.h"

typedef _Float16 vx_half2 __attribute__((ext_vector_type(2)));
typedef _Float16 vx_half8 __attribute__((ext_vector_type(8)));
typedef float vx_f32x16 __attribute__((ext_vector_type(16)));

// Records a message for vxh_last_error() and returns `code`.
#define vxh_fail vxh_set_error

#define VXH_CHECK(expr)                                                              \
    do {                                                                             \
        hipError_t e_ = (expr);                                                      \
        if (e_ != hipSuccess)                                                        \
            return vxh_fail(e_ == hipErrorOutOfMemory ? VXH_ERR_ALLOC : VXH_ERR_LAUNCH, \
                            "%s: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__,   \
                            __LINE__);                                               \
    } while (0)

#define VXH_LAUNCHED()                                                               \
    do {                                                                             \
        hipError_t e_ = hipGetLastError();                                           \
        if (e_ != hipSuccess)                                                        \
            return vxh_fail(VXH_ERR_LAUNCH, "launch: %s (%s:%d)", hipGetErrorString(e_), \
                            __FILE__, __LINE__);                                     \
    } while (0)

static inline hipStream_t vxh_hs(vxh_stream s) { return (hipStream_t)s; }

// Number of 16-byte panel units per block of 32 columns for M rows:
// 2 MFMA halves (s) x 2 lane halves (h) x 2M slots.
static inline int vxh_panel_units_per_block(int M) { return 2 * 2 * 2 * M; }

__device__ __forceinline__ float vx_half_bits_to_float(uint32_t bits16)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// inv = 1/sqrt(ss/K + 1e-5) as in the reference (src/tensor.c:134-139);
// returns 0 when the rms is below 1e-10 (the reference then writes zeros).
__device__ __forceinline__ float vx_rms_inv(float ss, int K)
{
    float rms = sqrtf(ss / (float)K + 1e-5f);
    return rms < 1e-10f ? 0.0f : 1.0f / rms;
}

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

// Deferred RMSNorm and bias of one q|k|v sum, then the RoPE rotation of a
// pair (src/tensor.c:249-270), written with explicit fmaf so that every
// kernel that derives q/k rows rounds them the same way.
__device__ __forceinline__ float vx_norm_bias(double x, float rin, const float *bias, int el)
{
    return bias ? fmaf((float)x, rin, bias[el]) : (float)x * rin;
}

__device__ __forceinline__ float2 vx_rope_rot(float a, float b, float c, float s)
{
    return make_float2(fmaf(a, c, -(b * s)), fmaf(a, s, b * c));
}

// Wavefront reductions in VALU: DPP within each row of 16 lanes (quad_perm
// [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror), then the gfx950 lane
// swaps for the lane ^ 16 and lane ^ 32 partners.  A swap of a register
// with itself returns {own value, partner value} in some order, so max and
// sum over the two results equal max/sum with the partner.  Every lane ends
// with the result (as the __shfl_xor butterfly, without its six dependent
// LDS-crossbar round trips).
template <int CTRL>
__device__ __forceinline__ float vx_dpp(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float vx_max_x16(float v)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float vx_max_x32(float v)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float vx_sum_x16(float v)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float vx_sum_x32(float v)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float vx_wave_max64(float v)
{
    v = fmaxf(v, vx_dpp<0xB1>(v));
    v = fmaxf(v, vx_dpp<0x4E>(v));
    v = fmaxf(v, vx_dpp<0x141>(v));
    v = fmaxf(v, vx_dpp<0x140>(v));
    return vx_max_x32(vx_max_x16(v));
}

__device__ __forceinline__ float vx_wave_sum64(float v)
{
    v += vx_dpp<0xB1>(v);
    v += vx_dpp<0x4E>(v);
    v += vx_dpp<0x141>(v);
    v += vx_dpp<0x140>(v);
    return vx_sum_x32(vx_sum_x16(v));
}

// The same sum for fp64 values (each 32-bit half moved by the same DPP or
// swap, so the halves stay paired); exact for integers below 2^53.
template <int CTRL>
__device__ __forceinline__ double vx_dpp_f64(double v)
{
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const int lo = (int)(unsigned)b, hi = (int)(unsigned)(b >> 32);
    const unsigned nlo = (unsigned)__builtin_amdgcn_update_dpp(lo, lo, CTRL, 0xF, 0xF, false);
    const unsigned nhi = (unsigned)__builtin_amdgcn_update_dpp(hi, hi, CTRL, 0xF, 0xF, false);
    return __longlong_as_double((long long)(((unsigned long long)nhi << 32) | nlo));
}

template <bool X32>
__device__ __forceinline__ double vx_sum_swap_f64(double v)
{
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const unsigned lo = (unsigned)b, hi = (unsigned)(b >> 32);
    const auto rl = X32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                        : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto rh = X32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                        : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    const double a = __longlong_as_double((long long)(((unsigned long long)rh[0] << 32) | rl[0]));
    const double c = __longlong_as_double((long long)(((unsigned long long)rh[1] << 32) | rl[1]));
    return a + c;
}

__device__ __forceinline__ double vx_wave_sum64_f64(double v)
{
    v += vx_dpp_f64<0xB1>(v);
    v += vx_dpp_f64<0x4E>(v);
    v += vx_dpp_f64<0x141>(v);
    v += vx_dpp_f64<0x140>(v);
    return vx_sum_swap_f64<true>(vx_sum_swap_f64<false>(v));
}
