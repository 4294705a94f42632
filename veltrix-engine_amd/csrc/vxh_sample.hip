// Vocab-wide softmax statistics, the draft sampler and the verify decisions
// (ratio test, residual resample, bonus draw) of speculative decoding.
//
// Probabilities follow the reference's sampler arithmetic
// (src/speculative.c:44-53): p_v = expf((l_v - max)/T) * (1/(sum + 1e-30)).
// Every draw is an inverse CDF over 2^32 fixed-point masses
// W_v = round(w_v * 2^32): the first v whose prefix sum reaches
// max(1, ceil(U*S/2^24)) for the uniform u = U/2^24.  Integer prefix sums do
// not depend on the summation order, so the GPU and a sequential CPU pick the
// same token from the same w.
#include <cstring>

#include "vxh_internal.h"

#define SB 1024   // threads per sampling workgroup

// round(w * 2^32) = floor(w * 2^32 + 0.5), exactly, in fp32 arithmetic, for
// the probabilities and residual masses every caller passes (0 <= w <= 1):
// x = w * 2^32 is exact; below 0.5 the result is 0; from 0.5 to 2^23 the sum
// x + 0.5 is either exact (same binade as x) or lies in the next binade
// below x's next integer, so truncation gives the floor; from 2^23 on x is
// an integer.  w = 1 gives 2^32 (larger w saturate there); NaN gives 0.
__device__ __forceinline__ uint64_t vx_fixed32(float w)
{
    // straight-line selects: unrolled over a thread's entries, early returns
    // became a branch per entry
    const float x = w * 4294967296.0f;
    float r = x < 8388608.0f ? x + 0.5f : x;
    r = x >= 0.5f ? r : 0.0f;
    const bool top = x >= 4294967296.0f;
    const uint32_t lo = top ? 0u : (uint32_t)fminf(r, 4294967040.0f);
    return ((uint64_t)(top ? 1u : 0u) << 32) | lo;
}

// --- workgroup reductions (SB threads, 16 waves) ----------------------------
__device__ __forceinline__ float vx_wg_max(float v, float *red)
{
    v = vx_wave_max64(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < SB / 64; i++) r = fmaxf(r, red[i]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ float vx_wg_sum(float v, float *red)
{
    v = vx_wave_sum64(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = 0.0f;
    for (int i = 0; i < SB / 64; i++) r += red[i];
    __syncthreads();
    return r;
}

__device__ __forceinline__ uint64_t vx_shfl_xor_u64(uint64_t v, int o)
{
    uint32_t lo = __shfl_xor((uint32_t)v, o, 64), hi = __shfl_xor((uint32_t)(v >> 32), o, 64);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t vx_wg_sum_u64(uint64_t v, uint64_t *red)
{
    for (int o = 32; o > 0; o >>= 1) v += vx_shfl_xor_u64(v, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t r = 0;
    for (int i = 0; i < SB / 64; i++) r += red[i];
    __syncthreads();
    return r;
}

// First index of the maximum (strict '>' scan order, src/speculative.c:93-98).
// Lanes start from (-inf, 0x7fffffff); a row with no value above -inf (all
// NaN or all -inf) keeps that sentinel, which maps to index 0 -- the
// reference's scan also stays on its first element -- so callers can always
// index the row with the result.
// (v, idx) <- the better of itself and (ov, oi): larger value, lower index on ties
__device__ __forceinline__ void vx_am_merge(float &v, int &idx, float ov, int oi)
{
    if (ov > v || (ov == v && oi < idx)) { v = ov; idx = oi; }
}

template <int CTRL>
__device__ __forceinline__ void vx_am_dpp(float &v, int &idx)
{
    const float ov = vx_dpp<CTRL>(v);
    const int oi = __builtin_amdgcn_update_dpp(idx, idx, CTRL, 0xF, 0xF, false);
    vx_am_merge(v, idx, ov, oi);
}

// wavefront argmax in VALU (the same DPP steps and lane swaps as vx_wave_max64)
__device__ __forceinline__ void vx_wave_argmax64(float &v, int &idx)
{
    vx_am_dpp<0xB1>(v, idx);
    vx_am_dpp<0x4E>(v, idx);
    vx_am_dpp<0x141>(v, idx);
    vx_am_dpp<0x140>(v, idx);
    {
        const auto rv = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        const auto ri = __builtin_amdgcn_permlane16_swap((unsigned)idx, (unsigned)idx, false, false);
        v = __uint_as_float(rv[0]);
        idx = (int)ri[0];
        vx_am_merge(v, idx, __uint_as_float(rv[1]), (int)ri[1]);
    }
    {
        const auto rv = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        const auto ri = __builtin_amdgcn_permlane32_swap((unsigned)idx, (unsigned)idx, false, false);
        v = __uint_as_float(rv[0]);
        idx = (int)ri[0];
        vx_am_merge(v, idx, __uint_as_float(rv[1]), (int)ri[1]);
    }
}

// *found (optional): whether some value was above -inf; the maximum itself
// is then *vmax (the caller reads l[0] otherwise, as the reference does)
__device__ __forceinline__ int vx_wg_argmax(float v, int idx, float *redv, int *redi, float *vmax = nullptr,
                                            bool *found = nullptr)
{
    vx_wave_argmax64(v, idx);
    if ((threadIdx.x & 63) == 0) { redv[threadIdx.x >> 6] = v; redi[threadIdx.x >> 6] = idx; }
    __syncthreads();
    float bv = redv[0];
    int bi = redi[0];
    for (int i = 1; i < SB / 64; i++)
        if (redv[i] > bv || (redv[i] == bv && redi[i] < bi)) { bv = redv[i]; bi = redi[i]; }
    __syncthreads();
    if (vmax) *vmax = bv;
    if (found) *found = bi != 0x7fffffff;
    return bi == 0x7fffffff ? 0 : bi;
}

// Thread t owns the contiguous index range [t*chunk, min((t+1)*chunk, n)).
// Returns the first index whose inclusive prefix of W reaches thr (n-1 if none).
template <typename WF>
__device__ int vx_wg_find_prefix(int n, uint64_t thr, WF W, uint64_t *scan, int *res)
{
    const int chunk = (n + SB - 1) / SB;
    const int b = threadIdx.x * chunk, e = min(b + chunk, n);
    uint64_t local = 0;
    for (int v = b; v < e; v++) local += W(v);
    scan[threadIdx.x] = local;
    if (threadIdx.x == 0) *res = n - 1;
    __syncthreads();
    // inclusive scan over SB entries (Hillis-Steele in shared memory)
    for (int o = 1; o < SB; o <<= 1) {
        uint64_t add = threadIdx.x >= o ? scan[threadIdx.x - o] : 0ull;
        __syncthreads();
        scan[threadIdx.x] += add;
        __syncthreads();
    }
    uint64_t before = threadIdx.x ? scan[threadIdx.x - 1] : 0ull;
    uint64_t after = scan[threadIdx.x];
    if (before < thr && after >= thr) {
        uint64_t c = before;
        for (int v = b; v < e; v++) {
            c += W(v);
            if (c >= thr) { *res = v; break; }
        }
    }
    __syncthreads();
    int r = *res;
    __syncthreads();
    return r;
}

__device__ __forceinline__ uint64_t vx_threshold(float u, uint64_t S)
{
    uint64_t U = (uint64_t)(u * 16777216.0f);
    uint64_t t = (U * S + 16777215ull) >> 24;
    return t ? t : 1ull;
}

// ---------------------------------------------------------------------------
// row statistics: stats[r] = {max, sum exp((l-max)/T), argmax}
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(SB) void vx_row_stats_kernel(const float *__restrict__ L, int ldl, int V,
                                                          float T, float *__restrict__ stats)
{
    __shared__ float redv[SB / 64];
    __shared__ int redi[SB / 64];
    const float *l = L + (size_t)blockIdx.x * ldl;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int v = threadIdx.x; v < V; v += SB) {
        float x = l[v];
        if (x > bv || (x == bv && v < bi)) { bv = x; bi = v; }
    }
    int am = vx_wg_argmax(bv, bi, redv, redi);
    float mx = l[am];
    float s = 0.0f;
    if (T > 0.0f)
        for (int v = threadIdx.x; v < V; v += SB) s += expf((l[v] - mx) / T);
    s = vx_wg_sum(s, redv);
    if (threadIdx.x == 0) {
        stats[blockIdx.x * 3 + 0] = mx;
        stats[blockIdx.x * 3 + 1] = s;
        stats[blockIdx.x * 3 + 2] = __int_as_float(am);
    }
}

extern "C" int vxh_row_stats(const float *L, int ldl, int R, int V, float T, float *stats,
                             vxh_stream s)
{
    if (R <= 0) return VXH_OK;
    vx_row_stats_kernel<<<R, SB, 0, vxh_hs(s)>>>(L, ldl, V, T, stats);
    VXH_LAUNCHED();
    return VXH_OK;
}

// ---------------------------------------------------------------------------
// draft sampler
// nuc = {max, inv, tau, tie_cut (int bits), mass, argmax (int bits), 0, 0}:
// member(v) = p_v > tau || (p_v == tau && v <= tie_cut); tau < 0: all tokens.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float vx_prob(const float *l, int v, float mx, float inv, float T)
{
    return expf((l[v] - mx) / T) * inv;
}

__global__ __launch_bounds__(SB) void vx_sample_kernel(const float *__restrict__ l, int V, float T,
                                                       float top_p, const float *__restrict__ u,
                                                       int *__restrict__ token_out,
                                                       float *__restrict__ nuc)
{
    __shared__ float redv[SB / 64];
    __shared__ int redi[SB / 64];
    __shared__ uint64_t red64[SB / 64];
    __shared__ uint64_t scan[SB];
    __shared__ int res;

    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int v = threadIdx.x; v < V; v += SB) {
        float x = l[v];
        if (x > bv || (x == bv && v < bi)) { bv = x; bi = v; }
    }
    const int am = vx_wg_argmax(bv, bi, redv, redi);
    if (!(T > 0.0f)) {
        if (threadIdx.x == 0) {
            token_out[0] = am;
            nuc[0] = l[am]; nuc[1] = 0.0f; nuc[2] = -1.0f; nuc[3] = __int_as_float(V - 1);
            nuc[4] = 0.0f; nuc[5] = __int_as_float(am); nuc[6] = 0.0f; nuc[7] = 0.0f;
        }
        return;
    }
    const float mx = l[am];
    float s = 0.0f;
    for (int v = threadIdx.x; v < V; v += SB) s += expf((l[v] - mx) / T);
    s = vx_wg_sum(s, redv);
    const float inv = 1.0f / (s + 1e-30f);

    float tau = -1.0f;
    int tie_cut = V - 1;
    if (top_p < 1.0f) {
        // at least one unit: the reference's nucleus always holds its first
        // token, also for top_p <= 0 (src/speculative.c:67-74)
        const double tpu = top_p > 0.0f ? ceil((double)top_p * 4294967296.0) : 0.0;
        const uint64_t TP = tpu < 1.0 ? 1ull : (uint64_t)tpu;
        // largest probability value tau with mass(p >= tau) >= TP (bisection
        // over the bit patterns of non-negative floats, which are ordered)
        uint32_t lo = 0u, hi = 0x3F800000u;     // mass(p >= 0) = all >= TP
        while (lo < hi) {
            uint32_t mid = lo + (hi - lo + 1) / 2;
            float t = __uint_as_float(mid);
            uint64_t acc = 0;
            for (int v = threadIdx.x; v < V; v += SB) {
                float p = vx_prob(l, v, mx, inv, T);
                if (p >= t) acc += vx_fixed32(p);
            }
            acc = vx_wg_sum_u64(acc, red64);
            if (acc >= TP) lo = mid; else hi = mid - 1;
        }
        tau = __uint_as_float(lo);
        uint64_t gt = 0;
        for (int v = threadIdx.x; v < V; v += SB) {
            float p = vx_prob(l, v, mx, inv, T);
            if (p > tau) gt += vx_fixed32(p);
        }
        gt = vx_wg_sum_u64(gt, red64);
        const uint64_t pt = vx_fixed32(tau);
        if (pt == 0 || gt >= TP) {
            tie_cut = V - 1;   // cannot happen for tau > 0; keep every tie
        } else {
            // ties at tau enter in index order until the mass reaches TP
            const uint64_t need_units = TP - gt;
            const uint64_t j = (need_units + pt - 1) / pt;    // number of ties needed
            tie_cut = vx_wg_find_prefix(V, j, [&](int v) -> uint64_t {
                return vx_prob(l, v, mx, inv, T) == tau ? 1ull : 0ull;
            }, scan, &res);
        }
        if (tau <= 0.0f) { tau = -1.0f; tie_cut = V - 1; }
    }
    auto member_w = [&](int v) -> uint64_t {
        float p = vx_prob(l, v, mx, inv, T);
        bool in = tau < 0.0f || p > tau || (p == tau && v <= tie_cut);
        return in ? vx_fixed32(p) : 0ull;
    };
    uint64_t S = 0;
    for (int v = threadIdx.x; v < V; v += SB) S += member_w(v);
    S = vx_wg_sum_u64(S, red64);
    int tok;
    if (S == 0) tok = am;
    else tok = vx_wg_find_prefix(V, vx_threshold(u[0], S), member_w, scan, &res);
    if (threadIdx.x == 0) {
        token_out[0] = tok;
        nuc[0] = mx; nuc[1] = inv; nuc[2] = tau; nuc[3] = __int_as_float(tie_cut);
        nuc[4] = (float)((double)S / 4294967296.0); nuc[5] = __int_as_float(am);
        nuc[6] = 0.0f; nuc[7] = 0.0f;
    }
}

// The sampler without a nucleus for V <= SB * SE: each thread loads its SE
// entries once; exponentials and masses stay in registers, the inverse-CDF
// search uses per-wavefront totals and one lane scan in the wavefront where
// the threshold lands (no passes over the row).  Same arithmetic as
// vx_sample_kernel with top_p = 1.
#define SE 32

__device__ __forceinline__ uint64_t vx_shfl_up_u64(uint64_t v, int o)
{
    uint32_t lo = __shfl_up((uint32_t)v, o, 64), hi = __shfl_up((uint32_t)(v >> 32), o, 64);
    return ((uint64_t)hi << 32) | lo;
}

// Wave-blocked entries: wavefront w owns entries [2048 w, 2048 w + 2048)
// (SB * SE = 32768 at most); its load j (0..7) covers entries 256 j ..
// 256 j + 255 of that block, 4 consecutive ones per lane, so each load and
// store of a wavefront is one contiguous KB (a thread owning 32 consecutive
// entries made every float4 access of a wavefront touch 64 cache lines, and
// the row's 128 KB thrashed the CU's L1).  In index order a wavefront's
// entries run j-major, then lane, then the lane's 4 entries.
#define SJ (SE / 4)

__global__ __launch_bounds__(SB) void vx_sample_reg_kernel(const float *__restrict__ l, int V, float T,
                                                           const float *__restrict__ u,
                                                           int *__restrict__ token_out,
                                                           float *__restrict__ nuc,
                                                           float *__restrict__ keep)
{
    __shared__ float redv[SB / 64];
    __shared__ int redi[SB / 64];
    __shared__ double wsum[SB / 64];
    __shared__ int res;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = wave * (64 * SE) + 4 * lane;   // entry (j, c) of this lane: b + 256 j + c
    float x[SE];
    if (wave * (64 * SE) + 64 * SE <= V) {
#pragma unroll
        for (int j = 0; j < SJ; j++) {
            const float4 v = *(const float4 *)(l + b + 256 * j);
            x[4 * j] = v.x; x[4 * j + 1] = v.y; x[4 * j + 2] = v.z; x[4 * j + 3] = v.w;
        }
        if (keep) {
#pragma unroll
            for (int j = 0; j < SJ; j++)
                *(float4 *)(keep + b + 256 * j) = make_float4(x[4 * j], x[4 * j + 1], x[4 * j + 2], x[4 * j + 3]);
        }
    } else {
        // the block holding entry V-1 and the ones after it: entries past V
        // read as -inf, so they never win the argmax and their exp is 0
#pragma unroll
        for (int j = 0; j < SJ; j++)
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int v = b + 256 * j + c;
                const float t = l[min(v, V - 1)];
                x[4 * j + c] = v < V ? t : -INFINITY;
            }
        if (keep) {
#pragma unroll
            for (int j = 0; j < SJ; j++)
#pragma unroll
                for (int c = 0; c < 4; c++)
                    if (b + 256 * j + c < V) keep[b + 256 * j + c] = x[4 * j + c];
        }
    }
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < SJ; j++)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            // bitwise, not short-circuit: selects instead of a branch per entry
            const int v = b + 256 * j + c;
            const float t = x[4 * j + c];
            const bool better = (v < V) & ((t > bv) | ((t == bv) & (v < bi)));
            bv = better ? t : bv;
            bi = better ? v : bi;
        }
    float amv;
    bool amf;
    const int am = vx_wg_argmax(bv, bi, redv, redi, &amv, &amf);
    if (!(T > 0.0f)) {
        if (threadIdx.x == 0) {
            token_out[0] = am;
            nuc[0] = l[am]; nuc[1] = 0.0f; nuc[2] = -1.0f; nuc[3] = __int_as_float(V - 1);
            nuc[4] = 0.0f; nuc[5] = __int_as_float(am); nuc[6] = 0.0f; nuc[7] = 0.0f;
        }
        return;
    }
    const float mx = amf ? amv : l[0];
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < SE; j++) {
        x[j] = expf((x[j] - mx) / T);
        sum += x[j];
    }
    sum = vx_wg_sum(sum, redv);
    const float inv = 1.0f / (sum + 1e-30f);
    // fixed-point masses; partial sums are integers far below 2^53, so the
    // fp64 reductions are exact and order-free
    uint64_t lt = 0;
#pragma unroll
    for (int j = 0; j < SE; j++) {
        x[j] *= inv;                      // p_v = expf((l_v - max)/T) * inv
        lt += vx_fixed32(x[j]);
    }
    const double wt = vx_wave_sum64_f64((double)lt);
    if (lane == 0) wsum[wave] = wt;
    if (threadIdx.x == 0) res = am;
    __syncthreads();
    double off = 0.0, Sd = 0.0;
    for (int w = 0; w < SB / 64; w++) {
        if (w < wave) off += wsum[w];
        Sd += wsum[w];
    }
    const uint64_t S = (uint64_t)Sd;
    if (S > 0) {
        const uint64_t thr = vx_threshold(u[0], S);
        const uint64_t before = (uint64_t)off;
        if (before < thr && before + (uint64_t)wt >= thr) {
            // the landing wavefront: which of its loads, then which lane,
            // then which of the lane's 4 entries first reaches thr
            uint64_t acc = before, acc_j = before;
            int js = SJ - 1;
            bool fj = false;
#pragma unroll
            for (int j = 0; j < SJ; j++) {
                uint64_t sj = 0;
#pragma unroll
                for (int c = 0; c < 4; c++) sj += vx_fixed32(x[4 * j + c]);
                const uint64_t tj = (uint64_t)vx_wave_sum64_f64((double)sj);
                const bool hit = !fj & (acc + tj >= thr);
                js = hit ? j : js;
                acc_j = hit ? acc : acc_j;
                fj = fj | hit;
                acc += tj;
            }
            float p[4] = {x[0], x[1], x[2], x[3]};
#pragma unroll
            for (int j = 1; j < SJ; j++)
#pragma unroll
                for (int c = 0; c < 4; c++) p[c] = js == j ? x[4 * j + c] : p[c];
            uint64_t s = 0;
#pragma unroll
            for (int c = 0; c < 4; c++) s += vx_fixed32(p[c]);
            uint64_t incl = s;
            for (int o = 1; o < 64; o <<= 1) {
                const uint64_t y = vx_shfl_up_u64(incl, o);
                if (lane >= o) incl += y;
            }
            const uint64_t bl = acc_j + incl - s;
            if (bl < thr && bl + s >= thr) {
                uint64_t c = bl;
                int tok = b + 256 * js + 3;
                bool found = false;
#pragma unroll
                for (int cc = 0; cc < 4; cc++) {
                    c += vx_fixed32(p[cc]);
                    const bool hit = !found & (c >= thr);
                    tok = hit ? b + 256 * js + cc : tok;
                    found = found | hit;
                }
                res = tok;
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        token_out[0] = res;
        nuc[0] = mx; nuc[1] = inv; nuc[2] = -1.0f; nuc[3] = __int_as_float(V - 1);
        nuc[4] = (float)((double)S / 4294967296.0); nuc[5] = __int_as_float(am);
        nuc[6] = 0.0f; nuc[7] = 0.0f;
    }
}

extern "C" int vxh_sample_keep(const float *l, int V, float T, float top_p, const float *u_dev,
                               int *token_out, float *nuc, float *keep, vxh_stream s)
{
    if (V <= 0) return vxh_fail(VXH_ERR_PARAM, "sample: V %d", V);
    if (keep == l) keep = nullptr;
    if (!(top_p < 1.0f) && V <= SB * SE && ((uintptr_t)l & 15) == 0 && ((uintptr_t)keep & 15) == 0) {
        // the register sampler stores the row into keep as it loads it
        vx_sample_reg_kernel<<<1, SB, 0, vxh_hs(s)>>>(l, V, T, u_dev, token_out, nuc, keep);
    } else {
        if (keep) VXH_CHECK(hipMemcpyAsync(keep, l, sizeof(float) * (size_t)V, hipMemcpyDeviceToDevice, vxh_hs(s)));
        vx_sample_kernel<<<1, SB, 0, vxh_hs(s)>>>(l, V, T, top_p, u_dev, token_out, nuc);
    }
    VXH_LAUNCHED();
    return VXH_OK;
}

extern "C" int vxh_sample(const float *l, int V, float T, float top_p, const float *u_dev,
                          int *token_out, float *nuc, vxh_stream s)
{
    return vxh_sample_keep(l, V, T, top_p, u_dev, token_out, nuc, nullptr, s);
}

// ---------------------------------------------------------------------------
// verify decisions
// ---------------------------------------------------------------------------
// q_j(v) of the draft: the renormalised nucleus of softmax(D_j/T), from the
// draft logit dv = D_j[v] and the row's nucleus descriptor.
struct vx_nuc {
    float mx, inv, tau, mass;
    int tie;
};
__device__ __forceinline__ vx_nuc vx_nuc_load(const float *nuc)
{
    return {nuc[0], nuc[1], nuc[2], nuc[4], __float_as_int(nuc[3])};
}
__device__ __forceinline__ float vx_draft_q_of(float dv, const vx_nuc &n, int v, float T)
{
    const float p = expf((dv - n.mx) / T) * n.inv;
    const bool in = (n.tau < 0.0f) | (p > n.tau) | ((p == n.tau) & (v <= n.tie));
    return in ? p / n.mass : 0.0f;
}
__device__ __forceinline__ float vx_draft_q(const float *d, const float *nuc, int v, float T)
{
    return vx_draft_q_of(d[v], vx_nuc_load(nuc), v, T);
}

// One pass over the decided row: thread t sums the fixed-point masses of its
// contiguous entries [t*C, t*C + C) (C = ceil(V / SB)); a workgroup scan of
// those sums gives the total and the chunk where the inverse CDF lands, and
// only that chunk is evaluated again (the first index whose inclusive prefix
// reaches the threshold).  Entries are evaluated V + C times instead of 3V.
template <typename WF>
__device__ int vx_wg_chunk_prefix(int n, uint64_t thr_u, bool by_u, float uval, WF W, uint64_t *wsum, int *res,
                                  uint64_t *total)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunk = (n + SB - 1) / SB;
    const int b = threadIdx.x * chunk, e = min(b + chunk, n);
    uint64_t local = 0;
    for (int v = b; v < e; v++) local += W(v);
    uint64_t incl = local;
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t y = vx_shfl_up_u64(incl, o);
        if (lane >= o) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    if (threadIdx.x == 0) *res = n - 1;
    __syncthreads();
    uint64_t off = 0, S = 0;
    for (int w = 0; w < SB / 64; w++) {
        if (w < wave) off += wsum[w];
        S += wsum[w];
    }
    *total = S;
    const uint64_t thr = by_u ? vx_threshold(uval, S) : thr_u;
    const uint64_t before = off + incl - local;
    if (S > 0 && before < thr && before + local >= thr) {
        uint64_t c = before;
        for (int v = b; v < e; v++) {
            c += W(v);
            if (c >= thr) { *res = v; break; }
        }
    }
    __syncthreads();
    const int r = *res;
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(SB) void vx_accept_kernel(const float *__restrict__ L, int ldl, int V,
                                                       const float *__restrict__ stats,
                                                       const float *__restrict__ D, int ldd, int Vd,
                                                       const float *__restrict__ nuc,
                                                       const int *__restrict__ drafts, int k,
                                                       float T, const float *__restrict__ u,
                                                       int *__restrict__ out)
{
    __shared__ float redv[SB / 64];
    __shared__ int redi[SB / 64];
    __shared__ uint64_t wsum[SB / 64];
    __shared__ int res;
    __shared__ int s_rej;

    if (!(T > 0.0f)) {
        // greedy: accept d_j while it is the first argmax of L_j
        if (threadIdx.x == 0) {
            int j = 0;
            for (; j < k; j++) {
                int a = __float_as_int(stats[j * 3 + 2]);
                out[2 + j] = a;
                if (a != drafts[j]) break;
            }
            if (j == k) out[2 + k] = __float_as_int(stats[k * 3 + 2]);
            out[0] = j < k ? j + 1 : k + 1;
            out[1] = j;
        }
        return;
    }
    if (threadIdx.x < 64) {
        // ratio tests of the drafts on parallel lanes; the first failing one
        // is where the sequential scan (src/speculative.c:199-200) stops
        const int lane = threadIdx.x;
        bool rej = true;
        if (lane < k) {
            const float *lj = L + (size_t)lane * ldl;
            const float mx = stats[lane * 3 + 0], inv = 1.0f / (stats[lane * 3 + 1] + 1e-30f);
            const int d = drafts[lane];
            const float pt = (d >= 0 && d < V) ? expf((lj[d] - mx) / T) * inv : 0.0f;
            const float qd = (d >= 0 && d < Vd) ? vx_draft_q(D + (size_t)lane * ldd, nuc + lane * 8, d, T) : 0.0f;
            const float alpha = fminf(1.0f, pt / fmaxf(qd, 1e-10f));
            rej = !(u[lane] < alpha);
        }
        // lanes k..63 count as failing, so the first failing lane is the
        // decided row (k when every draft is accepted); drafts beyond 64
        // continue sequentially below
        const uint64_t bal = __ballot(rej);
        int j = bal ? __builtin_ctzll(bal) : 64;
        if (lane < min(j, k)) out[2 + lane] = drafts[lane];
        if (lane == 0) {
            for (; j < k; j++) {   // only k > 64
                const float *lj = L + (size_t)j * ldl;
                const float mx = stats[j * 3 + 0], inv = 1.0f / (stats[j * 3 + 1] + 1e-30f);
                const int d = drafts[j];
                const float pt = (d >= 0 && d < V) ? expf((lj[d] - mx) / T) * inv : 0.0f;
                const float qd = (d >= 0 && d < Vd) ? vx_draft_q(D + (size_t)j * ldd, nuc + j * 8, d, T) : 0.0f;
                const float alpha = fminf(1.0f, pt / fmaxf(qd, 1e-10f));
                if (!(u[j] < alpha)) break;
                out[2 + j] = d;
            }
            s_rej = min(j, k);
        }
    }
    __syncthreads();
    const int j = s_rej;
    const float *lj = L + (size_t)j * ldl;
    const float mx = stats[j * 3 + 0], inv = 1.0f / (stats[j * 3 + 1] + 1e-30f);
    int tok;
    uint64_t S = 0;
    if (j < k) {
        const float *dj = D + (size_t)j * ldd;
        const float *nj = nuc + j * 8;
        auto resid = [&](int v) -> float {
            float p = expf((lj[v] - mx) / T) * inv;
            float q = v < Vd ? vx_draft_q(dj, nj, v, T) : 0.0f;
            return fmaxf(0.0f, p - q);
        };
        auto W = [&](int v) -> uint64_t { return vx_fixed32(resid(v)); };
        tok = vx_wg_chunk_prefix(V, 0, true, u[k], W, wsum, &res, &S);
        if (S == 0) {
            float bv = -INFINITY;
            int bi = 0x7fffffff;
            for (int v = threadIdx.x; v < V; v += SB) {
                float r = resid(v);
                if (r > bv || (r == bv && v < bi)) { bv = r; bi = v; }
            }
            tok = vx_wg_argmax(bv, bi, redv, redi);
        }
    } else {
        auto W = [&](int v) -> uint64_t { return vx_fixed32(expf((lj[v] - mx) / T) * inv); };
        tok = vx_wg_chunk_prefix(V, 0, true, u[k], W, wsum, &res, &S);
        if (S == 0) tok = __float_as_int(stats[j * 3 + 2]);
    }
    if (threadIdx.x == 0) {
        out[2 + j] = tok;
        out[0] = j + 1;
        out[1] = j;
    }
}

// vx_accept_kernel for V <= SB * SE: the ratio tests of the k drafts run on
// k lanes at once (the first rejection is the first failing lane, as in the
// sequential scan); the decided row is read once, wave-blocked and
// coalesced, for its total mass, and only the wavefront where the inverse
// CDF lands reads its entries again.  Same arithmetic as vx_accept_kernel.
__global__ __launch_bounds__(SB) void vx_accept_reg_kernel(const float *__restrict__ L, int ldl, int V,
                                                           const float *__restrict__ stats,
                                                           const float *__restrict__ D, int ldd, int Vd,
                                                           const float *__restrict__ nuc,
                                                           const int *__restrict__ drafts, int k, float T,
                                                           const float *__restrict__ u, int *__restrict__ out)
{
    __shared__ float redv[SB / 64];
    __shared__ int redi[SB / 64];
    __shared__ double wsum[SB / 64];
    __shared__ int res;
    __shared__ int s_rej;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (threadIdx.x < 64) {
        // ratio test of draft j = lane (src/speculative.c:199-200 on probabilities)
        bool rej = true;
        if (lane < k) {
            const int j = lane;
            const float *lj = L + (size_t)j * ldl;
            const float mx = stats[j * 3 + 0], inv = 1.0f / (stats[j * 3 + 1] + 1e-30f);
            const int d = drafts[j];
            const float pt = (d >= 0 && d < V) ? expf((lj[d] - mx) / T) * inv : 0.0f;
            const float qd = (d >= 0 && d < Vd) ? vx_draft_q(D + (size_t)j * ldd, nuc + j * 8, d, T) : 0.0f;
            const float alpha = fminf(1.0f, pt / fmaxf(qd, 1e-10f));
            rej = !(u[j] < alpha);
        }
        const uint64_t bal = __ballot(rej);
        const int jr = bal ? __builtin_ctzll(bal) : 64;
        const int j = jr < k ? jr : k;
        if (lane < j) out[2 + lane] = drafts[lane];
        if (lane == 0) s_rej = j;
    }
    __syncthreads();
    const int j = s_rej;
    const float *lj = L + (size_t)j * ldl;
    const float mx = stats[j * 3 + 0], inv = 1.0f / (stats[j * 3 + 1] + 1e-30f);
    const float *dj = D + (size_t)min(j, k - 1) * ldd;
    const float *nj = nuc + min(j, k - 1) * 8;
    const bool resample = j < k;
    const vx_nuc nq = vx_nuc_load(nj);
    // wave-blocked entries as in vx_sample_reg_kernel: load j (0..SJ-1) of
    // a lane covers entries b + 256 j .. b + 256 j + 3
    const int b = wave * (64 * SE) + 4 * lane;
    const bool vec = wave * (64 * SE) + 64 * SE <= min(V, Vd) &&
                     (((uintptr_t)lj | (uintptr_t)dj) & 15) == 0;
    // entries of load jj: the residual max(0, p - q) at a rejection, p for
    // the bonus draw; 0 past V.  Straight-line loads with clamped addresses
    // (a load inside a per-entry branch waits for itself); no per-entry
    // array stays live, the one wavefront that needs entries again (landing
    // search, argmax) recomputes them from L2.
    auto entries4 = [&](int jj, float r[4]) {
        const int v0 = b + 256 * jj;
        float lv[4], dv[4];
        if (vec) {
            const float4 a4 = *(const float4 *)(lj + v0);
            const float4 c4 = *(const float4 *)(dj + v0);
            lv[0] = a4.x; lv[1] = a4.y; lv[2] = a4.z; lv[3] = a4.w;
            dv[0] = c4.x; dv[1] = c4.y; dv[2] = c4.z; dv[3] = c4.w;
        } else {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                lv[t] = lj[min(v0 + t, V - 1)];
                dv[t] = dj[min(v0 + t, Vd - 1)];
            }
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int v = v0 + t;
            const float p = expf((lv[t] - mx) / T) * inv;
            const float q = v < Vd ? vx_draft_q_of(dv[t], nq, v, T) : 0.0f;
            const float x = resample ? fmaxf(0.0f, p - q) : p;
            r[t] = v < V ? x : 0.0f;
        }
    };
    uint64_t lt = 0;
#pragma unroll
    for (int jj = 0; jj < SJ; jj++) {
        float r[4];
        entries4(jj, r);
#pragma unroll
        for (int t = 0; t < 4; t++) lt += vx_fixed32(r[t]);
    }
    // fixed-point partial sums are integers far below 2^53: exact in fp64
    const double wt = vx_wave_sum64_f64((double)lt);
    if (lane == 0) wsum[wave] = wt;
    __syncthreads();
    double off = 0.0, Sd = 0.0;
    for (int wv = 0; wv < SB / 64; wv++) {
        if (wv < wave) off += wsum[wv];
        Sd += wsum[wv];
    }
    const uint64_t S = (uint64_t)Sd;
    int tok;
    if (S == 0) {
        if (resample) {
            // no residual mass: argmax of the residual (first index on ties)
            float bv = -INFINITY;
            int bi = 0x7fffffff;
            for (int jj = 0; jj < SJ; jj++) {
                float r[4];
                entries4(jj, r);
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const int v = b + 256 * jj + t;
                    const bool better = (v < V) & ((r[t] > bv) | ((r[t] == bv) & (v < bi)));
                    bv = better ? r[t] : bv;
                    bi = better ? v : bi;
                }
            }
            tok = vx_wg_argmax(bv, bi, redv, redi);
        } else {
            tok = __float_as_int(stats[j * 3 + 2]);
        }
    } else {
        const uint64_t thr = vx_threshold(u[k], S);
        const uint64_t before = (uint64_t)off;
        if (threadIdx.x == 0) res = V - 1;
        __syncthreads();
        if (before < thr && before + (uint64_t)wt >= thr) {
            // the landing wavefront: which load, then which lane, then
            // which of the lane's 4 entries first reaches thr
            uint64_t acc = before, acc_j = before;
            int js = SJ - 1;
            bool fj = false;
            for (int jj = 0; jj < SJ; jj++) {
                float r[4];
                entries4(jj, r);
                uint64_t sj = 0;
#pragma unroll
                for (int t = 0; t < 4; t++) sj += vx_fixed32(r[t]);
                const uint64_t tj = (uint64_t)vx_wave_sum64_f64((double)sj);
                const bool hit = !fj & (acc + tj >= thr);
                js = hit ? jj : js;
                acc_j = hit ? acc : acc_j;
                fj = fj | hit;
                acc += tj;
            }
            float r[4];
            entries4(js, r);
            uint64_t sl = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) sl += vx_fixed32(r[t]);
            uint64_t incl = sl;
            for (int o = 1; o < 64; o <<= 1) {
                const uint64_t y = vx_shfl_up_u64(incl, o);
                if (lane >= o) incl += y;
            }
            const uint64_t bl = acc_j + incl - sl;
            if (bl < thr && bl + sl >= thr) {
                uint64_t c = bl;
                int t_hit = b + 256 * js + 3;
                bool found = false;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    c += vx_fixed32(r[t]);
                    const bool hit = !found & (c >= thr);
                    t_hit = hit ? b + 256 * js + t : t_hit;
                    found = found | hit;
                }
                res = t_hit;
            }
        }
        __syncthreads();
        tok = res;
    }
    if (threadIdx.x == 0) {
        out[2 + j] = tok;
        out[0] = j + 1;
        out[1] = j;
    }
}

extern "C" int vxh_accept(const float *L, int ldl, int V, const float *stats, const float *D,
                          int ldd, int Vd, const float *nuc, const int *drafts, int k, float T,
                          const float *u, int *out, vxh_stream s)
{
    if (k < 0 || V <= 0) return vxh_fail(VXH_ERR_PARAM, "accept: k %d V %d", k, V);
    if (T > 0.0f && k >= 1 && k <= 64 && V <= SB * SE)
        vx_accept_reg_kernel<<<1, SB, 0, vxh_hs(s)>>>(L, ldl, V, stats, D, ldd, Vd, nuc, drafts, k, T, u, out);
    else
        vx_accept_kernel<<<1, SB, 0, vxh_hs(s)>>>(L, ldl, V, stats, D, ldd, Vd, nuc, drafts, k, T, u, out);
    VXH_LAUNCHED();
    return VXH_OK;
}

// ---------------------------------------------------------------------------
// Multi-workgroup vocab kernels
// ---------------------------------------------------------------------------
// A row of V entries is cut into G <= 64 chunks of CH entries (CH a multiple
// of 1024), one 256-thread workgroup per chunk.  Each workgroup writes its
// chunk's partial result into the caller's workspace with device-coherent
// stores, waits until they have completed, and counts itself in with an
// atomic add; the workgroup that arrives last reads every partial with
// device-coherent loads, finishes the row in chunk order and sets the
// counter back to zero for the next launch.  No workgroup ever waits for
// another (no grid barrier, no co-residency assumption).  Fixed-point masses
// are integers, so their sums, and the token an inverse CDF lands on, do
// not depend on the chunking.
#define MB 256          // threads per workgroup
#define MC_MAX_G 64     // chunks per row

static int vx_mc_chunk(int V)
{
    const int per = (V + 1024 * MC_MAX_G - 1) / (1024 * MC_MAX_G);
    return 1024 * (per > 0 ? per : 1);
}

__device__ __forceinline__ void vx_st_coh(uint64_t *p, uint64_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t vx_ld_coh(uint64_t *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// True in the last of G workgroups to arrive.  Every thread waits until its
// own (device-coherent) stores have completed before the workgroup counts
// itself in, so the last one's coherent loads see every partial.
__device__ __forceinline__ bool vx_arrive_last(unsigned *cnt, unsigned G, int *s_last)
{
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        *s_last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1;
    __syncthreads();
    return *s_last != 0;
}

__device__ __forceinline__ void vx_mc_release(unsigned *cnt)
{
    if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 256-thread reductions (4 wavefronts, combined in wave order)
__device__ __forceinline__ int vx_mb_argmax(float v, int idx, float *rv, int *ri, float *vmax, bool *found)
{
    vx_wave_argmax64(v, idx);
    if ((threadIdx.x & 63) == 0) { rv[threadIdx.x >> 6] = v; ri[threadIdx.x >> 6] = idx; }
    __syncthreads();
    float bv = rv[0];
    int bi = ri[0];
    for (int i = 1; i < MB / 64; i++)
        if (rv[i] > bv || (rv[i] == bv && ri[i] < bi)) { bv = rv[i]; bi = ri[i]; }
    __syncthreads();
    *vmax = bv;
    *found = bi != 0x7fffffff;
    return bi;
}

__device__ __forceinline__ float vx_mb_sum(float v, float *r)
{
    v = vx_wave_sum64(v);
    if ((threadIdx.x & 63) == 0) r[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = r[0];
    for (int i = 1; i < MB / 64; i++) s += r[i];
    __syncthreads();
    return s;
}

__device__ __forceinline__ uint64_t vx_mb_sum_u64(uint64_t v, uint64_t *r)
{
    for (int o = 32; o > 0; o >>= 1) v += vx_shfl_xor_u64(v, o);
    if ((threadIdx.x & 63) == 0) r[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t s = 0;
    for (int i = 0; i < MB / 64; i++) s += r[i];
    __syncthreads();
    return s;
}

// Inverse CDF inside chunk [b, e) given the mass `before` of the chunks
// ahead of it: thread t sums the masses of its contiguous entries, a
// workgroup scan places the threshold, and that thread walks its entries.
// Returns the first index whose inclusive prefix reaches thr (e - 1 if the
// chunk's masses never reach it).
template <typename WF>
__device__ int vx_mb_land(int b, int e, uint64_t before, uint64_t thr, WF W, uint64_t *r, int *res)
{
    const int per = (e - b + MB - 1) / MB;
    const int tb = b + threadIdx.x * per, te = min(tb + per, e);
    uint64_t mine = 0;
    for (int v = tb; v < te; v++) mine += W(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint64_t incl = mine;
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t y = vx_shfl_up_u64(incl, o);
        if (lane >= o) incl += y;
    }
    if (lane == 63) r[wave] = incl;
    if (threadIdx.x == 0) *res = e - 1;
    __syncthreads();
    uint64_t off = before;
    for (int w = 0; w < wave; w++) off += r[w];
    const uint64_t excl = off + incl - mine;
    if (mine && excl < thr && excl + mine >= thr) {
        uint64_t c = excl;
        for (int v = tb; v < te; v++) {
            c += W(v);
            if (c >= thr) { *res = v; break; }
        }
    }
    __syncthreads();
    const int t = *res;
    __syncthreads();
    return t;
}

// Row statistics, chunked: stats[r] = {max, sum exp((l - max)/T), argmax}.
// A chunk keeps its own maximum m_c and sum s_c = sum exp((l - m_c)/T); the
// last workgroup of the row takes the first maximum over the chunks and
// S = sum_c s_c exp((m_c - M)/T) in chunk order.  A row with no value above
// -inf gives argmax 0, max l[0] and (T > 0) sum NaN, as one pass over it
// with that maximum would.  keep (optional, one row): a copy of the row.
template <bool KEEP>
__global__ __launch_bounds__(MB) void vx_stats_mc_kernel(const float *__restrict__ L, int ldl, int V, float T,
                                                         int CH, float *__restrict__ stats, uint64_t *part,
                                                         unsigned *cnt, float *__restrict__ keep)
{
    __shared__ float rv[MB / 64];
    __shared__ int ri[MB / 64];
    __shared__ float sm[MC_MAX_G], ss[MC_MAX_G];
    __shared__ int sa[MC_MAX_G], sf[MC_MAX_G];
    __shared__ int s_last;
    const int r = blockIdx.y, c = blockIdx.x, G = gridDim.x;
    const float *l = L + (size_t)r * ldl;
    const int b0 = c * CH, b1 = min(b0 + CH, V);
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int v0 = b0 + 4 * (int)threadIdx.x; v0 < b1; v0 += 4 * MB) {
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; e++) x[e] = l[min(v0 + e, b1 - 1)];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int v = v0 + e;
            if (KEEP && v < b1) keep[v] = x[e];
            const bool better = (v < b1) & ((x[e] > bv) | ((x[e] == bv) & (v < bi)));
            bv = better ? x[e] : bv;
            bi = better ? v : bi;
        }
    }
    float mc;
    bool fc;
    const int ac = vx_mb_argmax(bv, bi, rv, ri, &mc, &fc);
    float s = 0.0f;
    if (T > 0.0f && fc)
        for (int v = b0 + (int)threadIdx.x; v < b1; v += MB) s += expf((l[v] - mc) / T);
    s = vx_mb_sum(s, rv);
    uint64_t *P = part + ((size_t)r * G + c) * 4;
    if (threadIdx.x == 0) {
        vx_st_coh(P + 0, (uint64_t)__float_as_uint(mc) | ((uint64_t)(fc ? 1 : 0) << 32));
        vx_st_coh(P + 1, (uint64_t)__float_as_uint(s));
        vx_st_coh(P + 2, (uint64_t)(uint32_t)ac);
    }
    if (!vx_arrive_last(&cnt[r], (unsigned)G, &s_last)) return;
    if ((int)threadIdx.x < G) {
        uint64_t *Q = part + ((size_t)r * G + threadIdx.x) * 4;
        const uint64_t w0 = vx_ld_coh(Q + 0);
        sm[threadIdx.x] = __uint_as_float((uint32_t)w0);
        sf[threadIdx.x] = (int)(w0 >> 32);
        ss[threadIdx.x] = __uint_as_float((uint32_t)vx_ld_coh(Q + 1));
        sa[threadIdx.x] = (int)(uint32_t)vx_ld_coh(Q + 2);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float M = -INFINITY;
        int A = 0x7fffffff;
        bool found = false;
        for (int i = 0; i < G; i++)
            if (sf[i] && (sm[i] > M || (sm[i] == M && sa[i] < A))) { M = sm[i]; A = sa[i]; found = true; }
        if (!found) { A = 0; M = l[0]; }
        float S = 0.0f;
        if (T > 0.0f) {
            if (found) {
                for (int i = 0; i < G; i++)
                    if (sf[i]) S += ss[i] * expf((sm[i] - M) / T);
            } else {
                S = __builtin_nanf("");
            }
        }
        stats[r * 3 + 0] = M;
        stats[r * 3 + 1] = S;
        stats[r * 3 + 2] = __int_as_float(A);
    }
    vx_mc_release(&cnt[r]);
}

// The draft draw without a nucleus, chunked (vx_sample_reg_kernel's
// arithmetic): p_v = expf((l_v - max)/T) * inv, inv = 1/(sum + 1e-30) from
// the row statistics, masses W_v = round(p_v * 2^32), token = inverse CDF.
__global__ __launch_bounds__(MB) void vx_draw_mc_kernel(const float *__restrict__ l, int V, float T, int CH,
                                                        const float *__restrict__ stats,
                                                        const float *__restrict__ u, int *__restrict__ token_out,
                                                        float *__restrict__ nuc, uint64_t *part, unsigned *cnt)
{
    __shared__ uint64_t r64[MB / 64];
    __shared__ uint64_t tot[MC_MAX_G];
    __shared__ int s_last, res;
    __shared__ int s_c;
    __shared__ uint64_t s_before, s_S, s_thr;
    const int c = blockIdx.x, G = gridDim.x;
    const float mx = stats[0], sum = stats[1];
    const int am = __float_as_int(stats[2]);
    if (!(T > 0.0f)) {
        if (c == 0 && threadIdx.x == 0) {
            token_out[0] = am;
            nuc[0] = mx; nuc[1] = 0.0f; nuc[2] = -1.0f; nuc[3] = __int_as_float(V - 1);
            nuc[4] = 0.0f; nuc[5] = __int_as_float(am); nuc[6] = 0.0f; nuc[7] = 0.0f;
        }
        return;
    }
    const float inv = 1.0f / (sum + 1e-30f);
    auto W = [&](int v) -> uint64_t { return vx_fixed32(expf((l[v] - mx) / T) * inv); };
    const int b0 = c * CH, b1 = min(b0 + CH, V);
    uint64_t t = 0;
    for (int v = b0 + (int)threadIdx.x; v < b1; v += MB) t += W(v);
    t = vx_mb_sum_u64(t, r64);
    if (threadIdx.x == 0) vx_st_coh(part + c, t);
    if (!vx_arrive_last(cnt, (unsigned)G, &s_last)) return;
    if ((int)threadIdx.x < G) tot[threadIdx.x] = vx_ld_coh(part + threadIdx.x);
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t S = 0;
        for (int i = 0; i < G; i++) S += tot[i];
        s_S = S;
        s_c = -1;
        if (S > 0) {
            const uint64_t thr = vx_threshold(u[0], S);
            uint64_t acc = 0;
            for (int i = 0; i < G; i++) {
                if (acc + tot[i] >= thr) { s_c = i; break; }
                acc += tot[i];
            }
            s_before = acc;
            s_thr = thr;
        }
    }
    __syncthreads();
    int tok = am;
    if (s_c >= 0) {
        const int lb = s_c * CH, le = min(lb + CH, V);
        tok = vx_mb_land(lb, le, s_before, s_thr, W, r64, &res);
    }
    if (threadIdx.x == 0) {
        token_out[0] = tok;
        nuc[0] = mx; nuc[1] = inv; nuc[2] = -1.0f; nuc[3] = __int_as_float(V - 1);
        nuc[4] = (float)((double)s_S / 4294967296.0); nuc[5] = __int_as_float(am);
        nuc[6] = 0.0f; nuc[7] = 0.0f;
    }
    vx_mc_release(cnt);
}

// The verify decision, chunked (vx_accept_kernel's arithmetic).  Every
// workgroup runs the k ratio tests (the first failing draft is the decided
// row j), then sums the fixed-point masses of its chunk of row j -- the
// residual max(0, p - q) at a rejection, p for the bonus draw -- and, at a
// rejection, the chunk's first maximum of the residual (the draw when the
// residual has no mass).  The last workgroup places the threshold.
__global__ __launch_bounds__(MB) void vx_accept_mc_kernel(const float *__restrict__ L, int ldl, int V,
                                                          const float *__restrict__ stats,
                                                          const float *__restrict__ D, int ldd, int Vd,
                                                          const float *__restrict__ nuc,
                                                          const int *__restrict__ drafts, int k, float T,
                                                          const float *__restrict__ u, int *__restrict__ out, int CH,
                                                          uint64_t *part, unsigned *cnt)
{
    __shared__ float rv[MB / 64];
    __shared__ int ri[MB / 64];
    __shared__ uint64_t r64[MB / 64];
    __shared__ uint64_t tot[MC_MAX_G];
    __shared__ float cmv[MC_MAX_G];
    __shared__ int cmi[MC_MAX_G];
    __shared__ int s_last, res, s_j, s_c;
    __shared__ uint64_t s_before, s_thr;
    const int c = blockIdx.x, G = gridDim.x;
    if (!(T > 0.0f)) {
        // greedy: accept d_j while it is the first argmax of L_j
        if (c == 0 && threadIdx.x == 0) {
            int j = 0;
            for (; j < k; j++) {
                const int a = __float_as_int(stats[j * 3 + 2]);
                out[2 + j] = a;
                if (a != drafts[j]) break;
            }
            if (j == k) out[2 + k] = __float_as_int(stats[k * 3 + 2]);
            out[0] = j < k ? j + 1 : k + 1;
            out[1] = j;
        }
        return;
    }
    if (threadIdx.x < 64) {
        // ratio tests of the drafts on parallel lanes; the first failing one
        // is where the sequential scan (src/speculative.c:199-200) stops
        const int lane = threadIdx.x;
        bool rej = true;
        if (lane < k) {
            const float *lj = L + (size_t)lane * ldl;
            const float mx = stats[lane * 3 + 0], inv = 1.0f / (stats[lane * 3 + 1] + 1e-30f);
            const int d = drafts[lane];
            const float pt = (d >= 0 && d < V) ? expf((lj[d] - mx) / T) * inv : 0.0f;
            const float qd = (d >= 0 && d < Vd) ? vx_draft_q(D + (size_t)lane * ldd, nuc + lane * 8, d, T) : 0.0f;
            const float alpha = fminf(1.0f, pt / fmaxf(qd, 1e-10f));
            rej = !(u[lane] < alpha);
        }
        const uint64_t bal = __ballot(rej);
        int j = bal ? __builtin_ctzll(bal) : 64;
        if (lane == 0) {
            for (; j < k; j++) {   // only k > 64
                const float *lj = L + (size_t)j * ldl;
                const float mx = stats[j * 3 + 0], inv = 1.0f / (stats[j * 3 + 1] + 1e-30f);
                const int d = drafts[j];
                const float pt = (d >= 0 && d < V) ? expf((lj[d] - mx) / T) * inv : 0.0f;
                const float qd = (d >= 0 && d < Vd) ? vx_draft_q(D + (size_t)j * ldd, nuc + j * 8, d, T) : 0.0f;
                const float alpha = fminf(1.0f, pt / fmaxf(qd, 1e-10f));
                if (!(u[j] < alpha)) break;
            }
            s_j = min(j, k);
        }
    }
    __syncthreads();
    const int j = s_j;
    const bool resample = j < k;
    const float *lj = L + (size_t)j * ldl;
    const float mx = stats[j * 3 + 0], inv = 1.0f / (stats[j * 3 + 1] + 1e-30f);
    const float *dj = D + (size_t)min(j, k - 1) * ldd;
    const vx_nuc nq = vx_nuc_load(nuc + min(j, k - 1) * 8);
    auto X = [&](int v) -> float {
        const float p = expf((lj[v] - mx) / T) * inv;
        if (!resample) return p;
        const float q = v < Vd ? vx_draft_q_of(dj[v], nq, v, T) : 0.0f;
        return fmaxf(0.0f, p - q);
    };
    auto W = [&](int v) -> uint64_t { return vx_fixed32(X(v)); };
    const int b0 = c * CH, b1 = min(b0 + CH, V);
    uint64_t t = 0;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int v = b0 + (int)threadIdx.x; v < b1; v += MB) {
        const float x = X(v);
        t += vx_fixed32(x);
        const bool better = (x > bv) | ((x == bv) & (v < bi));
        bv = better ? x : bv;
        bi = better ? v : bi;
    }
    t = vx_mb_sum_u64(t, r64);
    float cv = -INFINITY;
    bool cf = false;
    int ci = 0x7fffffff;
    if (resample) ci = vx_mb_argmax(bv, bi, rv, ri, &cv, &cf);
    uint64_t *P = part + (size_t)c * 3;
    if (threadIdx.x == 0) {
        vx_st_coh(P + 0, t);
        vx_st_coh(P + 1, (uint64_t)__float_as_uint(cv));
        vx_st_coh(P + 2, (uint64_t)(uint32_t)ci);
    }
    if (!vx_arrive_last(cnt, (unsigned)G, &s_last)) return;
    if ((int)threadIdx.x < G) {
        uint64_t *Q = part + (size_t)threadIdx.x * 3;
        tot[threadIdx.x] = vx_ld_coh(Q + 0);
        cmv[threadIdx.x] = __uint_as_float((uint32_t)vx_ld_coh(Q + 1));
        cmi[threadIdx.x] = (int)(uint32_t)vx_ld_coh(Q + 2);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t S = 0;
        for (int i = 0; i < G; i++) S += tot[i];
        s_c = -1;
        if (S > 0) {
            const uint64_t thr = vx_threshold(u[k], S);
            uint64_t acc = 0;
            for (int i = 0; i < G; i++) {
                if (acc + tot[i] >= thr) { s_c = i; break; }
                acc += tot[i];
            }
            s_before = acc;
            s_thr = thr;
        }
    }
    __syncthreads();
    int tok;
    if (s_c >= 0) {
        const int lb = s_c * CH, le = min(lb + CH, V);
        tok = vx_mb_land(lb, le, s_before, s_thr, W, r64, &res);
    } else if (resample) {
        // no residual mass: the residual's first maximum over the chunks
        float M = -INFINITY;
        int A = 0x7fffffff;
        for (int i = 0; i < G; i++)
            if (cmv[i] > M || (cmv[i] == M && cmi[i] < A)) { M = cmv[i]; A = cmi[i]; }
        tok = A == 0x7fffffff ? 0 : A;
    } else {
        tok = __float_as_int(stats[j * 3 + 2]);
    }
    if (threadIdx.x == 0) {
        for (int i = 0; i < j; i++) out[2 + i] = drafts[i];
        out[2 + j] = tok;
        out[0] = j + 1;
        out[1] = j;
    }
    vx_mc_release(cnt);
}

// Workspace: partials [max_rows + 2][MC_MAX_G][4] u64 -- regions 0 ..
// max_rows-1 for the rows of the statistics, region max_rows for the draw,
// max_rows + 1 for the decision -- then counters [max_rows + 2] in the same
// order, then 16 floats of the sampler's row statistics.
extern "C" int vxh_vocab_ws_alloc(vxh_vocab_ws *ws, int max_rows)
{
    if (!ws || max_rows < 1 || max_rows > 1024) return vxh_fail(VXH_ERR_PARAM, "vocab_ws_alloc: max_rows %d", max_rows);
    memset(ws, 0, sizeof(*ws));
    const size_t part = ((size_t)max_rows + 2) * MC_MAX_G * 4 * sizeof(uint64_t);
    const size_t cnt = ((size_t)max_rows + 2) * sizeof(unsigned);
    const size_t bytes = part + cnt + 16 * sizeof(float);
    void *p = nullptr;
    int rc = vxh_malloc(&p, bytes);
    if (rc) return rc;
    VXH_CHECK(hipMemset(p, 0, bytes));
    VXH_CHECK(hipDeviceSynchronize());
    ws->part = p;
    ws->cnt = (unsigned *)((char *)p + part);
    ws->stats = (float *)((char *)p + part + cnt);
    ws->max_rows = max_rows;
    return VXH_OK;
}

extern "C" void vxh_vocab_ws_free(vxh_vocab_ws *ws)
{
    if (!ws) return;
    vxh_free(ws->part);
    memset(ws, 0, sizeof(*ws));
}

static int vx_ws_check(const vxh_vocab_ws *ws, int rows, const char *what)
{
    if (!ws || !ws->part || rows > ws->max_rows)
        return vxh_fail(VXH_ERR_PARAM, "%s: workspace for %d rows, %d needed", what, ws ? ws->max_rows : 0, rows);
    return VXH_OK;
}

extern "C" int vxh_row_stats_mc(const float *L, int ldl, int R, int V, float T, float *stats, vxh_vocab_ws *ws,
                                vxh_stream s)
{
    if (R <= 0) return VXH_OK;
    if (V <= 0 || ldl < V) return vxh_fail(VXH_ERR_PARAM, "row_stats_mc: V %d ldl %d", V, ldl);
    int rc = vx_ws_check(ws, R, "row_stats_mc");
    if (rc) return rc;
    const int CH = vx_mc_chunk(V), G = (V + CH - 1) / CH;
    vx_stats_mc_kernel<false><<<dim3(G, R), MB, 0, vxh_hs(s)>>>(L, ldl, V, T, CH, stats, (uint64_t *)ws->part,
                                                                ws->cnt, nullptr);
    VXH_LAUNCHED();
    return VXH_OK;
}

extern "C" int vxh_sample_keep_mc(const float *l, int V, float T, float top_p, const float *u_dev, int *token_out,
                                  float *nuc, float *keep, vxh_vocab_ws *ws, vxh_stream s)
{
    if (V <= 0) return vxh_fail(VXH_ERR_PARAM, "sample_mc: V %d", V);
    // the nucleus sampler, and rows that the one-workgroup register sampler
    // holds (one launch; measured on MI355X at V = 32000: 18.4 us against
    // 13.6 + 8.4 us for the two chunked launches, whose device-coherent round
    // trips outweigh the exponentials they spread)
    if (top_p < 1.0f || V <= SB * SE) return vxh_sample_keep(l, V, T, top_p, u_dev, token_out, nuc, keep, s);
    int rc = vx_ws_check(ws, 1, "sample_mc");
    if (rc) return rc;
    if (keep == l) keep = nullptr;
    const int CH = vx_mc_chunk(V), G = (V + CH - 1) / CH;
    uint64_t *part = (uint64_t *)ws->part;
    // row statistics in row 0's slots, the draw's chunk totals in the region after them
    if (keep)
        vx_stats_mc_kernel<true><<<dim3(G, 1), MB, 0, vxh_hs(s)>>>(l, V, V, T, CH, ws->stats, part, ws->cnt, keep);
    else
        vx_stats_mc_kernel<false><<<dim3(G, 1), MB, 0, vxh_hs(s)>>>(l, V, V, T, CH, ws->stats, part, ws->cnt,
                                                                     nullptr);
    VXH_LAUNCHED();
    vx_draw_mc_kernel<<<G, MB, 0, vxh_hs(s)>>>(l, V, T, CH, ws->stats, u_dev, token_out, nuc,
                                               part + (size_t)ws->max_rows * MC_MAX_G * 4,
                                               ws->cnt + ws->max_rows);
    VXH_LAUNCHED();
    return VXH_OK;
}

extern "C" int vxh_accept_mc(const float *L, int ldl, int V, const float *stats, const float *D, int ldd, int Vd,
                             const float *nuc, const int *drafts, int k, float T, const float *u, int *out,
                             vxh_vocab_ws *ws, vxh_stream s)
{
    if (k < 0 || V <= 0) return vxh_fail(VXH_ERR_PARAM, "accept_mc: k %d V %d", k, V);
    if (T > 0.0f && k == 0) return vxh_accept(L, ldl, V, stats, D, ldd, Vd, nuc, drafts, k, T, u, out, s);
    int rc = vx_ws_check(ws, 1, "accept_mc");
    if (rc) return rc;
    const int CH = vx_mc_chunk(V), G = (V + CH - 1) / CH;
    vx_accept_mc_kernel<<<G, MB, 0, vxh_hs(s)>>>(L, ldl, V, stats, D, ldd, Vd, nuc, drafts, k, T, u, out, CH,
                                                 (uint64_t *)ws->part + ((size_t)ws->max_rows + 1) * MC_MAX_G * 4,
                                                 ws->cnt + ws->max_rows + 1);
    VXH_LAUNCHED();
    return VXH_OK;
}
