/*
 * vxh.h -- the thin C ABI between the engine's C host code (model.c,
 * speculative.c, quantize.c) and its hand-written gfx950 HIP kernels.
 *
 * Plain C: device memory is passed as void* / float* device addresses, sizes
 * as int / size_t, streams as an opaque handle.  No HIP or torch type appears
 * here.  Every entry point returns VXH_OK (0) or a negative VXH_ERR_* code;
 * vxh_last_error() describes the last failure of the calling thread.
 *
 * The reference engine has no device layer; these entry points replace the
 * bodies of its CPU kernels (see the per-group comments for which).
 */
#ifndef VXH_H
#define VXH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    VXH_OK = 0,
    VXH_ERR_NODEVICE = -1,
    VXH_ERR_ALLOC = -2,
    VXH_ERR_PARAM = -3,
    VXH_ERR_LAUNCH = -4,
    VXH_ERR_UNSUPPORTED = -5,
};

typedef struct vxh_stream_s *vxh_stream;   /* a HIP stream; NULL = the default stream */

/* ---- runtime ------------------------------------------------------------ */
int vxh_init(void);                               /* idempotent; selects device 0 */
const char *vxh_last_error(void);
/* Records a printf-style message for vxh_last_error() and returns code. */
int vxh_set_error(int code, const char *fmt, ...);
int vxh_device_name(char *buf, int len);
int vxh_malloc(void **dptr, size_t bytes);
int vxh_free(void *dptr);
int vxh_upload(void *dst, const void *src, size_t bytes, vxh_stream s);
int vxh_download(void *dst, const void *src, size_t bytes, vxh_stream s);
int vxh_copy(void *dst, const void *src, size_t bytes, vxh_stream s);
/* Page-locked host memory (hipHostMalloc), the source vxh_upload_async needs. */
int vxh_host_alloc(void **p, size_t bytes);
int vxh_host_free(void *p);
/* Host -> device copy enqueued on s without waiting for it: src must be
 * page-locked (vxh_host_alloc) and keep its contents until the stream has
 * run the copy (a later vxh_stream_sync, or a synchronous vxh_download on s). */
int vxh_upload_async(void *dst, const void *src, size_t bytes, vxh_stream s);
int vxh_fill_f32(float *dst, float value, size_t n, vxh_stream s);   /* kernel, graph-safe */
int vxh_stream_create(vxh_stream *s);
int vxh_stream_destroy(vxh_stream s);
int vxh_stream_sync(vxh_stream s);
int vxh_device_sync(void);                         /* waits for every stream */

/* Events on a stream, for timing the launches recorded between them. */
typedef struct vxh_event_s *vxh_event;
int vxh_event_create(vxh_event *e);
int vxh_event_destroy(vxh_event e);
int vxh_event_record(vxh_event e, vxh_stream s);
int vxh_event_elapsed_ms(vxh_event start, vxh_event stop, float *ms);

/* Graph capture of a stream's launches (no memset nodes are ever recorded). */
typedef struct vxh_graph_s *vxh_graph;
int vxh_capture_begin(vxh_stream s);
int vxh_capture_end(vxh_stream s, vxh_graph *g);
int vxh_graph_launch(vxh_graph g, vxh_stream s);
int vxh_graph_destroy(vxh_graph g);

/* ---- quantised matrices in HBM --------------------------------------------
 * Replaces the row-major GGUF block arrays the reference's GEMV kernels read
 * (src/simd/avx2.c:324, src/quantize.c:738).  Rows are grouped in tiles of
 * 32; within a tile the data is stored in the order one wavefront consumes
 * it, so every weight load of a wavefront is a contiguous 1 KiB:
 *
 *   Q4_0  qs: [tile][block pair p][lane 64][16 B]   lane l = row (l%32) of the
 *             tile, half h = l/32; its 16 B are bytes 8h..8h+7 of blocks 2p
 *             and 2p+1 with the nibbles of each dword permuted so the
 *             in-register unpack yields elements in natural order.
 *   Q8_0  qs: [tile][block b][lane 64][16 B]        bytes 16h..16h+15 of block
 *             b (bytes permuted within each dword).
 *   both  d : [tile][block pair p][row 32] -> (d[2p], d[2p+1]) as two fp16.
 *
 * Byte count equals GGUF's (18 or 34 bytes per 32 weights) apart from padding
 * rows to a multiple of 32 and blocks to an even count (padding has d = 0).
 *
 *   F32   qs: [row][n_pairs * 64] fp32, zero past n_cols and the logical rows;
 *             d unused.  GEMMs read it through vxh_gemm_acc only (exact,
 *             non-AVX2 panels); gathers copy rows unscaled.
 *
 * Q4_0 and Q8_0 matrices also hold a copy in 64-row tiles for the GEMMs of
 * 5..16 rows (the weights are the B operand of a 16x16x32 MFMA, one block
 * per weight row and instruction); nb = n_cols/32 blocks, lane l = 16G + n:
 *   Q4_0  tq: [tile][block][lane 64][4 dwords]  dword g = bytes 4G..4G+3 of
 *             the block of row 64 tile + 16g + n (nibbles permuted as above).
 *   Q8_0  tq: [tile][block][half j][lane 64][4 dwords]  dwords 2c, 2c+1 =
 *             bytes 8G..8G+7 of row 64 tile + 16(2j + c) + n (permuted).
 *   both  td: [tile][block][n 16][g 4] fp16 scale of row 64 tile + 16g + n.
 * Rows past n_rows read as zeros; the copy adds 18 (34) bytes per 32 weights
 * (HBM is not the constraint: 288 GB per MI355X). */
typedef struct {
    int type;          /* 2 = Q4_0, 8 = Q8_0, 0 = F32 (vx_type / GGML ids)  */
    int n_rows;        /* physical rows, a multiple of 32                     */
    int n_cols;        /* K, a multiple of 32                                 */
    int n_pairs;       /* ceil(K/64): block pairs per row                     */
    void *qs;          /* device                                              */
    void *d;           /* device                                              */
    int cached;        /* 0: the GEMMs stream qs with non-temporal loads (the
                        * default: a matrix read once per forward should not
                        * evict what the next launches reuse); nonzero: plain
                        * loads, so the matrix may stay in the caches between
                        * forwards (vxh_qmat_alloc sets 0; the 64-row copy is
                        * always streamed)                                  */
    void *tq;          /* device, 64-row tiled copy (Q4_0/Q8_0; NULL for F32) */
    void *td;          /* device                                              */
} vxh_qmat;

int vxh_qmat_alloc(vxh_qmat *m, int type, int n_rows, int n_cols);
int vxh_qmat_free(vxh_qmat *m);
/* Copy n_rows GGUF rows (n_cols/32 blocks each, host or device memory per
 * `src_on_device`) into the tiled layout.  Logical row r lands on physical
 * row (r / group) * group_stride + row_offset + r % group; group = n_rows,
 * group_stride = 0 is a plain copy at row_offset. */
int vxh_qmat_set_rows(vxh_qmat *m, const void *src, int src_on_device, int n_rows, int group,
                      int group_stride, int row_offset, vxh_stream s);
/* Inverse of vxh_qmat_set_rows: rebuild n_rows GGUF rows into host memory. */
int vxh_qmat_get_rows(const vxh_qmat *m, void *host_dst, int n_rows, int group,
                      int group_stride, int row_offset, vxh_stream s);
/* Fill n_rows x n_cols of GGUF blocks on the device with seeded weights
 * N(0, std^2) (Box-Muller on a splitmix64 counter stream keyed by seed) run
 * through the Q4_0 writer of the reference (src/quantize.c:88-114) or, for
 * Q8_0, d = amax/127 rounded to fp16 and q = round(x/d). */
int vxh_synth_blocks(void *dev_blocks, int type, int n_rows, int n_cols, uint64_t seed,
                     float std, vxh_stream s);
/* Gather rows of a tiled matrix as fp32: out[i][:] = scale * dequant(row
 * ids[i]) for i < n (ids read from device memory; out-of-range ids -> zeros;
 * F32 rows are copied without the scale, as the reference copies them).
 * Replaces the embedding lookup of src/model.c:454-500. */
int vxh_qmat_gather_rows(const vxh_qmat *m, const int *dev_ids, int n, float scale,
                         float *out, int ld_out, vxh_stream s);
/* The same gather, and the n_clr doubles at clr zeroed by the same launch
 * (a forward's accumulators that no kernel reads during it).  No counterpart
 * in the reference. */
int vxh_qmat_gather_rows_clear(const vxh_qmat *m, const int *dev_ids, int n, float scale,
                               float *out, int ld_out, double *clr, long n_clr, vxh_stream s);

/* Longest row a panel or a row kernel takes (elements). */
#define VXH_MAX_K 24576

/* ---- activation panels -----------------------------------------------------
 * A GEMM input of M rows (1 <= M <= 16) x K, as the fp16 hi/lo operand the
 * MFMA kernel reads from LDS: x' = hi + lo with hi = fp16(x'), lo =
 * fp16(x' - hi), x' = x * 2^-e_m (power-of-two row scale, exact).  Layout [block][mfma s][half h][slot][8 x fp16], slot m =
 * hi of row m, slot M+m = lo of row m.  AVX2-lane panels hold w_t*x_t (w_t =
 * 2 when t%8 >= 4) and a per-(block,row) correction, see vxh_prep_panel. */
typedef struct {
    void *data;        /* device, vxh_panel_bytes(M, K)                       */
    float *corr;       /* device, [K/32][M] (AVX2-lane panels)                */
    float *rscale;     /* device, [M]: row m of the panel holds x * 2^-e_m and
                          rscale[m] = 2^e_m is applied to the GEMM output, so
                          max |x * 2^-e_m| < 1 whatever the magnitude of x */
    float *xs;         /* device, fp32 copy for the dot-product path          */
    int M, K;
    int avx2;          /* 1: lane-pattern weights and corrections             */
    int rs_ld;         /* 0: one scale per row; n > 0: one per 1024 columns,
                          rscale[m * n + k / 1024] (vxh_swiglu_panel_norm)    */
} vxh_panel;

size_t vxh_panel_bytes(int M, int K);
int vxh_panel_alloc(vxh_panel *p, int max_M, int K);
int vxh_panel_free(vxh_panel *p);
/* Build a panel from fp32 rows x[M][ldx].  avx2 = 1 applies the lane
 * pattern of vx_gemv_q4_0_avx2 (src/simd/avx2.c:336-363): per block the
 * correction is sum of x at offsets 8..11, 16..19, 24..27, 32..35, where
 * offsets >= K read tail[m][0..3] (tail may be NULL: zeros). */
int vxh_prep_panel(vxh_panel *p, const float *x, int ldx, int M, int K, int avx2,
                   const float *tail, int ld_tail, vxh_stream s);
/* Fused RMSNorm + panel: xn[m] = w .* x[m] / sqrt(mean(x[m]^2) + 1e-5)
 * (src/tensor.c:128-142; w NULL = ones, src/model.c:253-258), written as a
 * panel; xn (fp32) is also stored when xn_out != NULL.  In AVX2 mode the
 * 4-float tail of row m is tail[m][0..3] (NULL: zeros). */
int vxh_rmsnorm_panel(const float *x, int ldx, int M, int K, const float *w, int avx2,
                      const float *tail, int ld_tail, vxh_panel *p, float *xn_out, int ld_xn,
                      vxh_stream s);
/* Residual add + RMSNorm + panel: x[m] += (float)acc[m] (the pending output
 * of a residual GEMM, src/model.c:546, :589; acc is cleared), then as
 * vxh_rmsnorm_panel on the updated x.  tail_self = 1 takes the AVX2 tail from
 * the updated x[m][0..3] (src/model.c:425-435). */
int vxh_resid_rmsnorm_panel(float *x, int ldx, double *acc, int ld_acc, int M, int K,
                            const float *w, int avx2, int tail_self, vxh_panel *p, float *xn_out,
                            int ld_xn, vxh_stream s);
/* SwiGLU + panel: h[m][i] = |silu(g)| < thr ? 0 : silu(g) * u (src/model.c:
 * 582-585, :169-201) for i < F, with g, u the fp32 roundings of the gate/up
 * accumulator (tile-interleaved: physical row 32(i/16) + i%16 is gate row i,
 * 16 rows further is up row i; cleared after reading), written as a panel
 * (and to h_out when not NULL).  The AVX2 tail of h is zeros. */
int vxh_swiglu_panel(double *acc, int ld_acc, int M, int F, float thr, int avx2, vxh_panel *p,
                     float *h_out, int ldh, vxh_stream s);
/* vxh_swiglu_panel on the sums of a prologue GEMM whose RMSNorm is still
 * pending: g and u are the fp32 roundings of the gate/up sums times
 * 1/sqrt(ss_in[m]/ss_K + 1e-5) (ss_in NULL: times 1), exactly as the
 * VXH_PRO_SWIGLU prologue forms them; the launch also zeroes n_clear doubles
 * at clear.  One workgroup per (row, 1024 columns), each with its own
 * power-of-two scale (p->rs_ld = chunks per row).  Exact-Q4_0 panel (no
 * AVX2 tail). */
int vxh_swiglu_panel_norm(double *acc, int ld_acc, int M, int F, float thr, const double *ss_in,
                          int ss_K, double *clear, size_t n_clear, vxh_panel *p, vxh_stream s);
/* The same with two events (either may be NULL) that the dispatch records
 * around the kernel, for kernel-execution timing. */
int vxh_swiglu_panel_norm_timed(double *acc, int ld_acc, int M, int F, float thr, const double *ss_in,
                                int ss_K, double *clear, size_t n_clear, vxh_panel *p, vxh_event e0,
                                vxh_event e1, vxh_stream s);

/* ---- skinny-M dequant GEMM ---------------------------------------------------
 * Y[m][n] = sum_k X[m][k] * W[n][k] for m < M, n < N, W quantised, X a panel.
 * Replaces vx_gemv_q4_0_avx2 / vx_gemv_q4_0 / dequantize+vx_gemv_f32
 * (src/model.c:203-245) for M rows at once.
 *
 * vxh_gemm_acc adds scale * Y into an fp64 accumulator acc[M][ld_acc] for
 * n < n_out.  The K range is split over workgroups whose fp32 partial sums are
 * added with fp64 atomics; they add exactly, so the result is independent of
 * arrival order.  gate != NULL leaves acc[m][n] untouched where |gate[m][n]|
 * < thr (src/model.c:169-201).  The consumers below (and vxh_rope_kv,
 * vxh_resid_rmsnorm_panel, vxh_swiglu_panel) round the accumulator to fp32
 * and clear it, so an accumulator that starts zeroed stays zeroed between
 * uses. */
/* path: VXH_PATH_AUTO and VXH_PATH_MFMA take the MFMA kernel; VXH_PATH_DOT
 * the same GEMM with v_dot2_f32_f16 per activation row instead of MFMA
 * (exact Q4_0/Q8_0 panels; kept to measure the MFMA kernel against). */
enum { VXH_PATH_AUTO = 0, VXH_PATH_MFMA = 1, VXH_PATH_DOT = 2 };

int vxh_gemm_acc(const vxh_qmat *W, const vxh_panel *X, int M, double *acc, int ld_acc,
                 int n_out, float scale, const float *gate, int ld_gate, float thr, int path,
                 vxh_stream s);
/* vxh_gemm_acc with the kernel's execution bracketed by two events that the
 * dispatch itself records (start and end of the kernel, no extra packets):
 * vxh_event_elapsed_ms(start, stop) is the kernel's own duration. */
int vxh_gemm_acc_timed(const vxh_qmat *W, const vxh_panel *X, int M, double *acc, int ld_acc,
                       int n_out, float scale, const float *gate, int ld_gate, float thr, int path,
                       vxh_event start, vxh_event stop, vxh_stream s);
/* y[m][i] = (r ? r[m][i] : 0) + (float)acc[m][i] for i < n; acc cleared. */
int vxh_acc_store(double *acc, int ld_acc, int M, int n, float *y, int ldy, const float *r,
                  int ldr, vxh_stream s);
/* h[m][i] = SwiGLU of the tile-interleaved gate/up accumulator (see
 * vxh_swiglu_panel) for i < F; acc cleared. */
int vxh_acc_swiglu(double *acc, int ld_acc, int M, int F, float thr, float *h, int ldh,
                   vxh_stream s);

/* One-call GEMM with an fp32 result: vxh_gemm_acc into the workspace's
 * accumulator followed by the epilogue: */
enum {
    VXH_EPI_STORE = 0,    /* y = scale*acc                                         */
    VXH_EPI_RESID = 1,    /* y = r + scale*acc          (residual add, model.c:546) */
    VXH_EPI_GATE = 2,     /* y = |g| < thr ? 0 : scale*acc   (src/model.c:169-201)  */
    VXH_EPI_SWIGLU = 3,   /* rows interleaved 16 gate / 16 up per tile:
                             h = |silu(g)| < thr ? 0 : silu(g)*u (src/model.c:582-585) */
};
typedef struct {
    int kind;
    float *y; int ldy;             /* output rows                                   */
    const float *r; int ldr;       /* residual (RESID) or gate (GATE)               */
    float thr;
    float scale;                   /* output multiplier (synthetic weight scale)     */
    int n_out;                     /* logical output columns (N, or F for SWIGLU)    */
} vxh_epilogue;

/* Per-stream scratch: the fp64 GEMM accumulator of vxh_gemm (allocated
 * zeroed, left zeroed by every call) and the attention partials. */
typedef struct {
    double *acc;
    size_t acc_elems;
    float *part;
    size_t part_floats;
} vxh_workspace;
int vxh_workspace_alloc(vxh_workspace *w, size_t acc_elems, size_t part_floats);
int vxh_workspace_free(vxh_workspace *w);
/* Accumulator elements vxh_gemm needs for an n_rows matrix and M rows. */
size_t vxh_gemm_workspace_elems(int n_rows, int M);

int vxh_gemm(const vxh_qmat *W, const vxh_panel *X, int M, const vxh_epilogue *ep,
             vxh_workspace *ws, int path, vxh_stream s);

/* vxh_gemm without a workspace and without any allocation: no counterpart in
 * the reference; for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The fp64 accumulator is a static device array of VXH_NOALLOC_ACC_ELEMS
 * doubles (4 MiB) that each GPU the library runs on holds until the process
 * ends; calls needing more (vxh_gemm_workspace_elems(W->n_rows, M) above it)
 * fail with VXH_ERR_PARAM before launching anything.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams,
 * other threads) race and must not be issued.  The part a call uses is
 * cleared by a fill kernel at its start.  Same results as vxh_gemm. */
#define VXH_NOALLOC_ACC_ELEMS (1 << 19)
int vxh_gemm_noalloc(const vxh_qmat *W, const vxh_panel *X, int M, const vxh_epilogue *ep, int path,
                     vxh_stream s);

/* ---- GEMM that builds its own panel ------------------------------------------
 * vxh_gemm_acc_timed whose workgroups build their K slice of the panel from
 * the source rows, so that no row kernel runs between two GEMMs of the
 * forward (src/model.c:514-594).  K = W's columns.
 *   VXH_PRO_ROWS    a = w .* x                          (w NULL: a = x)
 *   VXH_PRO_RESID   t = x + (float)src, a = w .* t; t is stored to x_out
 *                   (the residual add, src/model.c:546, :589)
 *   VXH_PRO_SWIGLU  a = |silu(g)| < thr ? 0 : silu(g) * u (src/model.c:582-585),
 *                   g, u the fp32 roundings of the tile-interleaved gate/up
 *                   sums in src (layout as vxh_swiglu_panel) times
 *                   1/sqrt(ss_in[m]/ss_K + 1e-5) (ss_in NULL: times 1)
 *   VXH_PRO_ATTN    a = the attention rows combined from the per-chunk
 *                   partials of vxh_attention_parts_qkv (part, n_chunks,
 *                   n_heads, n_kv_heads, head_dim as that call; K =
 *                   n_heads * head_dim; M <= VXH_PRO_ATTN_MAX_ROWS)
 * ROWS and RESID add sum x^2 (resp. t^2) of each row into ss[m] when ss is
 * not NULL, so that the RMSNorm (src/tensor.c:128-142) is applied to the
 * product instead of the input: W (w .* t) / sqrt(ss/K + 1e-5), by the
 * product's consumer (vxh_rope_kv_norm, vxh_acc_store_norm, a SWIGLU
 * prologue).  src is read, not cleared.  The n_clear doubles at clear (an
 * accumulator that this launch neither reads nor writes) are zeroed.
 * x, src, w, x_out: 16-byte aligned, ldx and ld_xout multiples of 4, ld_src
 * even; x_out must not overlap x; acc must not overlap src or clear. */
enum { VXH_PRO_ROWS = 1, VXH_PRO_RESID = 2, VXH_PRO_SWIGLU = 3, VXH_PRO_ATTN = 4 };
#define VXH_PRO_ATTN_MAX_ROWS 2
typedef struct {
    int kind;
    const float *x; int ldx;        /* ROWS, RESID: input rows [M][ldx]                 */
    const double *src; int ld_src;  /* RESID: pending GEMM sums; SWIGLU: gate/up sums    */
    const float *w;                 /* ROWS, RESID: RMSNorm weight [K] or NULL           */
    float *x_out; int ld_xout;      /* RESID: updated residual rows or NULL              */
    double *ss;                     /* ROWS, RESID: [M] sums of squares are added, or NULL */
    const double *ss_in; int ss_K;  /* SWIGLU: deferred RMSNorm of the gate/up product   */
    float thr;                      /* SWIGLU: gate-skip threshold                       */
    double *clear; size_t n_clear;  /* zeroed by the launch                              */
    const float *part; int n_chunks;/* ATTN: attention partials and their chunk count    */
    int n_heads, n_kv_heads, head_dim;
} vxh_pro;
int vxh_gemm_pro(const vxh_qmat *W, int M, const vxh_pro *p, double *acc, int ld_acc, int n_out,
                 float scale, vxh_event start, vxh_event stop, vxh_stream s);
/* y[m][i] = (float)acc[m][i] * 1/sqrt(ss[m]/ss_K + 1e-5) for i < n (the
 * RMSNorm of a VXH_PRO_ROWS/RESID product, 0 where the rms is below 1e-10 as
 * src/tensor.c:134-139); acc cleared. */
int vxh_acc_store_norm(double *acc, int ld_acc, int M, int n, float *y, int ldy, const double *ss,
                       int ss_K, vxh_stream s);

/* ---- prompt prefill at large M ---------------------------------------------------
 * The reference runs a prompt one token per forward (src/speculative.c:100-107,
 * src/model.c:450-616); these run a chunk of prompt rows as one batch.
 *
 * vxh_rows_panel: fp32 rows X[M][ldx] (16-byte aligned, ldx % 4 == 0,
 * K % 32 == 0) converted once into the large-M GEMM's activation operand:
 * each row scaled by a power of two 2^-e (e from its largest magnitude),
 * fp16 hi + lo of every scaled element, laid out as the GEMM's LDS stages
 * ([64-row group][64-column pair][16 KiB]), then the M row factors 2^e;
 * vxh_rows_panel_bytes(M, K) bytes.
 *
 * vxh_gemm_rows: Y[m][n] = (R ? R[m][n] : 0) + scale * sum_k X[m][k] W[n][k]
 * for m < M (any M >= 1), n < n_out, from the rows panel of X (built with
 * K = W->n_cols).  Compute-bound MFMA tiles of 64 rows x 128 columns;
 * weights enter as the exact fp16 pair d*q = hi + lo and the activations as
 * fp16 hi + lo, summed over all of K in fp32 (within the fp32 GEMV's
 * rounding of src/quantize.c:728-750).  Y may alias R. */
size_t vxh_rows_panel_bytes(int M, int K);
int vxh_rows_panel(const float *X, int ldx, int M, int K, void *px, vxh_stream s);
int vxh_gemm_rows(const vxh_qmat *W, const void *px, int M, float *Y, int ldy, int n_out,
                  const float *R, int ldr, float scale, vxh_stream s);
/* vxh_rope_kv for fp32 q|k|v rows qkv[M][ld_qkv] (no deferred norm, not
 * cleared): rotated q to q_out[M][ldq], k and v into the cache rows. */
int vxh_rope_kv_rows(const float *qkv, int ld_qkv, int M, int n_past, int n_ctx, int n_heads,
                     int n_kv_heads, int head_dim, const float *bq, const float *bk, const float *bv,
                     const float *cos_tab, const float *sin_tab, int n_pos, float *q_out, int ldq,
                     float *k_cache_layer, float *v_cache_layer, vxh_stream s);
/* h[m][i] = |silu(g)| < thr ? 0 : silu(g) * u for the tile-interleaved gate/up
 * rows gu[M][ld_gu] (gate at 32(i/16) + i%16, up 16 further; src/model.c:582-585). */
int vxh_swiglu_rows(const float *gu, int ld_gu, int M, int F, float thr, float *h, int ldh, vxh_stream s);

/* ---- attention block ---------------------------------------------------------
 * RoPE + KV write (src/tensor.c:173-271 portable branch, src/model.c:291-296):
 * qkv[m] = [q | k | v] (+ optional F32 biases), read from the fp64 GEMM
 * accumulator (rounded to fp32, then cleared).  Row m sits at position
 * pos_m = min(n_past + m, n_ctx - 1), rotated at rope position
 * rope_pos_m = n_past + m; cos/sin come from a host-built table
 * [n_pos][head_dim/2] (cosf/sinf of pos * (1/powf(theta, 2i/hd))).  Writes the
 * rotated q to q_out[m] and k, v to the layer's cache rows pos_m. */
int vxh_rope_kv(double *qkv, int ld_qkv, int M, int n_past, int n_ctx, int n_heads,
                int n_kv_heads, int head_dim, const float *bq, const float *bk, const float *bv,
                const float *cos_tab, const float *sin_tab, int n_pos,
                float *q_out, float *k_cache_layer, float *v_cache_layer, vxh_stream s);
/* vxh_rope_kv of a VXH_PRO_RESID/ROWS product: q, k, v are the accumulator's
 * fp32 roundings times 1/sqrt(ss[m]/ss_K + 1e-5) before the biases. */
int vxh_rope_kv_norm(double *qkv, int ld_qkv, int M, int n_past, int n_ctx, int n_heads,
                     int n_kv_heads, int head_dim, const float *bq, const float *bk,
                     const float *bv, const float *cos_tab, const float *sin_tab, int n_pos,
                     const double *ss, int ss_K, float *q_out, float *k_cache_layer,
                     float *v_cache_layer, vxh_stream s);
/* Causal attention of M rows against the layer's KV cache
 * (src/model.c:300-338): row m reads positions [0, min(pos_m + 1, cap)),
 * head h uses kv head h*n_kv/n_heads, softmax with 1/(sum + 1e-10).  Two
 * launches: per-chunk partial softmax, then the cross-chunk combine; the
 * partials live in ws->part.  head_dim: a multiple of 4, at most 128. */
int vxh_attention(const float *q, int M, int n_past, int n_ctx, int n_heads, int n_kv_heads,
                  int head_dim, int cap, const float *k_cache_layer,
                  const float *v_cache_layer, float *out, int ld_out,
                  vxh_workspace *ws, vxh_stream s);

/* vxh_rope_kv_norm + vxh_attention in two launches: the first reads q and
 * this forward's own k/v rows straight from the q|k|v sums qkv[M][ld_qkv]
 * (deferred RMSNorm from ss when not NULL, biases, RoPE; bit-for-bit the
 * values vxh_rope_kv_norm writes) and stores the new k/v rows into the cache;
 * the second combines the chunks and clears qkv.  A batch whose last row
 * reaches past n_ctx - 1 must be a single row (the reference's clamp keeps
 * one row at n_ctx - 1). */
#define VXH_ATTN_QKV_FAST_ROWS 16   /* head_dim 64/128 batches up to this many rows take the
                                      * fp32-MFMA kernel; larger ones a slower LDS kernel */
int vxh_attention_qkv(double *qkv, int ld_qkv, const double *ss, int ss_K, const float *bq,
                      const float *bk, const float *bv, const float *cos_tab, const float *sin_tab,
                      int n_pos, int M, int n_past, int n_ctx, int n_heads, int n_kv_heads,
                      int head_dim, int cap, float *k_cache_layer, float *v_cache_layer, float *out,
                      int ld_out, vxh_workspace *ws, vxh_stream s);
/* vxh_attention_qkv that leaves the q|k|v sums as they are, for a caller
 * whose accumulators are cleared elsewhere (the model forward's per-layer
 * accumulators, cleared at the start of each forward). */
int vxh_attention_qkv_keep(double *qkv, int ld_qkv, const double *ss, int ss_K, const float *bq,
                           const float *bk, const float *bv, const float *cos_tab, const float *sin_tab,
                           int n_pos, int M, int n_past, int n_ctx, int n_heads, int n_kv_heads,
                           int head_dim, int cap, float *k_cache_layer, float *v_cache_layer, float *out,
                           int ld_out, vxh_workspace *ws, vxh_stream s);

/* The first launch of vxh_attention_qkv alone: the partials stay in
 * ws->part for a VXH_PRO_ATTN GEMM, which combines them (and must clear qkv,
 * see vxh_pro.clear); *n_chunks receives their chunk count.  Layout: query
 * qi = (head % G) * M + m of kv head g (G = n_heads / n_kv_heads) has chunk c
 * at part + ((g * n_chunks + c) * G * M + qi) * (head_dim + 4): max, sum, two
 * unused floats, then the head_dim weighted value sums. */
int vxh_attention_parts_qkv(double *qkv, int ld_qkv, const double *ss, int ss_K, const float *bq,
                            const float *bk, const float *bv, const float *cos_tab,
                            const float *sin_tab, int n_pos, int M, int n_past, int n_ctx,
                            int n_heads, int n_kv_heads, int head_dim, int cap,
                            float *k_cache_layer, float *v_cache_layer, vxh_workspace *ws,
                            int *n_chunks, vxh_stream s);

/* vxh_attention_qkv / vxh_attention_parts_qkv over an IEEE fp16 KV cache
 * (k/v_cache_layer: [n_ctx][n_kv_heads * head_dim] halves, 8-byte aligned):
 * the new rows are rounded to nearest even when stored, and this forward's
 * own rows are attended to as rounded, so a batch and the same rows one at
 * a time see the same keys and values.  A flagged mode (the reference keeps
 * fp32, src/model.c:291-296, :404-411), for head_dim 64 or 128 and at most
 * VXH_ATTN_QKV_FAST_ROWS rows; it halves the attention's cache bytes. */
int vxh_attention_qkv_f16(double *qkv, int ld_qkv, const double *ss, int ss_K, const float *bq,
                          const float *bk, const float *bv, const float *cos_tab, const float *sin_tab,
                          int n_pos, int M, int n_past, int n_ctx, int n_heads, int n_kv_heads,
                          int head_dim, int cap, uint16_t *k_cache_layer, uint16_t *v_cache_layer,
                          float *out, int ld_out, vxh_workspace *ws, vxh_stream s);
int vxh_attention_parts_qkv_f16(double *qkv, int ld_qkv, const double *ss, int ss_K, const float *bq,
                                const float *bk, const float *bv, const float *cos_tab,
                                const float *sin_tab, int n_pos, int M, int n_past, int n_ctx,
                                int n_heads, int n_kv_heads, int head_dim, int cap,
                                uint16_t *k_cache_layer, uint16_t *v_cache_layer, vxh_workspace *ws,
                                int *n_chunks, vxh_stream s);

size_t vxh_attention_workspace_floats(int M, int n_ctx, int cap, int n_heads, int n_kv_heads,
                                      int head_dim);

/* ---- elementwise ------------------------------------------------------------- */
/* y[m][i] += x[m][i] for i < n (residual add, src/model.c:546, :589). */
int vxh_add_rows(float *y, int ldy, const float *x, int ldx, int M, int n, vxh_stream s);
/* dst[m][i] = src[m][i] for i < n. */
int vxh_copy_rows(float *dst, int ld_dst, const float *src, int ld_src, int M, int n,
                  vxh_stream s);
int vxh_rmsnorm(const float *x, int ldx, int M, int K, const float *w, float *out, int ld_out,
                vxh_stream s);
int vxh_fill_rows(float *y, int ld, int M, int col0, int n, float value, vxh_stream s);

/* ---- acceptance ----------------------------------------------------------------
 * Row statistics of logits L[R][V] at temperature T > 0: max, sum of
 * exp((l-max)/T) and the first argmax (src/speculative.c:44-53, :93-98).
 * stats[r] = {max, sum, argmax(as float bits)} (3 floats per row). */
int vxh_row_stats(const float *L, int ldl, int R, int V, float T, float *stats, vxh_stream s);
/* Draft sampler (src/speculative.c:35-91): token = inverse CDF at uniform
 * u_dev[0] over the nucleus of softmax(l/T) (the shortest prefix of tokens
 * sorted by descending probability, ties by index, whose fixed-point mass
 * reaches top_p; every token when top_p >= 1), drawn in index order.  T <= 0:
 * argmax.  Writes the token to token_out[0] and the nucleus descriptor
 * nuc[0..7] = {max, 1/(sum+1e-30), tau, tie_cut, mass, argmax, 0, 0}: token v
 * is in the nucleus iff p_v > tau or (p_v == tau and v <= tie_cut); tau < 0
 * means all tokens. */
int vxh_sample(const float *l, int V, float T, float top_p, const float *u_dev,
               int *token_out, float *nuc, vxh_stream s);
/* vxh_sample that also leaves a copy of l[0..V) in keep (device, or NULL):
 * the draft loop keeps each draft row for the verify decision without a
 * separate copy launch (src/speculative.c:167 stores the draft's logits
 * per drafted token). */
int vxh_sample_keep(const float *l, int V, float T, float top_p, const float *u_dev,
                    int *token_out, float *nuc, float *keep, vxh_stream s);
/* Verify decisions for k drafts (src/speculative.c:186-233 on probabilities):
 * L: target logits [k+1][ldl] with their vxh_row_stats, D: draft logits
 * [k][ldd] with nucleus descriptors nuc[k][8], drafts[k], uniforms u[k+1]
 * (device).  T <= 0 = greedy.  Writes out[0] = emitted count, out[1] =
 * accepted count, out[2..] = emitted tokens. */
int vxh_accept(const float *L, int ldl, int V, const float *stats, const float *D, int ldd,
               int Vd, const float *nuc, const int *drafts, int k, float T, const float *u,
               int *out, vxh_stream s);

/* ---- acceptance on many compute units ------------------------------------------
 * The same three operations with each row cut into up to 64 chunks of a
 * multiple of 1024 entries, one workgroup per chunk; the workgroup that
 * finishes last combines the chunks' partial results (fixed-point masses are
 * integers: the drawn token does not depend on the chunking).  They replace
 * the single-workgroup kernels of src/speculative.c:186-233 (vxh_accept),
 * :35-91 (vxh_sample, top_p >= 1) and the softmax statistics of :44-53.
 * The workspace holds the partials and completion counters (zeroed at
 * allocation, left zeroed by every call); one workspace serves one stream at
 * a time.  vxh_sample_keep_mc with top_p < 1, or with V <= 32768 (rows the
 * one-workgroup sampler holds in registers, where it is faster), runs
 * vxh_sample_keep;
 * vxh_accept_mc with T > 0 and k = 0 runs vxh_accept.  max_rows bounds R of
 * vxh_row_stats_mc. */
typedef struct {
    void *part;       /* partial results */
    unsigned *cnt;    /* completion counters */
    float *stats;     /* the sampler's row statistics */
    int max_rows;
} vxh_vocab_ws;
int vxh_vocab_ws_alloc(vxh_vocab_ws *ws, int max_rows);
void vxh_vocab_ws_free(vxh_vocab_ws *ws);
int vxh_row_stats_mc(const float *L, int ldl, int R, int V, float T, float *stats, vxh_vocab_ws *ws,
                     vxh_stream s);
int vxh_sample_keep_mc(const float *l, int V, float T, float top_p, const float *u_dev, int *token_out,
                       float *nuc, float *keep, vxh_vocab_ws *ws, vxh_stream s);
int vxh_accept_mc(const float *L, int ldl, int V, const float *stats, const float *D, int ldd, int Vd,
                  const float *nuc, const int *drafts, int k, float T, const float *u, int *out,
                  vxh_vocab_ws *ws, vxh_stream s);

#ifdef __cplusplus
}
#endif
#endif
