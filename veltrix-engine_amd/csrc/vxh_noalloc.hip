// vxh_gemm_noalloc: vxh_gemm without a workspace argument and without any
// allocation.  The fp64 accumulator the GEMM adds its K-slice partial sums
// into lives in `scratch`, a file-scope device array of fixed size that
// every GPU the library runs on holds until the process ends.
//
// In host code `scratch` names a host-side stand-in, not device memory: its
// device address is resolved once per device with hipGetSymbolAddress and
// only that address is handed to kernels and fills.
#include <string.h>

#include "vxh_internal.h"

static __device__ __align__(256) double scratch[VXH_NOALLOC_ACC_ELEMS];

#define VX_NOALLOC_MAX_DEVICES 64
static double *g_scratch_dev[VX_NOALLOC_MAX_DEVICES];   // device address per device ordinal

// The scratch array's device address on the current device (resolved on the
// entry point's first call on that device, with that device current).
static int vx_scratch_ptr(double **out)
{
    int dev = -1;
    VXH_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= VX_NOALLOC_MAX_DEVICES)
        return vxh_fail(VXH_ERR_PARAM, "gemm_noalloc: device ordinal %d out of range", dev);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return vxh_fail(VXH_ERR_LAUNCH, "gemm_noalloc: hipGetSymbolAddress(scratch): %s",
                            hipGetErrorString(e));
        g_scratch_dev[dev] = (double *)p;
    }
    *out = g_scratch_dev[dev];
    return VXH_OK;
}

extern "C" int vxh_gemm_noalloc(const vxh_qmat *W, const vxh_panel *X, int M, const vxh_epilogue *ep, int path,
                                vxh_stream s)
{
    int rc = vxh_init();
    if (rc) return rc;
    if (!W || !X || !ep) return vxh_fail(VXH_ERR_PARAM, "gemm_noalloc: NULL argument");
    if (M < 1 || M > 16) return vxh_fail(VXH_ERR_PARAM, "gemm_noalloc: M %d outside 1..16", M);
    const size_t need = vxh_gemm_workspace_elems(W->n_rows, M);
    if (need > (size_t)VXH_NOALLOC_ACC_ELEMS)
        return vxh_fail(VXH_ERR_PARAM,
                        "gemm_noalloc: %d rows x %d output columns need %zu accumulator elements, "
                        "above the static scratch of %d (use vxh_gemm with a workspace)",
                        M, W->n_rows, need, VXH_NOALLOC_ACC_ELEMS);
    double *acc = nullptr;
    if ((rc = vx_scratch_ptr(&acc))) return rc;
    // the array keeps whatever the last call (or a failed one) left: clear
    // the part this call accumulates into, with a fill kernel
    if ((rc = vxh_fill_f32((float *)acc, 0.0f, 2 * need, s))) return rc;
    vxh_workspace ws;
    memset(&ws, 0, sizeof(ws));
    ws.acc = acc;
    ws.acc_elems = need;
    return vxh_gemm(W, X, M, ep, &ws, path, s);
}
