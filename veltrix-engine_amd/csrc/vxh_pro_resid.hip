// vxh_gemm_pro instances of the residual prologue (t = x + src, panel of
// w .* t, t stored, sum t^2 added): the GEMMs that follow a residual GEMM.
#include "vxh_gemm_core.h"

int vx_gemm_pro_resid(const vxh_qmat *W, int M, vx_gemm_args &a, hipStream_t st, hipEvent_t e0,
                      hipEvent_t e1)
{
    return vx_dispatch<VX_PRO_RESID>(W, M, 0, a, st, e0, e1);
}
