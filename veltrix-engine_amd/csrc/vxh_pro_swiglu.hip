// vxh_gemm_pro instances of the SwiGLU prologue: the FFN down projection
// reads the gate/up sums directly.
#include "vxh_gemm_core.h"

int vx_gemm_pro_swiglu(const vxh_qmat *W, int M, vx_gemm_args &a, hipStream_t st, hipEvent_t e0,
                       hipEvent_t e1)
{
    return vx_dispatch<VX_PRO_SWIGLU>(W, M, 0, a, st, e0, e1);
}
