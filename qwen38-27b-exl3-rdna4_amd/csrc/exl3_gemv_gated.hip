// exl3_gemv_gated.hip -- the gate / up instantiations of the fused GEMV (SiLU-and-mul epilogue),
// compiled apart from the plain ones in exl3_gemv.hip.
#include "exl3_gemv_kernel.h"

int launch_gemv_gated(const GemvArgs& a, int bits, int cb, int wgs, hipStream_t s)
{
    return launch_gemv_impl<FORM_GATED>(a, bits, cb, wgs, s);
}
