// exl3_gemv_silu.hip -- the SiLU-input instantiations of the fused GEMV (the input rows are
// fp16(fp16(silu(gate)) * up), formed as they load), compiled apart from the plain ones in
// exl3_gemv.hip so those carry none of the extra loads.
#include "exl3_gemv_kernel.h"

int launch_gemv_silu_in(const GemvArgs& a, int bits, int cb, int wgs, hipStream_t s)
{
    return launch_gemv_impl<FORM_SILU_IN>(a, bits, cb, wgs, s);
}
