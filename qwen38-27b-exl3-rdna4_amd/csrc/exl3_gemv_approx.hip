// exl3_gemv_approx.hip -- the approximate mul1 instantiations of the fused GEMV (codebook ids 3:
// affine, unrounded weights; 4: int8 activations), compiled apart from the faithful ones in
// exl3_gemv.hip so the two sets build in parallel.
#include "exl3_gemv_kernel.h"

template <int BITS>
static int launch_approx_bits(const GemvArgs& a, int cb, int wgs, hipStream_t s)
{
    return cb == 3 ? launch_gemv_m<BITS, 3, FORM_PLAIN>(a, wgs, s) : launch_gemv_m<BITS, 4, FORM_PLAIN>(a, wgs, s);
}

int launch_gemv_approx(const GemvArgs& a, int bits, int cb, int wgs, hipStream_t s)
{
    switch (bits) {
        case 1: return launch_approx_bits<1>(a, cb, wgs, s);
        case 2: return launch_approx_bits<2>(a, cb, wgs, s);
        case 3: return launch_approx_bits<3>(a, cb, wgs, s);
        case 4: return launch_approx_bits<4>(a, cb, wgs, s);
        case 5: return launch_approx_bits<5>(a, cb, wgs, s);
        case 6: return launch_approx_bits<6>(a, cb, wgs, s);
        case 7: return launch_approx_bits<7>(a, cb, wgs, s);
        default: return launch_approx_bits<8>(a, cb, wgs, s);
    }
}
