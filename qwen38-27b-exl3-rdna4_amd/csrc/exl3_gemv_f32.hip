// exl3_gemv_f32.hip -- the fp32-output instantiations of the fused GEMV (single row: C kept in
// fp32, y = (float) (H C r) * svh), compiled apart so the fp16 forms carry none of their code.
#include "exl3_gemv_kernel.h"

namespace {

template <int BITS>
int launch_f32_cb(const GemvArgs& a, int cb, int wgs, hipStream_t s)
{
    switch (cb) {
        case 0: return launch_gemv_t<BITS, 0, 0, FORM_F32OUT>(a, wgs, s);
        case 1: return launch_gemv_t<BITS, 1, 0, FORM_F32OUT>(a, wgs, s);
        default: return launch_gemv_t<BITS, 2, 0, FORM_F32OUT>(a, wgs, s);
    }
}

}  // namespace

int launch_gemv_f32out(const GemvArgs& a, int bits, int cb, int wgs, hipStream_t s)
{
    if (a.M != 1) return EXL3_DECLINED;
    switch (bits) {
        case 1: return launch_f32_cb<1>(a, cb, wgs, s);
        case 2: return launch_f32_cb<2>(a, cb, wgs, s);
        case 3: return launch_f32_cb<3>(a, cb, wgs, s);
        case 4: return launch_f32_cb<4>(a, cb, wgs, s);
        case 5: return launch_f32_cb<5>(a, cb, wgs, s);
        case 6: return launch_f32_cb<6>(a, cb, wgs, s);
        case 7: return launch_f32_cb<7>(a, cb, wgs, s);
        default: return launch_f32_cb<8>(a, cb, wgs, s);
    }
}
