// exl3_had.hip -- the float32 128-point Hadamard transform on the matrix cores (the prefill's
// input transforms and exl3_had_r_128_f32), in a file of its own so that its build options apply
// to it alone.
#include "exl3_device.h"
#include "../../include/exl3_mi355x.h"

using namespace exl3;

namespace {

// The float32 transform on the matrix cores (had128_mfma16): y = fp16(fp16(x * pre) H * r * scale)
// [* post], one wave per 16 rows x one 128-block, all groups from one read of x (VALU ~3.5 ops per
// element against ~15 for float32 butterflies, which left the pass issue-bound).  PRE: every group
// has a pre-scale (else none has); POST: post is given.  The loads of x, post and the first group's
// pre go out together, and each group's pre is requested while the group before it is transformed,
// so a wave waits for one round trip before its first MFMA (loading each pre-scale piece where it
// is used had put four dependent round trips per group ahead of the matrix work).  UP: the input
// rows are fp16(fp16(silu(in)) * up) (a gated MLP's activation, up's rows ld_in apart as in's),
// formed as they load: the down projection's transform reads gate and up instead of an
// activation pass's output.  Each wave reads its whole tile before it writes: in place is safe.
template <bool PRE, bool POST, bool UP>
__global__ void __launch_bounds__(256) had_mfma_kernel(const uint16_t* __restrict__ in, const uint16_t* __restrict__ up,
                                                       int64_t ld_in, HadGroups hg, int groups, int64_t ld_out, int rows,
                                                       int cols, const uint16_t* __restrict__ post, float scale)
{
    // wave index in 32 bits (the host keeps waves < 2^31), divided by the block count on the scalar unit
    const uint32_t nblk = (uint32_t) cols / 128u;
    const uint32_t wid = blockIdx.x * 4u + (uint32_t) __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t row_groups = ((uint32_t) rows + 15u) / 16u;
    if (wid >= row_groups * nblk) return;                     // uniform per wave (no barrier below)
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    const uint32_t rg = wid / nblk;
    const int col0 = (int) (wid - rg * nblk) * 128 + 8 * g;   // this lane's first column
    const int64_t row = (int64_t) rg * 16 + j;
    const bool live = row < rows;
    u32x4 xb[4], pv[4], pn[4];
#pragma unroll
    for (int s_ = 0; s_ < 4; ++s_) {
        xb[s_] = live ? *reinterpret_cast<gc_u32x4*>(as_global(in) + row * ld_in + col0 + 32 * s_) : u32x4{0u, 0u, 0u, 0u};
        if constexpr (UP)
            if (live) xb[s_] = silu_mul_x8(xb[s_], *reinterpret_cast<gc_u32x4*>(as_global(up) + row * ld_in + col0 + 32 * s_));
        if constexpr (POST) pv[s_] = *reinterpret_cast<gc_u32x4*>(as_global(post) + col0 + 32 * s_);
        if constexpr (PRE) pn[s_] = *reinterpret_cast<gc_u32x4*>(as_global(hg.pre[0]) + col0 + 32 * s_);
    }
    const HadMfmaA A = had_mfma_a();
#pragma unroll
    for (int gi = 0; gi < EXL3_MAX_GROUPS; ++gi) {
        if (gi >= groups) break;
        // constant indices into the argument struct (a runtime index would copy it to scratch)
        uint16_t* out = gi == 0 ? hg.out[0] : gi == 1 ? hg.out[1] : gi == 2 ? hg.out[2] : hg.out[3];
        u32x4 xs[4];
        if constexpr (PRE) {
            u32x4 pc[4];
#pragma unroll
            for (int s_ = 0; s_ < 4; ++s_) pc[s_] = pn[s_];
            if (gi + 1 < EXL3_MAX_GROUPS && gi + 1 < groups) {
                const uint16_t* pre = gi == 0 ? hg.pre[1] : gi == 1 ? hg.pre[2] : hg.pre[3];
#pragma unroll
                for (int s_ = 0; s_ < 4; ++s_) pn[s_] = *reinterpret_cast<gc_u32x4*>(as_global(pre) + col0 + 32 * s_);
            }
#pragma unroll
            for (int s_ = 0; s_ < 4; ++s_)
                xs[s_] = __builtin_bit_cast(u32x4, __builtin_bit_cast(f16x8, xb[s_]) * __builtin_bit_cast(f16x8, pc[s_]));
        } else {
#pragma unroll
            for (int s_ = 0; s_ < 4; ++s_) xs[s_] = xb[s_];
        }
        had128_mfma16(A, xs, scale, POST, pv, [&](int p, u32x4 v) __attribute__((always_inline)) {
            if (live) *reinterpret_cast<g_u32x4*>(as_global(out) + row * ld_out + col0 + 32 * p) = v;
        });
    }
}

}  // namespace

// one launch of the float transform over `groups` outputs (launch_had, exl3_gemv.hip, has checked
// the arguments): pre for every group (has_pre) or for none; up (may be null): the input rows are
// fp16(fp16(silu(in)) * up)
void launch_had_mfma(const uint16_t* in, const uint16_t* up, int64_t ld_in, const HadGroups& hg, int groups,
                     int64_t ld_out, int rows, int cols, const uint16_t* post, float scale, bool has_pre, hipStream_t s)
{
    const int64_t waves = ((int64_t) rows + 15) / 16 * (cols / 128);
    using K = void (*)(const uint16_t*, const uint16_t*, int64_t, HadGroups, int, int64_t, int, int, const uint16_t*, float);
    static const K kernels[8] = {had_mfma_kernel<false, false, false>, had_mfma_kernel<false, false, true>,
                                 had_mfma_kernel<false, true, false>,  had_mfma_kernel<false, true, true>,
                                 had_mfma_kernel<true, false, false>,  had_mfma_kernel<true, false, true>,
                                 had_mfma_kernel<true, true, false>,   had_mfma_kernel<true, true, true>};
    const K kern = kernels[(has_pre ? 4 : 0) + (post ? 2 : 0) + (up ? 1 : 0)];
    hipLaunchKernelGGL(kern, dim3((unsigned) ((waves + 3) / 4)), dim3(256), 0, s, in, up, ld_in, hg, groups, ld_out,
                       rows, cols, post, scale);
}
