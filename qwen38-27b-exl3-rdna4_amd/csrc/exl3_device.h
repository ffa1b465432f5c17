// exl3_device.h -- gfx950 (CDNA4, wave64) device building blocks for the EXL3 trellis linear.
//
//  * q-block trellis decoder: one lane turns the 32 consecutive ring positions of a tile's
//    "q-block" (positions 32q .. 32q+31 == tile columns q and q+8, all 16 rows) into 16 packed
//    fp16 pairs, specialised per bitrate at compile time (window extraction plan, codebook).
//  * wave64 128-point Hadamard in three lane layouts, float32 or float64 butterflies.
//  * float64 -> fp16 round-to-nearest-even.
//
// Format facts restated from the reference oracle (reference/exl3_oracle.py):
//  * a tile is 16*bits little-endian u16 words == 8*bits u32 words, bits numbered MSB-first
//    across the u32 ring (:149-153);
//  * the state at position t is the 16-bit window ending at ring bit (t+1)*bits (:156-188);
//  * position t -> (row, col): L = t>>3, i = t&7, row = 2(L%4) + (i&1) + 8((i>>1)&1),
//    col = 2(L>>3) + ((L>>2)&1) + 8(i>>2) (:129-146);
//  * codebooks (:67-119): mul1 v = fp16((1024 + bytesum(w*0x83DCD12D)) * k_inv + k_bias) with one
//    rounding; mcg / 3inst: x = w*0xCBAC1FED or w*89226354 + 64248484, x' = (x & 0x8FFF8FFF) ^
//    0x3B603B60, v = fp16(fp16(x'.lo) + fp16(x'.hi)).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/exl3_mi355x.h"

namespace exl3 {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr double R_SCALE = 0.088388347648;   // the Hadamard scale of every reference call site

// Global-address-space views.  Pointers read from structs or pointer tables are generic, and
// loads through generic pointers compile to flat_load, which also counts against lgkmcnt: every
// LDS wait would then wait for in-flight HBM loads too.  Hot-path loads go through these.
typedef __attribute__((address_space(1))) const uint32_t gc_u32;
typedef __attribute__((address_space(1))) const uint16_t gc_u16;
typedef __attribute__((address_space(1))) uint16_t g_u16;
typedef __attribute__((address_space(1))) const u32x4 gc_u32x4;
typedef __attribute__((address_space(1))) u32x4 g_u32x4;
typedef __attribute__((address_space(1))) const u32x2 gc_u32x2;
typedef __attribute__((address_space(1))) const uint8_t gc_u8;

template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T* as_global(T* p)
{
    return (__attribute__((address_space(1))) T*) p;
}

// ------------------------------------------------------------------------------------------
// float64 -> fp16 bits, round to nearest even (exact single rounding).
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f64_to_f16_bits(double v)
{
    const uint64_t b = (uint64_t) __double_as_longlong(v);
    const uint32_t sign = (uint32_t) (b >> 48) & 0x8000u;
    const uint64_t mag = b & 0x7FFFFFFFFFFFFFFFull;
    const int e16 = (int) (mag >> 52) - 1023;
    if (e16 < -25) return sign;                        // below half the smallest subnormal
    if (e16 >= 16) return sign | 0x7C00u;              // overflow (no NaN inputs on this path)
    const uint64_t m = (mag & 0xFFFFFFFFFFFFFull) | (1ull << 52);
    const int shift = e16 >= -14 ? 42 : 42 + (-14 - e16);
    uint64_t kept = m >> shift;
    const uint64_t rem = m & ((1ull << shift) - 1);
    const uint64_t half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (kept & 1))) kept++;
    uint32_t r = e16 >= -14 ? (uint32_t) (((e16 + 15) << 10) + (int) kept - 1024) : (uint32_t) kept;
    if (r > 0x7C00u) r = 0x7C00u;
    return sign | r;
}

__device__ __forceinline__ f16 bits_f16(uint32_t b) { return __builtin_bit_cast(f16, (uint16_t) b); }
__device__ __forceinline__ uint32_t f16_bits(f16 h) { return (uint32_t) __builtin_bit_cast(uint16_t, h); }

// ------------------------------------------------------------------------------------------
// float64 -> fp16 through a round-to-odd float32 (two instructions plus a fix-up instead of the
// integer path above): rounding to odd at 24 bits, then to nearest-even at 11 bits, equals a
// single nearest-even rounding of the float64 value.
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ f16 f64_to_f16_rto(double v)
{
    const float f = (float) v;
    uint32_t fb = __float_as_uint(f);
    const double back = (double) f;
    if (back != v && !(fb & 1u)) fb += __builtin_fabs(back) < __builtin_fabs(v) ? 1u : 0xFFFFFFFFu;
    return (f16) __uint_as_float(fb);
}

// ------------------------------------------------------------------------------------------
// 128-point Hadamard.  Natural-order Sylvester H[i,j] = (-1)^popcount(i&j), computed as seven
// butterfly stages over the element-index bits 0, 1, ..., 6 in that order; each stage maps the
// pair (a, b) of elements differing in that bit to (a + b, a - b).  The stages run inside a lane
// or across lanes (DPP, ds_swizzle, v_permlane32_swap) depending on the layout, but every layout
// performs the same additions in the same order, so all layouts give identical results for a
// given element type T:
//   T = double: exact whenever a block's nonzero values span at most 35 binades (53-bit sums of
//               128 fp16 values: 35 + 11 mantissa + 7 carry bits), and then bit-exact to the
//               oracle's float64 matrix product; fp16 spans 40 binades, so an adversarial block
//               can still round differently.
//               Used where exactness is the contract: the exl3_had_r_128 entry point and the fused
//               GEMV's input and output transforms (the reference's strict M = 1 gates assume
//               correctly rounded fp16 values).
//   T = float:  24-bit sums, one rounding per stage; the fp16 result can differ from the exact one
//               in the last place.  No caller at present: the prefill's float32 transforms run on
//               the matrix cores (had128_mfma16 below).
// ------------------------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ double dpp_x(double x)
{
    const uint64_t u = (uint64_t) __double_as_longlong(x);
    const uint32_t lo = (uint32_t) __builtin_amdgcn_mov_dpp((int) (uint32_t) u, CTRL, 0xF, 0xF, true);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_mov_dpp((int) (uint32_t) (u >> 32), CTRL, 0xF, 0xF, true);
    return __longlong_as_double((long long) (((uint64_t) hi << 32) | lo));
}

template <int CTRL>
__device__ __forceinline__ float dpp_x(float x)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

constexpr int DPP_QP_XOR1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int DPP_QP_XOR2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int DPP_QP_REV = 0x1B;      // quad_perm [3,2,1,0]   (lane ^ 3)
constexpr int DPP_HALF_MIRROR = 0x141; // lane ^ 7 within 8
constexpr int DPP_ROR8 = 0x128;       // row_ror:8 == lane ^ 8 within 16

// value of lane (lane ^ 16): ds_swizzle within 32-lane halves (and 0x1F, xor 0x10)
__device__ __forceinline__ double swz16_x(double x)
{
    const uint64_t u = (uint64_t) __double_as_longlong(x);
    const uint32_t lo = (uint32_t) __builtin_amdgcn_ds_swizzle((int) (uint32_t) u, 0x401F);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_ds_swizzle((int) (uint32_t) (u >> 32), 0x401F);
    return __longlong_as_double((long long) (((uint64_t) hi << 32) | lo));
}

__device__ __forceinline__ float swz16_x(float x)
{
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401F));
}

// (value of the lower half's lane, value of the upper half's lane) for lane & 31:
// v_permlane32_swap(x, x) swaps the upper half of its first operand with the lower half of its
// second, so its first result holds the lower half's values in both halves of the wave
__device__ __forceinline__ void halves_x(double x, double& lo, double& hi)
{
    const uint64_t u = (uint64_t) __double_as_longlong(x);
    const auto w0 = __builtin_amdgcn_permlane32_swap((uint32_t) u, (uint32_t) u, false, false);
    const auto w1 = __builtin_amdgcn_permlane32_swap((uint32_t) (u >> 32), (uint32_t) (u >> 32), false, false);
    lo = __longlong_as_double((long long) (((uint64_t) w1[0] << 32) | w0[0]));
    hi = __longlong_as_double((long long) (((uint64_t) w1[1] << 32) | w0[1]));
}

__device__ __forceinline__ void halves_x(float x, float& lo, float& hi)
{
    const auto w = __builtin_amdgcn_permlane32_swap((uint32_t) __float_as_int(x), (uint32_t) __float_as_int(x), false, false);
    lo = __int_as_float((int) w[0]);
    hi = __int_as_float((int) w[1]);
}

// fp16 of v * scale: double -> one rounding of the exact float64 product (round to odd float32,
// then to fp16); float -> the product rounded to float32, then to fp16
__device__ __forceinline__ f16 scaled_f16(double v, double scale) { return f64_to_f16_rto(v * scale); }
__device__ __forceinline__ f16 scaled_f16(float v, float scale) { return (f16) (v * scale); }

// one cross-lane butterfly stage: the lane holding a (bit clear) takes a + b, the lane holding b
// takes a - b; fma with +-1 rounds once, as the separate add / subtract would
template <class T, int N>
__device__ __forceinline__ void had_stage(T (&v)[N], const T (&p)[N], bool upper)
{
    const T s = upper ? T(-1) : T(1);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = __builtin_fma(s, v[i], p[i]);
}

// in-lane stages over element bits 0 .. log2(N) - 1
template <class T, int N>
__device__ __forceinline__ void had_in_lane(T (&v)[N])
{
#pragma unroll
    for (int h = 1; h < N; h <<= 1)
#pragma unroll
        for (int i = 0; i < N; ++i)
            if (!(i & h)) {
                const T a = v[i], b = v[i + h];
                v[i] = a + b;
                v[i + h] = a - b;
            }
}

// 16 lanes per block: lane r = lane & 15 holds elements 8r .. 8r+7 (a wave transforms 4 blocks);
// element bits 0..2 in the lane, bits 3..6 lane xor 1, 2, 4, 8 (quad_perm, row_half_mirror, row_ror)
template <class T>
__device__ __forceinline__ void wht128_x8(T (&v)[8])
{
    had_in_lane(v);
    const int r = __lane_id() & 15;
    T p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = dpp_x<DPP_QP_XOR1>(v[i]);
    had_stage(v, p, r & 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = dpp_x<DPP_QP_XOR2>(v[i]);
    had_stage(v, p, r & 2);
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = dpp_x<DPP_QP_REV>(dpp_x<DPP_HALF_MIRROR>(v[i]));
    had_stage(v, p, r & 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = dpp_x<DPP_ROR8>(v[i]);
    had_stage(v, p, r & 8);
}

// 8 fp16 in (16 B) -> 8 fp16 out: fp16(Had128(in [* pre]) * scale) [* post]; pre / post are the
// matching 8 scale values (ignored when has_pre / has_post are false).  Each fp16 product is a
// single rounding (packed fp16 multiplies), as in the reference kernels' hmul2 stages.
template <class T>
__device__ __forceinline__ u32x4 had128_x8(u32x4 in, u32x4 pre, bool has_pre, u32x4 post, bool has_post, T scale)
{
    f16x8 x = __builtin_bit_cast(f16x8, in);
    if (has_pre) x = x * __builtin_bit_cast(f16x8, pre);
    T v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (T) x[i];
    wht128_x8(v);
    f16x8 y;
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = scaled_f16(v[i], scale);
    if (has_post) y = y * __builtin_bit_cast(f16x8, post);
    return __builtin_bit_cast(u32x4, y);
}

// One 128-block per 8 lanes, 16 elements per lane (lane r = lane & 7 holds elements 16r ..
// 16r + 15): element bits 0..3 in the lane, bits 4..6 lane xor 1, 2, 4 (quad_perm, then
// row_half_mirror + quad_perm reverse).  Fewer cross-lane moves per element than had128_x8.
template <class T>
__device__ __forceinline__ void had128_x16(const u32x4 (&in)[2], const u32x4 (&pre)[2], bool has_pre,
                                           const u32x4 (&post)[2], bool has_post, T scale, u32x4 (&out)[2])
{
    T v[16];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        f16x8 x = __builtin_bit_cast(f16x8, in[c]);
        if (has_pre) x = x * __builtin_bit_cast(f16x8, pre[c]);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[8 * c + i] = (T) x[i];
    }
    had_in_lane(v);
    const int r = __lane_id() & 7;
    T p[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) p[i] = dpp_x<DPP_QP_XOR1>(v[i]);
    had_stage(v, p, r & 1);
#pragma unroll
    for (int i = 0; i < 16; ++i) p[i] = dpp_x<DPP_QP_XOR2>(v[i]);
    had_stage(v, p, r & 2);
#pragma unroll
    for (int i = 0; i < 16; ++i) p[i] = dpp_x<DPP_QP_REV>(dpp_x<DPP_HALF_MIRROR>(v[i]));
    had_stage(v, p, r & 4);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        f16x8 y;
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = scaled_f16(v[8 * c + i], scale);
        if (has_post) y = y * __builtin_bit_cast(f16x8, post[c]);
        out[c] = __builtin_bit_cast(u32x4, y);
    }
}

// One 128-block per wave, two elements per lane (lane l holds elements 2l and 2l + 1): element
// bit 0 in the lane, bits 1..4 lane xor 1, 2, 4, 8 (DPP as in wht128_x8), bit 5 lane xor 16
// (ds_swizzle), bit 6 lane xor 32 (v_permlane32_swap).  A fourth of wht128_x8's instructions per
// lane: the latency form for the GEMV's single-row input and output transforms, which are on every
// launch's critical path.
// The stages of the single-row layout after bit 0 (v = {a + b, a - b} of the lane's two elements).
template <class T>
__device__ __forceinline__ void wht128_x2_rest(T (&v)[2])
{
    const int l = __lane_id();
    T p[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) p[i] = dpp_x<DPP_QP_XOR1>(v[i]);
    had_stage(v, p, l & 1);
#pragma unroll
    for (int i = 0; i < 2; ++i) p[i] = dpp_x<DPP_QP_XOR2>(v[i]);
    had_stage(v, p, l & 2);
#pragma unroll
    for (int i = 0; i < 2; ++i) p[i] = dpp_x<DPP_QP_REV>(dpp_x<DPP_HALF_MIRROR>(v[i]));
    had_stage(v, p, l & 4);
#pragma unroll
    for (int i = 0; i < 2; ++i) p[i] = dpp_x<DPP_ROR8>(v[i]);
    had_stage(v, p, l & 8);
#pragma unroll
    for (int i = 0; i < 2; ++i) p[i] = swz16_x(v[i]);
    had_stage(v, p, l & 16);
    // bit 6: lower lanes take lo + hi, upper lanes lo - hi
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        T lo, hi;
        halves_x(v[i], lo, hi);
        v[i] = __builtin_fma(l & 32 ? T(-1) : T(1), hi, lo);
    }
}

template <class T>
__device__ __forceinline__ uint32_t had128_x2(uint32_t in, uint32_t pre, bool has_pre, uint32_t post, bool has_post,
                                              T scale)
{
    f16x2 x = __builtin_bit_cast(f16x2, in);
    if (has_pre) x = x * __builtin_bit_cast(f16x2, pre);
    const T a = (T) x[0], b = (T) x[1];
    T v[2] = {a + b, a - b};
    wht128_x2_rest(v);
    f16x2 y = {scaled_f16(v[0], scale), scaled_f16(v[1], scale)};
    if (has_post) y = y * __builtin_bit_cast(f16x2, post);
    return __builtin_bit_cast(uint32_t, y);
}

// The same layout on two fp32 inputs with an fp32 output: float64 butterflies (exact sums of the
// fp32 values while a block spans at most 22 binades), then (float) (v * scale) * post, post the
// lane's two fp16 scale values (the fp32-output GEMV's output transform)
__device__ __forceinline__ void had128_x2_f32(float a, float b, uint32_t post, double scale, float& o0, float& o1)
{
    double v[2] = {(double) a + (double) b, (double) a - (double) b};
    wht128_x2_rest(v);
    const f16x2 p = __builtin_bit_cast(f16x2, post);
    o0 = (float) (v[0] * scale) * (float) p[0];
    o1 = (float) (v[1] * scale) * (float) p[1];
}

// the Hadamard scale of every reference call site, per element type
template <class T> constexpr T r_scale() { return (T) R_SCALE; }

// SiLU-and-mul of 8 fp16 pairs with the activation kernels' roundings: silu in fp32
// (g / (1 + exp(-g))) rounded to fp16, then the fp16 product (exact in fp32) rounded once.
__device__ __forceinline__ u32x4 silu_mul_x8(u32x4 g, u32x4 u)
{
    const f16x8 gh = __builtin_bit_cast(f16x8, g), uh = __builtin_bit_cast(f16x8, u);
    f16x8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float gf = (float) gh[i];
        const f16 act = (f16) (gf / (1.0f + expf(-gf)));
        r[i] = (f16) ((float) act * (float) uh[i]);
    }
    return __builtin_bit_cast(u32x4, r);
}

// the same for two elements (one 32-bit register)
__device__ __forceinline__ uint32_t silu_mul_x2(uint32_t g, uint32_t u)
{
    const f16x2 gh = __builtin_bit_cast(f16x2, g), uh = __builtin_bit_cast(f16x2, u);
    f16x2 r;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float gf = (float) gh[i];
        const f16 act = (f16) (gf / (1.0f + expf(-gf)));
        r[i] = (f16) ((float) act * (float) uh[i]);
    }
    return __builtin_bit_cast(uint32_t, r);
}

// the (pre, out) pair of each group of one launch (a fused module's input transforms read one x)
struct HadGroups {
    const uint16_t* pre[EXL3_MAX_GROUPS];
    uint16_t* out[EXL3_MAX_GROUPS];
};

// ------------------------------------------------------------------------------------------
// 128-point Hadamard of 16 rows on the matrix cores (float32 sums): D = H^T X^T per 16-column
// tile t (v_mfma_f32_16x16x32_f16, K = 128 in four 32-steps s).  The B operand is the rows' input
// (lane l: row l & 15, the 8 columns 32 s + 8 (l >> 4) .. + 7), the A operand the +-1 entries
// H[c(t, i)][32 s + k] (lane l: i = l & 15, the same k), with output column
// c(t, i) = 32 (t >> 1) + 8 (i >> 2) + 4 (t & 1) + (i & 3), so that lane l of tiles 2p and 2p + 1
// holds the 8 consecutive outputs 32 p + 8 (l >> 4) .. + 7 of its row.  The sign
// (-1)^popcount(c & (32 s + k)) splits into (-1)^popcount((t >> 1) & s), which flips a whole
// 32-step, and a part that depends on the lane, the element and t & 1 only: the constant A
// fragments below, kept with both signs so that the flip selects a fragment instead of negating
// the input.  The products are exact and the sums fp32, so
// each output is the rounding of a value within the error bound of an fp32 summation of the
// block's 128 terms.  Every caller (the standalone float transform and the prefill epilogues)
// runs this same instruction sequence: their values agree bitwise.
// ------------------------------------------------------------------------------------------
struct HadMfmaA {
    f16x8 a[2], an[2];          // t & 1 = 0, 1; an = -a
};

__device__ __forceinline__ HadMfmaA had_mfma_a()
{
    const int lane = __lane_id(), j = lane & 15, g = lane >> 4;
    HadMfmaA A;
    // c & k: bits 0-1 (j & 3) & (e & 3), bit 2 (t & 1) & (e >> 2), bits 3-4 (j >> 2) & g
#pragma unroll
    for (int tau = 0; tau < 2; ++tau)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int par = (__builtin_popcount((j & 3) & (e & 3)) + (tau & (e >> 2)) + __builtin_popcount((j >> 2) & g)) & 1;
            A.a[tau][e] = par ? (f16) -1.0f : (f16) 1.0f;
            A.an[tau][e] = par ? (f16) 1.0f : (f16) -1.0f;
        }
    return A;
}

// xb[s]: this lane's row input (pre-scale applied) at columns 32 s + 8 (lane >> 4); emit(p, y) is
// called for p = 0 .. 3 as soon as tile pair p is done, y = the row's outputs 32 p + 8 (lane >> 4)
// .. + 7, fp16(D * scale) [* post[p] in fp16] (a caller's store then overlaps the next pair's MFMAs)
template <class Emit>
__device__ __forceinline__ void had128_mfma16(const HadMfmaA& A, const u32x4 (&xb)[4], float scale, bool has_post,
                                              const u32x4 (&post)[4], Emit&& emit)
{
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        f32x4 acc[2];
#pragma unroll
        for (int tau = 0; tau < 2; ++tau) {
            acc[tau] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const bool neg = __builtin_popcount(p & s) & 1;          // (t >> 1) & s, t = 2 p + tau
                acc[tau] = __builtin_amdgcn_mfma_f32_16x16x32_f16(neg ? A.an[tau] : A.a[tau],
                                                                  __builtin_bit_cast(f16x8, xb[s]), acc[tau], 0, 0, 0);
            }
        }
        f16x8 y;
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = (f16) (acc[e >> 2][e & 3] * scale);
        if (has_post) y = y * __builtin_bit_cast(f16x8, post[p]);
        emit(p, __builtin_bit_cast(u32x4, y));
    }
}

// ------------------------------------------------------------------------------------------
// Codebook constants
// ------------------------------------------------------------------------------------------
// CB 3 and 4 are the mul1 hash without the per-weight fp16 scale: the decoder emits the exact fp16
// integers 1024 + s (CB 3) or s (CB 4), and the GEMV applies k_inv and k_bias per output instead
// (the affine and int8-activation routes of the fused GEMV; never used for decoded weight tiles)
template <int CB> struct Codebook;
template <> struct Codebook<2> { static constexpr uint32_t lo = 0xD12Du, hi = 0x83DCu, add = 0; };       // mul1
template <> struct Codebook<3> : Codebook<2> {};                                                          // mul1, unscaled
template <> struct Codebook<4> : Codebook<2> {};                                                          // mul1, unscaled
template <> struct Codebook<1> { static constexpr uint32_t lo = 0x1FEDu, hi = 0xCBACu, add = 0; };       // mcg
template <> struct Codebook<0> { static constexpr uint32_t lo = 0x7C72u, hi = 0x0551u, add = 64248484u; }; // 3inst

// 32-bit hash of the 16-bit state held in half H (0 = lo, 1 = hi) of r, in two full-rate ops:
//   q = (s*C_hi [+ add_hi]) << 16 [| add_lo]   (v_pk_mul_lo_u16 / v_pk_mad_u16, lo lane * 0)
//   x = s*C_lo + q                              (v_mad_u32_u16)
// Both read only the selected 16 bits of r, so window extraction never needs masking.
template <int CB, int H>
__device__ __forceinline__ uint32_t state_hash(uint32_t r, uint32_t k_hi, uint32_t k_add, uint32_t k_lo)
{
    uint32_t q, x;
    if constexpr (CB == 0)
        asm("v_pk_mad_u16 %0, %1, %2, %3 op_sel:[%4,0,0] op_sel_hi:[%4,1,1]"
            : "=v"(q) : "v"(r), "s"(k_hi), "v"(k_add), "n"(H));
    else
        asm("v_pk_mul_lo_u16 %0, %1, %2 op_sel:[%3,0] op_sel_hi:[%3,1]" : "=v"(q) : "v"(r), "s"(k_hi), "n"(H));
    asm("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[%4,0,0,0]" : "=v"(x) : "v"(r), "s"(k_lo), "v"(q), "n"(H));
    return x;
}

// ------------------------------------------------------------------------------------------
// q-block window plan.  A lane holds words w[-1 .. BITS-1] of its q-block (relative to the q-block's
// first word; w[-1] is the ring predecessor) as W[0 .. BITS].  State p in [0, 32) is the window
// ending at bit e = (p+1)*BITS.  It is read from a 32-bit register r, half H:
//   e % 32 == 0            -> r = w[e/32 - 1], lo
//   e % 32 == 16           -> r = w[e/32],     hi
//   BITS | 16, e%32 < 16   -> r = R(e + 16),   hi    (one alignbit serves windows e and e+16)
//   otherwise              -> r = R(e),        lo
// where R(E) = the 32 ring bits ending at E = alignbit(w[E/32 - 1], w[E/32], 32*(E/32 + 1) - E).
// ------------------------------------------------------------------------------------------
struct WinSrc { int kind; int a; int b; int shift; int half; };   // kind 0: word a; kind 1: alignbit(a, b, shift)

template <int BITS>
__host__ __device__ constexpr WinSrc win_src(int p)
{
    const int e = (p + 1) * BITS;
    if (e % 32 == 0) return {0, e / 32 - 1, 0, 0, 0};
    if (e % 32 == 16) return {0, e / 32, 0, 0, 1};
    int E = e, half = 0;
    if ((16 % BITS) == 0 && (e % 32) < 16) { E = e + 16; half = 1; }
    return {1, E / 32 - 1, E / 32, 32 * (E / 32 + 1) - E, half};
}

// Register for state p: W[] is indexed from word -1.
template <int BITS, int P>
__device__ __forceinline__ uint32_t win_reg(const uint32_t* W)
{
    constexpr WinSrc s = win_src<BITS>(P);
    if constexpr (s.kind == 0) return W[s.a + 1];
    else return __builtin_amdgcn_alignbit(W[s.a + 1], W[s.b + 1], (uint32_t) s.shift);
}

template <int BITS, int CB, int P>
__device__ __forceinline__ uint32_t state_x(const uint32_t* W, uint32_t k_hi, uint32_t k_add, uint32_t k_lo)
{
    constexpr WinSrc s = win_src<BITS>(P);
    return state_hash<CB, s.half>(win_reg<BITS, P>(W), k_hi, k_add, k_lo);
}

// Decode the pair of states (2I, 2I+1) of the q-block into one packed fp16 pair (lo = state 2I).
template <int BITS, int CB, int I>
__device__ __forceinline__ uint32_t decode_pair(const uint32_t* W, uint32_t k_hi, uint32_t k_add, uint32_t k_lo,
                                                uint32_t c6400)
{
    const uint32_t x0 = state_x<BITS, CB, 2 * I>(W, k_hi, k_add, k_lo);
    const uint32_t x1 = state_x<BITS, CB, 2 * I + 1>(W, k_hi, k_add, k_lo);
    if constexpr (CB >= 2) {
        // 0x6400 + bytesum is the fp16 bit pattern of 1024 + s (exact for s <= 1020).  Byte sums
        // of differences against zero: v_sad_u8 adds s0 to 0x64006400, v_sad_hi_u8 adds s1 << 16,
        // which packs the pair (1024 + s1, 1024 + s0) in two ops with no carry between halves.
        const uint32_t lo = __builtin_amdgcn_sad_u8(x0, 0u, c6400);
        f16x2 h = __builtin_bit_cast(f16x2, __builtin_amdgcn_sad_hi_u8(x1, 0u, lo));
        if constexpr (CB == 2) {
            const f16x2 k_inv = {bits_f16(0x1EEEu), bits_f16(0x1EEEu)};
            const f16x2 k_bias = {bits_f16(0xC931u), bits_f16(0xC931u)};
            h = __builtin_elementwise_fma(h, k_inv, k_bias);       // v_pk_fma_f16: one rounding
        } else if constexpr (CB == 4) {
            // the byte sums themselves (exact: s <= 1020): int8 products v * s stay below 2^17
            // and a 128-input slice's sum below 2^24, so fp32 accumulation keeps it exact
            h = h - f16x2{(f16) 1024.0f, (f16) 1024.0f};
        }
        return __builtin_bit_cast(uint32_t, h);
    } else {
        // gather lo halves and hi halves of the two hashes, then the mask/xor (half-symmetric
        // constants commute with the byte permutation) and one packed fp16 add
        uint32_t lo = __builtin_amdgcn_perm(x1, x0, 0x05040100u);
        uint32_t hi = __builtin_amdgcn_perm(x1, x0, 0x07060302u);
        lo = (lo & 0x8FFF8FFFu) ^ 0x3B603B60u;
        hi = (hi & 0x8FFF8FFFu) ^ 0x3B603B60u;
        const f16x2 r = __builtin_bit_cast(f16x2, lo) + __builtin_bit_cast(f16x2, hi);
        return __builtin_bit_cast(uint32_t, r);
    }
}

template <int BITS, int CB, int I>
__device__ __forceinline__ void decode_pairs_rec(const uint32_t* W, uint32_t* P, uint32_t k_hi, uint32_t k_add,
                                                 uint32_t k_lo, uint32_t c6400)
{
    if constexpr (I < 16) {
        P[I] = decode_pair<BITS, CB, I>(W, k_hi, k_add, k_lo, c6400);
        decode_pairs_rec<BITS, CB, I + 1>(W, P, k_hi, k_add, k_lo, c6400);
    }
}

// Decode all 32 states of a q-block: P[i] = (state 2i, state 2i+1) as fp16 pairs.
// State p of q-block q is tile position t = 32q + p: column q + 8*((p>>2)&1),
// row 8*((p>>1)&1) + 2*(p>>3) + (p&1).
template <int BITS, int CB>
__device__ __forceinline__ void decode_qblock(const uint32_t* W, uint32_t* P)
{
    // constants live in SGPRs / one VGPR; the asm constraints keep them out of literals
    const uint32_t k_hi = Codebook<CB>::hi << 16;
    const uint32_t k_add = CB == 0 ? Codebook<0>::add : 0u;   // (CB 3 / 4: the mul1 hash, unscaled)
    const uint32_t k_lo = Codebook<CB>::lo;
    const uint32_t c6400 = 0x64006400u;
    decode_pairs_rec<BITS, CB, 0>(W, P, k_hi, k_add, k_lo, c6400);
}

// Load the BITS+1 words a lane needs for q-block q of a tile (tile32 = tile base as u32 words,
// a global-address-space pointer).
template <int BITS>
__device__ __forceinline__ void load_qblock(gc_u32* __restrict__ tile32, int q, uint32_t* W)
{
    gc_u32* p = tile32 + q * BITS;
    if constexpr (BITS % 4 == 0) {
#pragma unroll
        for (int i = 0; i < BITS / 4; ++i) {
            const u32x4 v = *reinterpret_cast<gc_u32x4*>(p + 4 * i);
            W[1 + 4 * i] = v[0]; W[2 + 4 * i] = v[1]; W[3 + 4 * i] = v[2]; W[4 + 4 * i] = v[3];
        }
    } else if constexpr (BITS % 2 == 0) {
#pragma unroll
        for (int i = 0; i < BITS / 2; ++i) {
            const u32x2 v = *reinterpret_cast<gc_u32x2*>(p + 2 * i);
            W[1 + 2 * i] = v[0]; W[2 + 2 * i] = v[1];
        }
    } else {
#pragma unroll
        for (int i = 0; i < BITS; ++i) W[1 + i] = p[i];
    }
    const int prev = q == 0 ? 8 * BITS - 1 : q * BITS - 1;
    W[0] = tile32[prev];
}

// The same q-block load from a uniform base plus per-lane byte offsets (32-bit): the loads then
// use the scalar-base + vector-offset address form, with no per-step address arithmetic.
// off_main addresses word q*BITS of the lane's tile, off_prev the ring predecessor word.
template <int BITS>
__device__ __forceinline__ void load_qblock_at(gc_u8* __restrict__ base, uint32_t off_main, uint32_t off_prev,
                                               uint32_t* W)
{
    gc_u8* p = base + off_main;
    if constexpr (BITS % 4 == 0) {
#pragma unroll
        for (int i = 0; i < BITS / 4; ++i) {
            const u32x4 v = *reinterpret_cast<gc_u32x4*>(p + 16 * i);
            W[1 + 4 * i] = v[0]; W[2 + 4 * i] = v[1]; W[3 + 4 * i] = v[2]; W[4 + 4 * i] = v[3];
        }
    } else if constexpr (BITS % 2 == 0) {
#pragma unroll
        for (int i = 0; i < BITS / 2; ++i) {
            const u32x2 v = *reinterpret_cast<gc_u32x2*>(p + 8 * i);
            W[1 + 2 * i] = v[0]; W[2 + 2 * i] = v[1];
        }
    } else {
#pragma unroll
        for (int i = 0; i < BITS; ++i) W[1 + i] = *reinterpret_cast<gc_u32*>(p + 4 * i);
    }
    W[0] = *reinterpret_cast<gc_u32*>(base + off_prev);
}

// s_waitcnt immediate waiting for vmcnt <= n (n < 64) only (gfx9 encoding: vmcnt bits 3:0 and
// 15:14, expcnt 6:4 and lgkmcnt 11:8 at their no-wait maxima)
constexpr int vmcnt_imm(int n)
{
    return (n & 0xF) | ((n >> 4) << 14) | 0x0F70;
}

// Vector-memory instructions of one load_qblock_buf call (for explicit vmcnt waits).  The main
// words go out as the fewest loads that can carry them (16-byte loads, then one 12/8/4-byte load
// of the rest), so no load of the call can be merged with another (no load is wider than 16 bytes)
// and the count cannot shrink under the compiler; the ring predecessor is one more.
template <int BITS>
constexpr int qblock_loads()
{
    return (BITS + 3) / 4 + 1;
}

// Buffer-resource form: the trellis is one raw buffer (dword 3 of the resource: gfx9 raw 32-bit
// format), the unit's byte offset a scalar, the lane's byte offsets fixed VGPRs.  No address
// arithmetic per load, and the hardware range check turns any stray offset into zeros.
constexpr int RAW_BUFFER_FLAGS = 0x00020000;
// cache-policy operand of buffer loads / stores: device scope (sc1).  Stores write through the
// XCD's L2; loads miss it, so they see device-scope stores from any XCD.
constexpr int SC1 = 0x10;

typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

// The lane's BITS main words as BITS / 4 16-byte loads and one load of the BITS % 4 remaining
// words (dword-aligned multi-word buffer loads), then the ring predecessor: qblock_loads<BITS>()
// instructions exactly.
template <int BITS>
__device__ __forceinline__ void load_qblock_buf(__amdgpu_buffer_rsrc_t rsrc, uint32_t off_main, uint32_t off_prev,
                                                uint32_t soff, uint32_t* W)
{
#pragma unroll
    for (int i = 0; i < BITS / 4; ++i) {
        const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off_main + 16 * i, soff, 0));
        W[1 + 4 * i] = v[0]; W[2 + 4 * i] = v[1]; W[3 + 4 * i] = v[2]; W[4 + 4 * i] = v[3];
    }
    constexpr int B = 4 * (BITS / 4), R = BITS % 4;
    if constexpr (R == 3) {
        const u32x3 v = __builtin_bit_cast(u32x3, __builtin_amdgcn_raw_buffer_load_b96(rsrc, off_main + 4 * B, soff, 0));
        W[1 + B] = v[0]; W[2 + B] = v[1]; W[3 + B] = v[2];
    } else if constexpr (R == 2) {
        const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rsrc, off_main + 4 * B, soff, 0));
        W[1 + B] = v[0]; W[2 + B] = v[1];
    } else if constexpr (R == 1) {
        W[1 + B] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, off_main + 4 * B, soff, 0);
    }
    W[0] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, off_prev, soff, 0);
}

}  // namespace exl3
