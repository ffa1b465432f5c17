// exl3_gemm.hip -- prefill (large-M) EXL3 linear and dense fp16 GEMM for gfx950.
//
// exl3_gemm_trellis: y = had_out(fp16(had_in(x) . W), svh) in three launches:
//   1. had_in   xh = fp16(Had128(fp16(x * suh)))                       (had_kernel)
//   2. GEMM     C = fp16(xh . W): 128x128 output tile per workgroup, K step 64; every step the
//               workgroup decodes its 4x8 trellis tiles (one q-block per thread) straight into
//               LDS in MFMA B-fragment order and stages the matching xh rows in A-fragment
//               order; v_mfma_f32_16x16x32_f16 with fp32 accumulation.  LDS is double-buffered
//               so the decode of step i+1 overlaps the MFMAs of step i.
//   3. had_out  y = fp16(fp16(Had128(C)) * svh)                        (had_kernel, in place)
// exl3_hgemm_recon is the same GEMM with a dense fp16 W[k, n] as the B source.
#include "exl3_device.h"
#include "../../include/exl3_mi355x.h"

#include <stdlib.h>

using namespace exl3;

namespace {

constexpr int MT_ROWS = 128, NT_COLS = 128, KSTEP = 64;
constexpr int FRAG_BYTES = 2 * 8 * 64 * 16;          // [ks 2][tile 8][lane 64][16 B] = 16 KB

// A fragment slot of the 8 halves x[row][kbase + 8c .. +8] (c = 0..7 within the K step):
// MFMA k-substep ks = c / 4, lane group = c % 4, lane = group*16 + row % 16, tile = row / 16.
__device__ __forceinline__ int afrag_off(int row, int c) { return (((c >> 2) * 8 + (row >> 4)) * 64 + (c & 3) * 16 + (row & 15)) * 16; }

template <int BITS, int CB>
struct TrellisB {
    const uint32_t* trellis;
    int nt_total;
    // thread t decodes q-block (t & 7) of tile (k-tile t >> 6, n-tile (t >> 3) & 7) of the step
    __device__ __forceinline__ void fetch(int kt0, int nt0, int t, uint32_t* W) const
    {
        const int ktl = t >> 6, ntl = (t >> 3) & 7, q = t & 7;
        gc_u32* tp = as_global(trellis) + ((int64_t) (kt0 + ktl) * nt_total + nt0 + ntl) * (8 * BITS);
        load_qblock<BITS>(tp, q, W);
    }
    __device__ __forceinline__ void decode_store(const uint32_t* W, int t, char* bfrag) const
    {
        uint32_t P[16];
        decode_qblock<BITS, CB>(W, P);
        const int ktl = t >> 6, ntl = (t >> 3) & 7, q = t & 7;
        const int ks = ktl >> 1;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int rh = 0; rh < 2; ++rh) {
                const int lane = (2 * (ktl & 1) + rh) * 16 + q + 8 * h;
                const u32x4 v = {P[2 * h + rh], P[4 + 2 * h + rh], P[8 + 2 * h + rh], P[12 + 2 * h + rh]};
                *reinterpret_cast<u32x4*>(bfrag + ((ks * 8 + ntl) * 64 + lane) * 16) = v;
            }
    }
};

// Dense B fragments: lane (group g, column c) of column tile ct holds W[kbase + 32 ks + 8 g + 0..7][16 ct + c].
template <class BSRC, bool DENSE>
__global__ void __launch_bounds__(256) gemm_kernel(const uint16_t* __restrict__ xh, int64_t ldx, BSRC bsrc,
                                                   const uint16_t* __restrict__ Wd, int64_t ldw,
                                                   uint16_t* __restrict__ y, int64_t ldy, int M, int K, int N,
                                                   int xcd_remap)
{
    __shared__ __align__(16) char lds[2][2 * FRAG_BYTES];      // [buffer][A frags | B frags]
    const int t = threadIdx.x;
    const int tiles_n = N / NT_COLS, tiles_m = (M + MT_ROWS - 1) / MT_ROWS;
    int tm, tn;
    {
        const int b = blockIdx.x, total = tiles_m * tiles_n;
        const int u = xcd_remap ? (b & 7) * (total / 8) + (b >> 3) : b;   // consecutive units share an XCD
        tm = u / tiles_n;
        tn = u % tiles_n;
    }
    const int row0 = tm * MT_ROWS, col0 = tn * NT_COLS;
    const int steps = K / KSTEP;
    const int wave = t >> 6, lane = t & 63;
    const int wr = wave >> 1, wc = wave & 1;

    // ---- staging helpers -------------------------------------------------------------------
    auto load_a = [&](int st, u32x4* av) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int seg = t + 256 * i;                 // 128 rows x 8 segments of 8 halves
            const int row = seg >> 3, c = seg & 7;
            const int gr = row0 + row;
            u32x4 v = {0u, 0u, 0u, 0u};
            if (gr < M) v = *reinterpret_cast<const u32x4*>(xh + (int64_t) gr * ldx + st * KSTEP + c * 8);
            av[i] = v;
        }
    };
    auto store_a = [&](int buf, const u32x4* av) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int seg = t + 256 * i;
            *reinterpret_cast<u32x4*>(&lds[buf][afrag_off(seg >> 3, seg & 7)]) = av[i];
        }
    };
    // dense B: thread owns column (t & 127) of the step, 32-row half (t >> 7): 4 slots of 8 rows
    auto load_bd = [&](int st, uint16_t (*bv)[8]) {
        const int c = t & 127, half = t >> 7;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                bv[s][e] = Wd[(int64_t) (st * KSTEP + half * 32 + s * 8 + e) * ldw + col0 + c];
    };
    auto store_bd = [&](int buf, uint16_t (*bv)[8]) {
        const int c = t & 127, half = t >> 7;
        char* bf = &lds[buf][FRAG_BYTES];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int krow = half * 32 + s * 8;           // k offset within the step
            const int ks = krow >> 5, g = (krow >> 3) & 3;
            const int ct = c >> 4, ln = g * 16 + (c & 15);
            u32x4 v;
            v[0] = bv[s][0] | ((uint32_t) bv[s][1] << 16);
            v[1] = bv[s][2] | ((uint32_t) bv[s][3] << 16);
            v[2] = bv[s][4] | ((uint32_t) bv[s][5] << 16);
            v[3] = bv[s][6] | ((uint32_t) bv[s][7] << 16);
            *reinterpret_cast<u32x4*>(bf + ((ks * 8 + ct) * 64 + ln) * 16) = v;
        }
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 av[4];
    uint32_t Wt[9];
    uint16_t bv[4][8];
    // prologue: stage step 0
    load_a(0, av);
    if constexpr (DENSE) load_bd(0, bv);
    else bsrc.fetch(0, col0 / 16, t, Wt);
    store_a(0, av);
    if constexpr (DENSE) store_bd(0, bv);
    else bsrc.decode_store(Wt, t, &lds[0][FRAG_BYTES]);
    __syncthreads();

    for (int st = 0; st < steps; ++st) {
        const int cur = st & 1;
        const bool more = st + 1 < steps;
        if (more) {
            load_a(st + 1, av);
            if constexpr (DENSE) load_bd(st + 1, bv);
            else bsrc.fetch((st + 1) * 4, col0 / 16, t, Wt);
        }
        // MFMAs on the current buffer
        const char* af = &lds[cur][0];
        const char* bf = &lds[cur][FRAG_BYTES];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            f16x8 A[4], B[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                A[i] = *reinterpret_cast<const f16x8*>(af + ((ks * 8 + wr * 4 + i) * 64 + lane) * 16);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                B[j] = *reinterpret_cast<const f16x8*>(bf + ((ks * 8 + wc * 4 + j) * 64 + lane) * 16);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[i], B[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            store_a(cur ^ 1, av);
            if constexpr (DENSE) store_bd(cur ^ 1, bv);
            else bsrc.decode_store(Wt, t, &lds[cur ^ 1][FRAG_BYTES]);
        }
        __syncthreads();
    }

    // ---- epilogue: C = fp16(acc); lane holds rows 4*(lane>>4)+v of column lane&15 ----------------
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int r = row0 + wr * 64 + i * 16 + 4 * (lane >> 4) + v;
                const int c = col0 + wc * 64 + j * 16 + (lane & 15);
                if (r < M) y[(int64_t) r * ldy + c] = f16_bits((f16) acc[i][j][v]);
            }
}

int codebook_of(int mcg, int mul1) { return mul1 ? 2 : (mcg ? 1 : 0); }

template <int BITS, int CB>
int launch_trellis_gemm(const uint16_t* xh, int64_t ldx, const void* trellis, uint16_t* y, int64_t ldy, int M, int K,
                        int N, hipStream_t s)
{
    TrellisB<BITS, CB> b{(const uint32_t*) trellis, N / 16};
    const int total = ((M + MT_ROWS - 1) / MT_ROWS) * (N / NT_COLS);
    hipLaunchKernelGGL((gemm_kernel<TrellisB<BITS, CB>, false>), dim3(total), dim3(256), 0, s, xh, ldx, b,
                       (const uint16_t*) nullptr, (int64_t) 0, y, ldy, M, K, N, (int) (total % 8 == 0));
    return hipGetLastError() == hipSuccess ? EXL3_OK : EXL3_ELAUNCH;
}

template <int BITS>
int launch_trellis_gemm_cb(int cb, const uint16_t* xh, int64_t ldx, const void* tr, uint16_t* y, int64_t ldy, int M,
                           int K, int N, hipStream_t s)
{
    if (cb == 0) return launch_trellis_gemm<BITS, 0>(xh, ldx, tr, y, ldy, M, K, N, s);
    if (cb == 1) return launch_trellis_gemm<BITS, 1>(xh, ldx, tr, y, ldy, M, K, N, s);
    return launch_trellis_gemm<BITS, 2>(xh, ldx, tr, y, ldy, M, K, N, s);
}

}  // namespace

extern "C" {

int exl3_hgemm_recon(const void* x, int64_t ldx, const void* W, int64_t ldw, void* y, int64_t ldy, int m, int k, int n,
                     void* stream)
{
    if (!x || !W || !y || m < 0 || k % KSTEP || n % NT_COLS || k < KSTEP || n < NT_COLS || ldx < k || ldw < n ||
        ldy < n || ldx % 8 || (((uintptr_t) x) & 15) || (((uintptr_t) W) & 1) || (((uintptr_t) y) & 1))
        return EXL3_EINVAL;
    if (m == 0) return EXL3_OK;
    const int total = ((m + MT_ROWS - 1) / MT_ROWS) * (n / NT_COLS);
    TrellisB<1, 2> unused{nullptr, 0};
    hipLaunchKernelGGL((gemm_kernel<TrellisB<1, 2>, true>), dim3(total), dim3(256), 0, (hipStream_t) stream,
                       (const uint16_t*) x, ldx, unused, (const uint16_t*) W, ldw, (uint16_t*) y, ldy, m, k, n,
                       (int) (total % 8 == 0));
    return hipGetLastError() == hipSuccess ? EXL3_OK : EXL3_ELAUNCH;
}

int exl3_gemm_trellis(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh, void* xh,
                      const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* stream)
{
    if (!x || !trellis || !y || !suh || !xh || !svh || m < 0 || K < 1 || K > 8 || k % 128 || n % 128 || k < 128 ||
        n < 128 || ldx < k || ldy < n || ldx % 2 || ldy % 2 || (((uintptr_t) xh) & 15) || (((uintptr_t) trellis) & 15))
        return EXL3_EINVAL;
    if (m == 0) return EXL3_OK;
    int rc = exl3_had_r_128(x, ldx, xh, k, m, k, suh, nullptr, 1.0f, stream);
    if (rc) return rc;
    const int cb = codebook_of(mcg, mul1);
    hipStream_t s = (hipStream_t) stream;
    const uint16_t* xhp = (const uint16_t*) xh;
    uint16_t* yp = (uint16_t*) y;
    switch (K) {
        case 1: rc = launch_trellis_gemm_cb<1>(cb, xhp, k, trellis, yp, ldy, m, k, n, s); break;
        case 2: rc = launch_trellis_gemm_cb<2>(cb, xhp, k, trellis, yp, ldy, m, k, n, s); break;
        case 3: rc = launch_trellis_gemm_cb<3>(cb, xhp, k, trellis, yp, ldy, m, k, n, s); break;
        case 4: rc = launch_trellis_gemm_cb<4>(cb, xhp, k, trellis, yp, ldy, m, k, n, s); break;
        case 5: rc = launch_trellis_gemm_cb<5>(cb, xhp, k, trellis, yp, ldy, m, k, n, s); break;
        case 6: rc = launch_trellis_gemm_cb<6>(cb, xhp, k, trellis, yp, ldy, m, k, n, s); break;
        case 7: rc = launch_trellis_gemm_cb<7>(cb, xhp, k, trellis, yp, ldy, m, k, n, s); break;
        default: rc = launch_trellis_gemm_cb<8>(cb, xhp, k, trellis, yp, ldy, m, k, n, s); break;
    }
    if (rc) return rc;
    return exl3_had_r_128(y, ldy, y, ldy, m, n, nullptr, svh, 1.0f, stream);
}

int exl3_gemm(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh, void* A_had,
              const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
              void* stream)
{
    if (m <= 0) return m == 0 ? 1 : EXL3_EINVAL;
    if (m <= EXL3_GEMV_MAX_ROWS) {
        const int rc = exl3_gemv_mr(x, ldx, trellis, y, ldy, suh, A_had, svh, m, k, n, K, mcg, mul1, workspace,
                                    ws_bytes, stream);
        return rc == EXL3_OK ? 1 : (rc > 0 ? EXL3_EINVAL : rc);
    }
    const int rc = exl3_gemm_trellis(x, ldx, trellis, y, ldy, suh, A_had, svh, m, k, n, K, mcg, mul1, stream);
    return rc == EXL3_OK ? 2 : rc;
}

}  // extern "C"
