// exl3_gemm.hip -- prefill (large-M) EXL3 linear and dense fp16 GEMM for gfx950.
//
// exl3_gemm_trellis: y = had_out(fp16(had_in(x) . W), svh) in two launches:
//   1. had_in   xh = fp16(Had128(fp16(x * suh)))                       (had_kernel)
//   2. GEMM     C = fp16(xh . W) on 128 x 128 output tiles, K step 64: each step the workgroup
//               decodes its 4 x 8 trellis tiles (one q-block per thread) straight into LDS in
//               MFMA B-fragment order and stages the xh rows in A-fragment order;
//               v_mfma_f32_16x16x32_f16, fp32 accumulation; LDS double-buffered.  The epilogue
//               applies y = fp16(fp16(Had128(C)) * svh) to the tile's whole 128-column blocks.
// exl3_hgemm_recon is the same GEMM with a dense fp16 W[k, n] as the B source and a plain
// fp16 C epilogue.
#include "exl3_device.h"
#include "../../include/exl3_mi355x.h"

#include <stdlib.h>

using namespace exl3;

namespace {

constexpr int NT_COLS = 128, KSTEP = 64;
// Workgroup tile rows.  128 (LDS 64 KB, two workgroups per CU whose MFMA and decode phases
// overlap) measured faster on MI355X than 256-row tiles with one workgroup per CU, with four
// waves interleaving their own MFMAs and decode or with eight waves split into decoders and
// MFMA-only waves.
constexpr int GEMM_MT = 128;
constexpr int FRAG = 64 * 16;                          // one MFMA operand tile: 64 lanes x 16 B

// A fragment tile T = ks * RT + r (RT = row tiles of the workgroup tile) holds, in lane g*16 + i,
// the 8 halves x[16 r + i][kbase + 32 ks + 8 g .. +8].  Store i of wave w fills tile w + 4 i with
// its 64 lanes: contiguous 1 KB per store.
// B fragment tile ks * 8 + j (n-tile j of the step) holds, in lane g*16 + c, the 8 halves
// W[kbase + 32 ks + 8 g .. +8][16 j + c]; its lanes are stored XOR-swizzled by bswz(j) so that the
// decoders' stores (one wave = 8 n-tiles x 8 q-blocks) spread over all LDS banks, while every
// 16- and 32-lane group of an MFMA operand read still covers a contiguous 256 / 512 bytes.
__device__ __forceinline__ int bswz(int j) { return ((j & 1) << 3) | ((j & 2) << 3); }

// 4 waves in 2 x 2, each (MT / 2) x 64; every thread decodes one q-block per step.
template <int MT>
struct Tile {
    static constexpr int WR = 2;                       // wave rows (waves = WR x 2)
    static constexpr int THREADS = 128 * WR;
    static constexpr int RT = MT / 16;                 // A row tiles
    static constexpr int MI = MT / 32;                 // MFMA row tiles per wave
    static constexpr int A_BYTES = 2 * RT * FRAG;      // two k-substeps
    static constexpr int B_BYTES = 2 * 8 * FRAG;
    static constexpr int BUF = A_BYTES + B_BYTES;
    static constexpr int A_PER_WAVE = 2 * RT / (2 * WR);   // A tiles staged per wave and step (4)
    static constexpr int C_ROW = 136;                  // LDS row (halves) of the C tile in the epilogue
    static constexpr int LDS = 2 * BUF > MT * C_ROW * 2 ? 2 * BUF : MT * C_ROW * 2;
};

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
                const int lane = ((2 * (ktl & 1) + rh) * 16 + q + 8 * h) ^ bswz(ntl);
                const u32x4 v = {P[2 * h + rh], P[4 + 2 * h + rh], P[8 + 2 * h + rh], P[12 + 2 * h + rh]};
                *reinterpret_cast<u32x4*>(bfrag + ((ks * 8 + ntl) * 64 + lane) * 16) = v;
            }
    }
};

// Workgroup tile MT x 128 (waves as in Tile), K step 64, LDS double-buffered.
// Iteration st: the global loads for step st + 1 (x) and st + 2 (trellis) go out, the MFMAs of
// step st run on buffer st & 1 while the same basic block decodes step st + 1 into the other
// buffer (the last iteration restages the last step into the unused buffer: in bounds, never
// read).  FUSE_OUT: the epilogue stages fp16 C in LDS and applies y = fp16(fp16(Had128(C)) * svh)
// row by row (the tile holds whole 128-column blocks); otherwise it stores C.
template <class BSRC, bool DENSE, int MT, bool FUSE_OUT>
__global__ void __launch_bounds__(Tile<MT>::THREADS) gemm_kernel(const uint16_t* __restrict__ xh, int64_t ldx, BSRC bsrc,
                                                   const uint16_t* __restrict__ Wd, int64_t ldw,
                                                   uint16_t* __restrict__ y, int64_t ldy,
                                                   const uint16_t* __restrict__ svh, int M, int K, int N,
                                                   int xcd_remap)
{
    using TL = Tile<MT>;
    extern __shared__ __align__(16) char lds[];
    const int t = threadIdx.x;
    const int tiles_n = N / NT_COLS, tiles_m = (M + MT - 1) / MT;
    int tm, tn;
    {
        const int b = blockIdx.x, total = tiles_m * tiles_n;
        const int u = xcd_remap ? (b & 7) * (total / 8) + (b >> 3) : b;   // consecutive units share an XCD
        tm = u / tiles_n;
        tn = u % tiles_n;
    }
    const int row0 = tm * MT, col0 = tn * NT_COLS;
    const int steps = K / KSTEP;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
    const int wr = wave >> 1, wc = wave & 1;

    auto load_a = [&](int st, u32x4* av) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TL::A_PER_WAVE; ++i) {
            const int T = wave + 2 * TL::WR * i;
            const int row = (T % TL::RT) * 16 + (lane & 15), kc = (T / TL::RT) * 32 + (lane >> 4) * 8;
            const int gr = row0 + row;
            u32x4 v = {0u, 0u, 0u, 0u};
            if (gr < M) v = *reinterpret_cast<const u32x4*>(xh + (int64_t) gr * ldx + st * KSTEP + kc);
            av[i] = v;
        }
    };
    auto store_a = [&](char* buf, const u32x4* av) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TL::A_PER_WAVE; ++i)
            *reinterpret_cast<u32x4*>(buf + ((wave + 2 * TL::WR * i) * 64 + lane) * 16) = av[i];
    };
    // dense B: thread owns column (t & 127) of the step, 32-row half (t >> 7): 4 slots of 8 rows
    auto load_bd = [&](int st, uint16_t (*bv)[8]) __attribute__((always_inline)) {
        const int c = t & 127, half = t >> 7;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                bv[s][e] = Wd[(int64_t) (st * KSTEP + half * 32 + s * 8 + e) * ldw + col0 + c];
    };
    auto store_bd = [&](char* bf, uint16_t (*bv)[8]) __attribute__((always_inline)) {
        const int c = t & 127, half = t >> 7;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int krow = half * 32 + s * 8;           // k offset within the step
            const int ks = krow >> 5, g = (krow >> 3) & 3;
            const int ct = c >> 4, ln = (g * 16 + (c & 15)) ^ bswz(ct);
            u32x4 v;
            v[0] = bv[s][0] | ((uint32_t) bv[s][1] << 16);
            v[1] = bv[s][2] | ((uint32_t) bv[s][3] << 16);
            v[2] = bv[s][4] | ((uint32_t) bv[s][5] << 16);
            v[3] = bv[s][6] | ((uint32_t) bv[s][7] << 16);
            *reinterpret_cast<u32x4*>(bf + ((ks * 8 + ct) * 64 + ln) * 16) = v;
        }
    };

    f32x4 acc[TL::MI][4];
#pragma unroll
    for (int i = 0; i < TL::MI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // x tiles and trellis words are fetched two steps ahead of their use (register double buffers)
    u32x4 avx[TL::A_PER_WAVE], avy[TL::A_PER_WAVE];
    uint32_t Wc[9], Wn[9];
    uint16_t bv[4][8];
    char* const buf0 = lds;
    char* const buf1 = lds + TL::BUF;
    // prologue: stage step 0 into buffer 0; x of step 1 and the trellis of step 1 are in flight
    load_a(0, avx);
    if constexpr (DENSE) load_bd(0, bv);
    else bsrc.fetch(0, col0 / 16, t, Wc);
    store_a(buf0, avx);
    if constexpr (DENSE) {
        store_bd(buf0 + TL::A_BYTES, bv);
    } else {
        bsrc.decode_store(Wc, t, buf0 + TL::A_BYTES);
        bsrc.fetch(min(1, steps - 1) * 4, col0 / 16, t, Wc);
    }
    load_a(min(1, steps - 1), avy);
    __syncthreads();

    // one step: av_next holds x of step st + 1 (fetched an iteration ago), av_load receives step st + 2
    auto step = [&](int st, u32x4* av_next, u32x4* av_load) __attribute__((always_inline)) {
        char* const cur = (st & 1) ? buf1 : buf0;
        char* const nxt = (st & 1) ? buf0 : buf1;
        const int s1 = min(st + 1, steps - 1), s2 = min(st + 2, steps - 1);
        load_a(s2, av_load);
        if constexpr (DENSE) load_bd(s1, bv);
        else bsrc.fetch(s2 * 4, col0 / 16, t, Wn);
        // MFMAs on the current buffer
        const char* af = cur;
        const char* bf = cur + TL::A_BYTES;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            f16x8 A[TL::MI], B[4];
#pragma unroll
            for (int i = 0; i < TL::MI; ++i)
                A[i] = *reinterpret_cast<const f16x8*>(af + ((ks * TL::RT + wr * TL::MI + i) * 64 + lane) * 16);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                B[j] = *reinterpret_cast<const f16x8*>(bf + ((ks * 8 + wc * 4 + j) * 64 + (lane ^ bswz(wc * 4 + j))) * 16);
#pragma unroll
            for (int i = 0; i < TL::MI; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[i], B[j], acc[i][j], 0, 0, 0);
        }
        // Keep the MFMA phase and the decode phase apart: a wave interleaving its own MFMAs with
        // VALU work runs slower here than two workgroups per CU overlapping their phases.
        __builtin_amdgcn_sched_barrier(0);
        // stage step st + 1 into the other buffer (free since the previous iteration's barrier); the
        // last iteration restages the last step into the unused buffer (in bounds, never read)
        store_a(nxt, av_next);
        if constexpr (DENSE) {
            store_bd(nxt + TL::A_BYTES, bv);
        } else {
            bsrc.decode_store(Wc, t, nxt + TL::A_BYTES);
#pragma unroll
            for (int i = 0; i < 9; ++i) Wc[i] = Wn[i];
        }
        __syncthreads();
    };
    int st = 0;
    for (; st + 1 < steps; st += 2) {
        step(st, avy, avx);
        step(st + 1, avx, avy);
    }
    if (st < steps) step(st, avy, avx);

    // ---- epilogue: lane holds rows 4*(lane>>4)+v of column lane&15 of each 16 x 16 tile ----------
    if constexpr (FUSE_OUT) {
        uint16_t* ct = reinterpret_cast<uint16_t*>(lds);          // [MT][C_ROW] fp16 C (buffers are free)
#pragma unroll
        for (int i = 0; i < TL::MI; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int r = wr * (MT / 2) + i * 16 + 4 * (lane >> 4) + v;
                    const int c = wc * 64 + j * 16 + (lane & 15);
                    ct[r * TL::C_ROW + c] = f16_bits((f16) acc[i][j][v]);
                }
        __syncthreads();
        // 16 lanes per row: y = fp16(fp16(Had128(C)) * svh), 16-byte stores
        const int l16 = t & 15;
        const u32x4 sv = *reinterpret_cast<const u32x4*>(svh + col0 + 8 * l16);
        for (int r0 = 0; r0 < MT; r0 += TL::THREADS / 16) {
            const int r = r0 + (t >> 4);
            const u32x4 c = *reinterpret_cast<const u32x4*>(ct + r * TL::C_ROW + 8 * l16);
            const u32x4 res = had128_x8(c, u32x4{0u, 0u, 0u, 0u}, false, sv, true, R_SCALE);
            if (row0 + r < M) *reinterpret_cast<u32x4*>(y + (int64_t) (row0 + r) * ldy + col0 + 8 * l16) = res;
        }
    } else {
#pragma unroll
        for (int i = 0; i < TL::MI; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int r = row0 + wr * (MT / 2) + i * 16 + 4 * (lane >> 4) + v;
                    const int c = col0 + wc * 64 + j * 16 + (lane & 15);
                    if (r < M) y[(int64_t) r * ldy + c] = f16_bits((f16) acc[i][j][v]);
                }
    }
}

int codebook_of(int mcg, int mul1) { return mul1 ? 2 : (mcg ? 1 : 0); }

template <class BSRC, bool DENSE, int MT, bool FUSE>
int launch_gemm(const uint16_t* xh, int64_t ldx, BSRC b, const uint16_t* Wd, int64_t ldw, uint16_t* y, int64_t ldy,
                const uint16_t* svh, int M, int K, int N, hipStream_t s)
{
    auto kern = gemm_kernel<BSRC, DENSE, MT, FUSE>;
    static bool attr_set = false;            // dynamic LDS above 64 KB must be enabled per kernel
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*) kern, hipFuncAttributeMaxDynamicSharedMemorySize, Tile<MT>::LDS) !=
            hipSuccess)
            return EXL3_ELAUNCH;
        attr_set = true;
    }
    const int total = ((M + MT - 1) / MT) * (N / NT_COLS);
    hipLaunchKernelGGL(kern, dim3(total), dim3(Tile<MT>::THREADS), Tile<MT>::LDS, s, xh, ldx, b, Wd, ldw, y, ldy, svh, M, K, N,
                       (int) (total % 8 == 0));
    return hipGetLastError() == hipSuccess ? EXL3_OK : EXL3_ELAUNCH;
}

template <int BITS, int CB>
int launch_trellis_gemm(const uint16_t* xh, int64_t ldx, const void* trellis, uint16_t* y, int64_t ldy,
                        const uint16_t* svh, int M, int K, int N, hipStream_t s)
{
    TrellisB<BITS, CB> b{(const uint32_t*) trellis, N / 16};
    return launch_gemm<TrellisB<BITS, CB>, false, GEMM_MT, true>(xh, ldx, b, nullptr, 0, y, ldy, svh, M, K, N, s);
}

template <int BITS>
int launch_trellis_gemm_cb(int cb, const uint16_t* xh, int64_t ldx, const void* tr, uint16_t* y, int64_t ldy,
                           const uint16_t* svh, int M, int K, int N, hipStream_t s)
{
    if (cb == 0) return launch_trellis_gemm<BITS, 0>(xh, ldx, tr, y, ldy, svh, M, K, N, s);
    if (cb == 1) return launch_trellis_gemm<BITS, 1>(xh, ldx, tr, y, ldy, svh, M, K, N, s);
    return launch_trellis_gemm<BITS, 2>(xh, ldx, tr, y, ldy, svh, M, K, N, s);
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
    TrellisB<1, 2> unused{nullptr, 0};
    return launch_gemm<TrellisB<1, 2>, true, GEMM_MT, false>((const uint16_t*) x, ldx, unused, (const uint16_t*) W,
                                                             ldw, (uint16_t*) y, ldy, nullptr, m, k, n,
                                                             (hipStream_t) stream);
}

int exl3_gemm_trellis(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh, void* xh,
                      const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* stream)
{
    if (!x || !trellis || !y || !suh || !xh || !svh || m < 0 || K < 1 || K > 8 || k % 128 || n % 128 || k < 128 ||
        n < 128 || ldx < k || ldy < n || ldx % 8 || ldy % 8 || (((uintptr_t) xh) & 15) || (((uintptr_t) y) & 15) ||
        (((uintptr_t) svh) & 15) || (((uintptr_t) trellis) & 15))
        return EXL3_EINVAL;
    if (m == 0) return EXL3_OK;
    int rc = exl3_had_r_128(x, ldx, xh, k, m, k, suh, nullptr, 1.0f, stream);
    if (rc) return rc;
    const int cb = codebook_of(mcg, mul1);
    hipStream_t s = (hipStream_t) stream;
    const uint16_t* xhp = (const uint16_t*) xh;
    uint16_t* yp = (uint16_t*) y;
    const uint16_t* sv = (const uint16_t*) svh;
    switch (K) {
        case 1: return launch_trellis_gemm_cb<1>(cb, xhp, k, trellis, yp, ldy, sv, m, k, n, s);
        case 2: return launch_trellis_gemm_cb<2>(cb, xhp, k, trellis, yp, ldy, sv, m, k, n, s);
        case 3: return launch_trellis_gemm_cb<3>(cb, xhp, k, trellis, yp, ldy, sv, m, k, n, s);
        case 4: return launch_trellis_gemm_cb<4>(cb, xhp, k, trellis, yp, ldy, sv, m, k, n, s);
        case 5: return launch_trellis_gemm_cb<5>(cb, xhp, k, trellis, yp, ldy, sv, m, k, n, s);
        case 6: return launch_trellis_gemm_cb<6>(cb, xhp, k, trellis, yp, ldy, sv, m, k, n, s);
        case 7: return launch_trellis_gemm_cb<7>(cb, xhp, k, trellis, yp, ldy, sv, m, k, n, s);
        default: return launch_trellis_gemm_cb<8>(cb, xhp, k, trellis, yp, ldy, sv, m, k, n, s);
    }
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
