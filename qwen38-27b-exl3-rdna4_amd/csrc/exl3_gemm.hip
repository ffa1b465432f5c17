// exl3_gemm.hip -- prefill (large-M) EXL3 linear and dense fp16 GEMM for gfx950.
//
// exl3_gemm_trellis: y = had_out(fp16(had_in(x) . W), svh) in two launches:
//   1. had_in   xh = fp16(Had128(fp16(x * suh)))    (had_mfma_kernel: fp32 sums on the matrix cores)
//   2. GEMM     C = fp16(xh . W): the producer / consumer kernel below (256 x 128 tiles), or for
//               operands beyond 32-bit buffer offsets the 128 x 128 kernel here, K step 64: each
//               step the workgroup decodes its 4 x 8 trellis tiles (one q-block per thread)
//               straight into LDS in MFMA B-fragment order and stages the xh rows in A-fragment
//               order; v_mfma_f32_16x16x32_f16, fp32 accumulation; LDS double-buffered.  Both
//               epilogues apply y = fp16(fp16(Had128(C)) * svh) to the tile's whole 128-column
//               blocks on the matrix cores (had128_mfma16, the values of exl3_had_r_128_f32; the
//               rows are checked to the rel-L2 bar).
// exl3_hgemm_recon is the same GEMM with a dense fp16 W[k, n] as the B source and a plain
// fp16 C epilogue.
#include "exl3_device.h"
#include "../../include/exl3_mi355x.h"

#include <stdlib.h>

#include <algorithm>

using namespace exl3;

// had_r_128 of one input into several outputs in one launch (exl3_gemv.hip)
int launch_had(const void* in, int64_t ld_in, void* const* out, int64_t ld_out, int rows, int cols, const void* const* pre,
               int groups, const void* post, float scale, void* stream, bool exact, const void* in_up);

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
        // y = fp16(fp16(Had128(C)) * svh) on the matrix cores, 16 rows per wave pass
        // (had128_mfma16: the values of exl3_had_r_128_f32 with post), 16-byte stores
        const int jr = t & 15, gq = (t >> 4) & 3;
        u32x4 sv[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) sv[p] = *reinterpret_cast<const u32x4*>(svh + col0 + 32 * p + 8 * gq);
        const HadMfmaA HA = had_mfma_a();
        for (int rg = t >> 6; rg < MT / 16; rg += TL::THREADS / 64) {
            const int r = rg * 16 + jr;
            u32x4 xb[4];
#pragma unroll
            for (int s_ = 0; s_ < 4; ++s_) xb[s_] = *reinterpret_cast<const u32x4*>(ct + r * TL::C_ROW + 32 * s_ + 8 * gq);
            had128_mfma16(HA, xb, r_scale<float>(), true, sv, [&](int p, u32x4 v) __attribute__((always_inline)) {
                if (row0 + r < M) *reinterpret_cast<u32x4*>(y + (int64_t) (row0 + r) * ldy + col0 + 32 * p + 8 * gq) = v;
            });
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

// ============================================================================================
// Producer / consumer prefill GEMM (trellis B).  Tile 256 x 128, K step 64, one workgroup of
// 8 waves per CU:
//   waves 0-3 (consumers, one per SIMD): wave w owns rows 64w .. 64w+63 of the tile, all 128
//     columns (4 x 8 MFMA tiles of 16 x 16, fp32 accumulators in registers); it only reads A and B
//     fragments from LDS and issues v_mfma_f32_16x16x32_f16;
//   waves 4-7 (producers, one per SIMD) decode the trellis tiles of the next K step (one q-block
//     per lane) into LDS in B-fragment order and request the xh rows of the step after it
//     straight into LDS (buffer loads with the lds bit: no registers, no LDS store instructions).
// Every SIMD pairs one MFMA wave with one VALU wave for the whole loop, so matrix and vector work
// overlap by construction.
// xh rows are read with whole 128-byte lines per instruction (8 lanes per row: 8 rows x 64 k per
// wave load), which halves the memory-pipeline line requests of a fragment-shaped load (16 rows x
// 64 bytes); the row tile's 2 KB of LDS holds (row r, 16-byte chunk c) in slot
// (r >> 1) * 16 + 8 (r & 1) + (c ^ (r >> 1)), so the consumers' fragment reads (16 rows of one
// chunk) hit 16 distinct 16-byte bank groups, and a load's 64 consecutive slots (the lds bit
// writes lane l at slot base + l) are 8 whole rows.
// Pipeline: three LDS stages and one workgroup barrier B_s per K step.  Between B_{s-1} and B_s
// the producers decode step s + 1 (its trellis words were requested three intervals earlier into
// a register ring), request the xh rows of step s + 2 into the stage step s - 1 used and the
// trellis words of step s + 3, then wait for the xh rows of step s + 1; the consumers run the
// step's four 16-MFMA sub-blocks on stage s % 3, each sub-block's fragments read during the
// previous sub-block, and pass B_s before the last sub-block so that the first fragments of step
// s + 1 are read under its MFMAs.
// Groups (the checkpoint tensors of a fused module: one x, a rotated input per group) are
// flattened into one tile list, so a module pays one GEMM launch and fills the GPU as one.  Each
// output element sees the MFMA sequence of gemm_kernel (k steps in order, two k-substeps each) on
// the same operands: both kernels give bitwise-equal C.
// ============================================================================================
struct PcGroup {
    const uint16_t* xh;         // [M][ldx] rotated input of the group (M * ldx * 2 < 2^31)
    const uint32_t* trellis;
    const uint16_t* svh;
    uint16_t* y;                // first output column of the group (rows ldy apart)
    int n;                      // columns
    int tile0;                  // first tile of the group in the flattened tile list
};

struct PcArgs {
    int64_t ldx, ldy;
    int M, K, groups, total, xcd_remap;
    // Balanced tail: items [0, n_full) are whole tiles; every later tile (the last, partial wave of
    // a plain tile grid) is split along K into `split` pieces (split == 1: no split).  A piece
    // leaves its fp32 partial tile in `part`; the last of a tile's pieces (completion counter)
    // adds them in piece order and applies the epilogue.
    int n_full, split;
    // cut > 0 (split 2): a tile's pieces are K steps [0, cut) and [cut, all) (unequal), and the
    // items hold every tile's first piece before any second piece (the long pieces go first; the
    // short ones fill the CUs that finish early)
    int cut;
    f32x4* part;                // [(tiles - n_full) * split][32][256] partial tiles
    uint32_t part_bytes;        // their size (the raw buffer's range)
    uint32_t* counters;         // [tiles - n_full], zero between calls (the last piece resets)
    PcGroup g[EXL3_MAX_GROUPS];
};

struct PC {
    static constexpr int MT = 256, THREADS = 512;
    static constexpr int RT_BYTES = 16 * 128;          // one row tile of xh for one K step (2 KB)
    static constexpr int A_BYTES = (MT / 16) * RT_BYTES;   // 32 KB
    static constexpr int B_BYTES = 2 * 8 * FRAG;       // 16 KB
    static constexpr int BUF = A_BYTES + B_BYTES;      // one stage
    static constexpr int STAGES = 3;
    static constexpr int C_ROW = 136;                  // LDS row (halves) of the epilogue's C tile
    static constexpr int LDS = STAGES * BUF > MT * C_ROW * 2 ? STAGES * BUF : MT * C_ROW * 2;
};

// byte offset of (row r, 16-byte chunk c) inside a row tile's 2 KB of A
__device__ __forceinline__ int a_slot(int r, int c) { return ((r >> 1) * 16 + 8 * (r & 1) + (c ^ (r >> 1))) * 16; }

// Workgroup barrier after this wave's LDS writes completed (lgkmcnt(0)), with no global-memory
// wait (prefetches stay in flight across it) and no instruction moved across it by the scheduler.
__device__ __forceinline__ void barrier_lds()
{
    __builtin_amdgcn_sched_barrier(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);                // lgkmcnt(0), vmcnt / expcnt not waited
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_sched_barrier(0);
}

template <int BITS, int CB>
__global__ void __launch_bounds__(PC::THREADS) gemm_pc_kernel(PcArgs a)
{
    extern __shared__ __align__(16) char lds[];
    __shared__ int s_last;
    const int t = threadIdx.x;
    const int b = blockIdx.x;
    const bool piece = b >= a.n_full;
    int u, q = 0;
    if (!piece) {
        u = a.xcd_remap ? (b & 7) * (a.n_full / 8) + (b >> 3) : b;    // consecutive tiles share an XCD
    } else {
        const int bb = b - a.n_full;
        if (a.cut) {
            const int tail = a.total - a.n_full;
            q = bb >= tail;
            u = a.n_full + bb - q * tail;
        } else {
            u = a.n_full + bb / a.split;
            q = bb - (bb / a.split) * a.split;
        }
    }
    // constant indices only into the kernel-argument struct (a runtime index copies it to scratch)
    int gi = 0;
    if (a.groups > 1 && u >= a.g[1].tile0) gi = 1;
    if (a.groups > 2 && u >= a.g[2].tile0) gi = 2;
    if (a.groups > 3 && u >= a.g[3].tile0) gi = 3;
    const PcGroup gg = gi == 0 ? a.g[0] : gi == 1 ? a.g[1] : gi == 2 ? a.g[2] : a.g[3];
    const int tiles_n = gg.n / NT_COLS, v = u - gg.tile0;
    const int tm = v / tiles_n, tn = v - tm * tiles_n;
    const int row0 = tm * PC::MT, col0 = tn * NT_COLS;
    const int M = a.M;
    // K steps [sb, sb + steps) of the tile (all of them unless this item is a piece)
    const int all_steps = a.K / KSTEP;
    const int sb = !piece ? 0 : a.cut ? (q ? a.cut : 0) : q * all_steps / a.split;
    const int steps = !piece ? all_steps : a.cut ? (q ? all_steps - a.cut : a.cut) : (q + 1) * all_steps / a.split - sb;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
    auto stage = [&](int s) __attribute__((always_inline)) { return lds + (s % PC::STAGES) * PC::BUF; };
    // partial tile of piece pq of this tile: consumer thread t's 32 accumulator quads, 16 B apart
    // per thread (coalesced); system-coherent (sc1) accesses, read by another CU after the counter
    const int tile_r = u - a.n_full;
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(a.part, 0, (int) a.part_bytes, RAW_BUFFER_FLAGS);
    auto part_off = [&](int pq, int ij) __attribute__((always_inline)) {
        return (uint32_t) ((((tile_r * a.split + pq) * 32 + ij) * 256 + t) * 16);
    };

    if (wave < 4) {
        // ---- consumer ---------------------------------------------------------------------
        f32x4 acc[4][8];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        // A fragments of k-substep ks: row tiles 4 wave + i, lane (g, r) = (row r, chunk 4 ks + g)
        const int a_lane = a_slot(lane & 15, lane >> 4);           // chunk g of k-substep 0
        const int a_lane1 = a_slot(lane & 15, 4 + (lane >> 4));    // chunk g of k-substep 1
        auto rd_a = [&](const char* stg, int ks, f16x8* A) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                A[i] = *reinterpret_cast<const f16x8*>(stg + (4 * wave + i) * PC::RT_BYTES + (ks ? a_lane1 : a_lane));
        };
        // B fragments of sub-block (ks, jh): column tiles 4 jh .. 4 jh + 3 of k-substep ks
        auto rd_b = [&](const char* stg, int ks, int jh, f16x8* B) __attribute__((always_inline)) {
            const char* bf = stg + PC::A_BYTES;
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const int j = 4 * jh + jj;
                B[jj] = *reinterpret_cast<const f16x8*>(bf + ((ks * 8 + j) * 64 + (lane ^ bswz(j))) * 16);
            }
        };
        // row tiles of this wave holding live rows: a wave of a small-M tile skips the MFMAs of
        // its dead row tiles (a loop of its own: a guard inside the full tiles' loop cost 1 %)
        const int live_rt = min(4, max(0, (M - row0 - 64 * wave + 15) / 16));
        f16x8 A0[4], A1[4], B0[4], B1[4];
        barrier_lds();                                     // B_-1: stage 0 staged
        rd_a(stage(0), 0, A0);
        rd_b(stage(0), 0, 0, B0);
        // sched_barrier pins the issue order: the reads of the next sub-block go out before the
        // MFMAs that hide them, and nothing crosses the workgroup barrier
        auto main_loop = [&](auto FULL) __attribute__((always_inline)) {
            auto mm = [&](const f16x8* A, int jh, const f16x8* B) __attribute__((always_inline)) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (decltype(FULL)::value || i < live_rt) {
#pragma unroll
                        for (int jj = 0; jj < 4; ++jj)
                            acc[i][4 * jh + jj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[i], B[jj], acc[i][4 * jh + jj], 0, 0, 0);
                    }
            };
            for (int s = 0; s < steps; ++s) {
                const char* stg = stage(s);
                rd_b(stg, 0, 1, B1);
                rd_a(stg, 1, A1);
                __builtin_amdgcn_sched_barrier(0);
                mm(A0, 0, B0);
                __builtin_amdgcn_sched_barrier(0);
                rd_b(stg, 1, 0, B0);
                __builtin_amdgcn_sched_barrier(0);
                mm(A0, 1, B1);
                __builtin_amdgcn_sched_barrier(0);
                rd_b(stg, 1, 1, B1);
                __builtin_amdgcn_sched_barrier(0);
                mm(A1, 0, B0);
                barrier_lds();                                 // B_s: stage s read, stage s + 1 staged
                if (s + 1 < steps) {
                    rd_a(stage(s + 1), 0, A0);
                    rd_b(stage(s + 1), 0, 0, B0);
                }
                __builtin_amdgcn_sched_barrier(0);
                mm(A1, 1, B1);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        if (live_rt == 4) main_loop(std::true_type{});
        else main_loop(std::false_type{});
        if (piece) {
            // this piece's partial out (its live row tiles); then count the pieces in, and the last
            // one sums them all
            if (live_rt == 4) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][j]), prs,
                                                               part_off(q, i * 8 + j), 0, SC1);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)                // constant indices into acc
                    if (i < live_rt) {
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][j]), prs,
                                                                   part_off(q, i * 8 + j), 0, SC1);
                    }
            }
            __builtin_amdgcn_s_waitcnt(0x0F70);            // vmcnt(0): the partial has landed
            __syncthreads();
            if (t == 0) {
                const uint32_t prev = __hip_atomic_fetch_add(&a.counters[tile_r], 1u, __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_AGENT);
                s_last = prev == (uint32_t) (a.split - 1);
                if (s_last) __hip_atomic_store(&a.counters[tile_r], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();
            if (!s_last) return;                           // uniform: the whole workgroup leaves
            // C = sum of the pieces' partials in piece order (this piece's own from registers), 8
            // accumulator quads at a time: their 8 loads of one piece go out together, one round
            // trip per piece and batch (a load per quad and piece in turn was 32 x (split - 1)
            // dependent round trips at the end of the launch)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (i >= live_rt) continue;                // dead row tiles: never stored
                f32x4 sum[8];
                for (int pq = 0; pq < a.split; ++pq) {
                    f32x4 v[8];
                    if (pq == q) {
#pragma unroll
                        for (int j = 0; j < 8; ++j) v[j] = acc[i][j];
                    } else {
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            v[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, part_off(pq, i * 8 + j),
                                                                                                  0, SC1));
                    }
#pragma unroll
                    for (int j = 0; j < 8; ++j) sum[j] = pq == 0 ? v[j] : sum[j] + v[j];
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[i][j] = sum[j];
            }
        }
        // C = fp16(acc) into LDS: every read and write of the stages finished before the last B_s
        uint16_t* ct = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = wave * 64 + i * 16 + 4 * (lane >> 4) + e;
                    const int c = j * 16 + (lane & 15);
                    ct[r * PC::C_ROW + c] = f16_bits((f16) acc[i][j][e]);
                }
    } else {
        // ---- producer ---------------------------------------------------------------------
        // the producer is the longer path of a step: its VALU issue goes first (measured faster)
        __builtin_amdgcn_s_setprio(3);
        const int pw = wave - 4, pt = t - 256;
        // xh rows go straight to LDS (buffer loads with the lds bit, 16 bytes a lane): wave pw's
        // load j fills the 1 KB block L = 8 pw + j of the stage's A tiles, row tile L >> 1, slots
        // 64 (L & 1) + lane.  Inverting slot = a_slot(r, c) gives lane's row r and chunk c: each
        // group of 8 lanes reads one row's 8 chunks, a whole 128-byte line.  Rows past M take an
        // offset past the buffer's range: the load still issues (the waits below count every
        // load), but it touches no memory (out-of-range buffer reads return 0), and those rows'
        // outputs are never stored (rows do not interact)
        const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(gg.xh), 0, (int) ((uint32_t) M * (uint32_t) a.ldx * 2u), RAW_BUFFER_FLAGS);
        uint32_t aoff[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int L = 8 * pw + j;
            const int qq = 4 * (L & 1) + (lane >> 4), rem = lane & 15;
            const int r = (L >> 1) * 16 + 2 * qq + (rem >> 3);             // row in the tile
            const int c = (rem & 7) ^ qq;                                 // 16-byte chunk
            const int gr = row0 + r;
            aoff[j] = gr < M ? ((uint32_t) gr * (uint32_t) a.ldx + c * 8) * 2u : 0xFFFFFFF0u;
        }
        auto dma_a = [&](int st, char* stg) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void*) (stg + (8 * pw + j) * 1024),
                                                         16, aoff[j], (sb + st) * (KSTEP * 2), 0, 0);
        };
        const int ktl = pt >> 6, ntl = (pt >> 3) & 7, q = pt & 7;
        const int nt_total = gg.n / 16;
        // the trellis as one raw buffer (k * n * K / 8 < 2^31 on the host): a step advances the
        // scalar offset by 4 k-tile rows; the lane's q-block and ring-predecessor word offsets are fixed
        const __amdgpu_buffer_rsrc_t trs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint32_t*>(gg.trellis), 0, (int) ((uint32_t) (a.K / 16) * (uint32_t) nt_total * 32u * BITS),
            RAW_BUFFER_FLAGS);
        const uint32_t tile_w = (uint32_t) (ktl * nt_total + col0 / 16 + ntl) * (8 * BITS);
        const uint32_t off_main = (tile_w + q * BITS) * 4u;
        const uint32_t off_prev = (tile_w + (q == 0 ? 8 * BITS - 1 : q * BITS - 1)) * 4u;
        const uint32_t step_bytes = (uint32_t) nt_total * 4u * 32u * BITS;   // 4 k-tile rows
        auto fetch = [&](int st, uint32_t* W) __attribute__((always_inline)) {
            load_qblock_buf<BITS>(trs, off_main, off_prev, (uint32_t) (sb + st) * step_bytes, W);
        };
        // B fragment tile ks * 8 + ntl, lanes XOR-swizzled by n-tile (conflict-free stores)
        auto decode_store = [&](const uint32_t* W, char* stg) __attribute__((always_inline)) {
            uint32_t P[16];
            decode_qblock<BITS, CB>(W, P);
            char* bf = stg + PC::A_BYTES;
            const int ks = ktl >> 1;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int rh = 0; rh < 2; ++rh) {
                    const int ln = ((2 * (ktl & 1) + rh) * 16 + q + 8 * h) ^ bswz(ntl);
                    const u32x4 val = {P[2 * h + rh], P[4 + 2 * h + rh], P[8 + 2 * h + rh], P[12 + 2 * h + rh]};
                    *reinterpret_cast<u32x4*>(bf + ((ks * 8 + ntl) * 64 + ln) * 16) = val;
                }
        };
        // step j's trellis words live in register ring slot j % 3 (compile-time slot indices: the
        // loop is unrolled by 3), requested three intervals before they are decoded; its xh rows
        // go to stage j % 3 two intervals before it is read
        // The explicit waits below count vector-memory instructions: 8 per dma_a and exactly NW per
        // fetch (no fetch load can merge with another, qblock_loads), issued in the order written
        // (sched_barrier between every request group).  tests/isa_waits.py checks the built code
        // object: on every path into every barrier, only the most recent 8 row loads may be in flight.
        constexpr int NW = qblock_loads<BITS>();
        uint32_t R0[BITS + 1], R1[BITS + 1], R2[BITS + 1];
        dma_a(0, stage(0));
        __builtin_amdgcn_sched_barrier(0);
        fetch(0, R0);
        __builtin_amdgcn_sched_barrier(0);
        dma_a(min(1, steps - 1), stage(1));
        __builtin_amdgcn_sched_barrier(0);
        fetch(min(1, steps - 1), R1);
        fetch(min(2, steps - 1), R2);
        __builtin_amdgcn_sched_barrier(0);
        decode_store(R0, stage(0));
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(8 + 2 * NW));  // xh rows of step 0 in LDS (8 + 3 NW after them)
        barrier_lds();                                     // B_-1
        // interval s (between B_s-1 and B_s): decode step s + 1, request the xh rows of step s + 2
        // into the stage step s - 1 used (read before B_s-1) and the trellis words of step s + 3,
        // then wait for the xh rows of step s + 1 (requested one interval earlier; the loads
        // complete in order and 8 + 2 NW were requested after them).  The last intervals restage
        // the last step into stages no longer read, so every interval has the same requests in
        // flight; the last one waits for all of them (the epilogue reuses the stages' LDS).
        auto interval = [&](int s, const uint32_t* Wd, uint32_t* Wf) __attribute__((always_inline)) {
            decode_store(Wd, stage(s + 1));
            __builtin_amdgcn_sched_barrier(0);
            dma_a(min(s + 2, steps - 1), stage(s + 2));
            __builtin_amdgcn_sched_barrier(0);
            fetch(min(s + 3, steps - 1), Wf);
            __builtin_amdgcn_sched_barrier(0);
            if (s + 1 < steps) __builtin_amdgcn_s_waitcnt(vmcnt_imm(8 + 2 * NW));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            barrier_lds();                                 // B_s
        };
        int s = 0;
        for (; s + 2 < steps; s += 3) {
            interval(s, R1, R0);
            interval(s + 1, R2, R1);
            interval(s + 2, R0, R2);
        }
        if (s < steps) interval(s, R1, R0);
        if (s + 1 < steps) interval(s + 1, R2, R1);
        __builtin_amdgcn_s_setprio(0);
        if (piece) {                                       // the consumers' two completion barriers
            __syncthreads();
            __syncthreads();
            if (!s_last) return;
        }
    }
    __syncthreads();                                       // C tile complete in LDS

    // ---- epilogue: y = fp16(fp16(Had128(C)) * svh) on the matrix cores, 16 rows per wave pass
    // (had128_mfma16: the values of exl3_had_r_128_f32 with post), 16-byte stores ----------------
    const uint16_t* ct = reinterpret_cast<const uint16_t*>(lds);
    const int jr = t & 15, gq = (t >> 4) & 3;
    // svh as device-scope (sc1) raw-buffer loads: a split tile's last piece reaches here after its
    // counter atomic, and every load after a counter atomic carries sc1 (checked on the built code)
    u32x4 sv[4];
    const __amdgpu_buffer_rsrc_t svs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(gg.svh), 0, 0x7FFFFFFF,
                                                                         RAW_BUFFER_FLAGS);
#pragma unroll
    for (int p = 0; p < 4; ++p)
        sv[p] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(svs, (uint32_t) ((col0 + 32 * p + 8 * gq) * 2),
                                                                                0, SC1));
    // the tile's rows as one raw buffer from row row0 (offsets below 256 * ldy * 2 bytes); the
    // stores write through L2 (device scope), so the end-of-kernel writeback finds no dirty output
    const __amdgpu_buffer_rsrc_t ysrc = __builtin_amdgcn_make_buffer_rsrc(gg.y + (int64_t) row0 * a.ldy, 0, 0x7FFFFFFF,
                                                                          RAW_BUFFER_FLAGS);
    const HadMfmaA HA = had_mfma_a();
    for (int rg = t >> 6; rg < PC::MT / 16 && row0 + 16 * rg < M; rg += PC::THREADS / 64) {
        const int r = rg * 16 + jr;
        u32x4 xb[4];
#pragma unroll
        for (int s_ = 0; s_ < 4; ++s_) xb[s_] = *reinterpret_cast<const u32x4*>(ct + r * PC::C_ROW + 32 * s_ + 8 * gq);
        had128_mfma16(HA, xb, r_scale<float>(), true, sv, [&](int p, u32x4 v) __attribute__((always_inline)) {
            if (row0 + r < M)
                __builtin_amdgcn_raw_buffer_store_b128(v, ysrc, (uint32_t) (((int64_t) r * a.ldy + col0 + 32 * p + 8 * gq) * 2), 0, SC1);
        });
    }
}

template <int BITS, int CB>
int launch_gemm_pc(const PcArgs& a, int items, hipStream_t s)
{
    auto kern = gemm_pc_kernel<BITS, CB>;
    static bool attr_set = false;            // dynamic LDS above 64 KB must be enabled per kernel
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*) kern, hipFuncAttributeMaxDynamicSharedMemorySize, PC::LDS) != hipSuccess)
            return EXL3_ELAUNCH;
        attr_set = true;
    }
    hipLaunchKernelGGL(kern, dim3(items), dim3(PC::THREADS), PC::LDS, s, a);
    return hipGetLastError() == hipSuccess ? EXL3_OK : EXL3_ELAUNCH;
}

// Tile plan of one producer/consumer launch: whole tiles for every full wave over the CUs (one
// workgroup per CU), the last, partial wave's tiles split along K into up to CUs / tail pieces of
// at least 8 K steps (or, below one wave, the two unequal pieces below: at least 5), so the launch
// ends in balance.  A function of the shape only.
constexpr int PC_CUS = 256;                    // MI355X compute units
constexpr size_t PC_COUNTER_BYTES = 4096;      // workspace head: completion counters of split tiles
constexpr size_t PC_PIECE_BYTES = (size_t) PC::MT * NT_COLS * 4;   // one fp32 partial tile

struct PcPlan {
    int tiles, n_full, split, cut;
    size_t ws_bytes;                           // 0: no split
};

PcPlan pc_plan(int M, int K, const int* widths, int groups)
{
    PcPlan p{};
    const int tiles_m = (M + PC::MT - 1) / PC::MT;
    for (int i = 0; i < groups; ++i) p.tiles += tiles_m * (widths[i] / NT_COLS);
    const int full = p.tiles / PC_CUS, tail = p.tiles - full * PC_CUS;
    p.split = 1;
    if (full >= 1 && tail > 0) p.split = std::min(PC_CUS / tail, (K / KSTEP) / 8);
    // a launch of at most half a wave of tiles (small M: one row tile of few columns, e.g. the
    // 40 tiles of a 17408 -> 5120 layer) splits every tile, so that the pieces fill the CUs
    if (full == 0 && 2 * tail <= PC_CUS) p.split = std::min(PC_CUS / tail, (K / KSTEP) / 8);
    // more than half a wave and at most two thirds of one (e.g. the 136 tiles of a 5120 -> 17408
    // layer at M <= 256): two unequal pieces per tile, 2/3 and 1/3 of the K steps.  The long pieces
    // and some short ones start at once; the other short ones (2 tiles - CUs of them, at most the
    // CUs - tiles that took a short one) follow on the CUs whose short piece ended, so the launch
    // takes ~2/3 of the steps (5 equal pieces measured 9-50 % slower than unsplit from M = 33 on)
    if (full == 0 && 2 * tail > PC_CUS && 3 * tail <= 2 * PC_CUS && K / KSTEP >= 16) {
        p.split = 2;
        p.cut = (2 * (K / KSTEP) + 2) / 3;
    }
    if (p.split < 2) p.split = 1;
    p.n_full = p.split > 1 ? full * PC_CUS : p.tiles;
    p.ws_bytes = p.split > 1 ? PC_COUNTER_BYTES + (size_t) (p.tiles - p.n_full) * p.split * PC_PIECE_BYTES : 0;
    return p;
}

// One GEMM launch over `groups` groups sharing M and K: group i reads xh[i] and writes widths[i]
// columns at y[i] (rows ldy apart).  Operands too large for 32-bit raw-buffer offsets take the
// 128 x 128 kernel, one launch per group.  Without a workspace of the plan's size the tail is not
// split: less balance, and the tail tiles' fp32 sums run in another order (whole K instead of piece
// partials added in piece order), so their outputs can differ from a split launch's in the last place.
template <int BITS, int CB>
int launch_trellis_gemm(const uint16_t* const* xh, int64_t ldx, const void* const* trellis, uint16_t* const* y,
                        int64_t ldy, const uint16_t* const* svh, const int* widths, int groups, int M, int K,
                        void* ws, size_t ws_bytes, hipStream_t s)
{
    bool fits = (uint64_t) M * (uint64_t) ldx * 2 < (1ull << 31) && (uint64_t) PC::MT * (uint64_t) ldy * 2 < (1ull << 31);
    for (int i = 0; i < groups; ++i) fits = fits && (uint64_t) K * widths[i] * BITS / 8 < (1ull << 31);
    const char* e = getenv("EXL3_GEMM_KERNEL");              // "tile": the 128 x 128 kernel (comparison)
    if (!fits || (e && e[0] == 't')) {
        for (int i = 0; i < groups; ++i) {
            TrellisB<BITS, CB> b{(const uint32_t*) trellis[i], widths[i] / 16};
            const int rc = launch_gemm<TrellisB<BITS, CB>, false, GEMM_MT, true>(xh[i], ldx, b, nullptr, 0, y[i], ldy,
                                                                                 svh[i], M, K, widths[i], s);
            if (rc) return rc;
        }
        return EXL3_OK;
    }
    PcPlan pl = pc_plan(M, K, widths, groups);
    if (pl.split > 1 && (!ws || ws_bytes < pl.ws_bytes || pl.ws_bytes - PC_COUNTER_BYTES >= (1ull << 31))) {
        pl.split = 1;
        pl.cut = 0;
        pl.n_full = pl.tiles;
    }
    PcArgs a{};
    a.ldx = ldx;
    a.ldy = ldy;
    a.M = M;
    a.K = K;
    a.groups = groups;
    const int tiles_m = (M + PC::MT - 1) / PC::MT;
    int tiles = 0;
    for (int i = 0; i < groups; ++i) {
        a.g[i] = {xh[i], (const uint32_t*) trellis[i], svh[i], y[i], widths[i], tiles};
        tiles += tiles_m * (widths[i] / NT_COLS);
    }
    a.total = tiles;
    a.n_full = pl.n_full;
    a.split = pl.split;
    a.cut = pl.cut;
    a.xcd_remap = a.n_full % 8 == 0;
    if (pl.split > 1) {
        a.counters = (uint32_t*) ws;
        a.part = (f32x4*) ((char*) ws + PC_COUNTER_BYTES);
        a.part_bytes = (uint32_t) (pl.ws_bytes - PC_COUNTER_BYTES);
    }
    return launch_gemm_pc<BITS, CB>(a, a.n_full + (tiles - a.n_full) * a.split, s);
}

template <int BITS>
int launch_trellis_gemm_cb(int cb, const uint16_t* const* xh, int64_t ldx, const void* const* tr, uint16_t* const* y,
                           int64_t ldy, const uint16_t* const* svh, const int* widths, int groups, int M, int K,
                           void* ws, size_t wsb, hipStream_t s)
{
    if (cb == 0) return launch_trellis_gemm<BITS, 0>(xh, ldx, tr, y, ldy, svh, widths, groups, M, K, ws, wsb, s);
    if (cb == 1) return launch_trellis_gemm<BITS, 1>(xh, ldx, tr, y, ldy, svh, widths, groups, M, K, ws, wsb, s);
    return launch_trellis_gemm<BITS, 2>(xh, ldx, tr, y, ldy, svh, widths, groups, M, K, ws, wsb, s);
}

// x -> per-group xh (input Hadamards), then one GEMM launch over every group's tiles; x_up (may be
// null): the input rows are fp16(fp16(silu(x)) * x_up), formed by the transform as it loads them
int gemm_trellis_common(const void* x, int64_t ldx, const void* const* trellis, uint16_t* const* y, int64_t ldy,
                        const void* const* suh, uint16_t* xh, const void* const* svh, const int* widths, int groups,
                        int m, int k, int K, int mcg, int mul1, void* ws, size_t wsb, hipStream_t s,
                        const void* x_up = nullptr)
{
    const uint16_t* xhs[EXL3_MAX_GROUPS];
    const uint16_t* svs[EXL3_MAX_GROUPS];
    void* xo[EXL3_MAX_GROUPS];
    for (int i = 0; i < groups; ++i) {
        uint16_t* xi = xh + (int64_t) i * m * k;
        xo[i] = xi;
        xhs[i] = xi;
        svs[i] = (const uint16_t*) svh[i];
    }
    // the groups' input transforms (one x, each group's suh) in one launch
    const int rc = launch_had(x, ldx, xo, k, m, k, suh, groups, nullptr, 1.0f, s, false, x_up);
    if (rc) return rc;
    const int cb = codebook_of(mcg, mul1);
    switch (K) {
        case 1: return launch_trellis_gemm_cb<1>(cb, xhs, k, trellis, y, ldy, svs, widths, groups, m, k, ws, wsb, s);
        case 2: return launch_trellis_gemm_cb<2>(cb, xhs, k, trellis, y, ldy, svs, widths, groups, m, k, ws, wsb, s);
        case 3: return launch_trellis_gemm_cb<3>(cb, xhs, k, trellis, y, ldy, svs, widths, groups, m, k, ws, wsb, s);
        case 4: return launch_trellis_gemm_cb<4>(cb, xhs, k, trellis, y, ldy, svs, widths, groups, m, k, ws, wsb, s);
        case 5: return launch_trellis_gemm_cb<5>(cb, xhs, k, trellis, y, ldy, svs, widths, groups, m, k, ws, wsb, s);
        case 6: return launch_trellis_gemm_cb<6>(cb, xhs, k, trellis, y, ldy, svs, widths, groups, m, k, ws, wsb, s);
        case 7: return launch_trellis_gemm_cb<7>(cb, xhs, k, trellis, y, ldy, svs, widths, groups, m, k, ws, wsb, s);
        default: return launch_trellis_gemm_cb<8>(cb, xhs, k, trellis, y, ldy, svs, widths, groups, m, k, ws, wsb, s);
    }
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
    uint16_t* yp = (uint16_t*) y;
    return gemm_trellis_common(x, ldx, &trellis, &yp, ldy, &suh, (uint16_t*) xh, &svh, &n, 1, m, k, K, mcg, mul1,
                               nullptr, 0, (hipStream_t) stream);
}

size_t exl3_gemm_trellis_workspace_size(int m, int k, const int* widths, int groups)
{
    if (!widths || groups < 1 || groups > EXL3_MAX_GROUPS || m < 1 || k < 128 || k % 128) return 0;
    for (int i = 0; i < groups; ++i)
        if (widths[i] < 128 || widths[i] % 128) return 0;
    return pc_plan(m, k, widths, groups).ws_bytes;
}

size_t exl3_gemm_trellis_workspace_bound(void)
{
    // pieces of one plan: full >= 1 or 2 tail <= CUs: tail * min(CUs / tail, .) <= CUs; the
    // two-piece form: 2 tail with 3 tail <= 2 CUs
    return PC_COUNTER_BYTES + (size_t) std::max(PC_CUS, 2 * (2 * PC_CUS / 3)) * PC_PIECE_BYTES;
}

int exl3_gemm_trellis_grouped(const void* x, int64_t ldx, const void* const* trellis, void* y, int64_t ldy,
                              const void* const* suh, void* xh, const void* const* svh, const int* widths, int groups,
                              int m, int k, int K, int mcg, int mul1, void* workspace, size_t ws_bytes, void* stream)
{
    if (!x || !trellis || !y || !suh || !xh || !svh || !widths || groups < 1 || groups > EXL3_MAX_GROUPS || m < 0 ||
        K < 1 || K > 8 || k % 128 || k < 128 || ldx < k || ldx % 8 || ldy % 8 || (((uintptr_t) xh) & 15) ||
        (((uintptr_t) y) & 15))
        return EXL3_EINVAL;
    int64_t total = 0;
    uint16_t* ys[EXL3_MAX_GROUPS];
    for (int i = 0; i < groups; ++i) {
        if (!trellis[i] || !suh[i] || !svh[i] || widths[i] < 128 || widths[i] % 128 || (((uintptr_t) svh[i]) & 15) ||
            (((uintptr_t) trellis[i]) & 15))
            return EXL3_EINVAL;
        ys[i] = (uint16_t*) y + total;
        total += widths[i];
    }
    if (ldy < total) return EXL3_EINVAL;
    if (m == 0) return EXL3_OK;
    return gemm_trellis_common(x, ldx, trellis, ys, ldy, suh, (uint16_t*) xh, svh, widths, groups, m, k, K, mcg, mul1,
                               workspace, ws_bytes, (hipStream_t) stream);
}

int exl3_gemm_trellis_silu_in(const void* gate, const void* up, int64_t ldx, const void* trellis, void* y, int64_t ldy,
                              const void* suh, void* xh, const void* svh, int m, int k, int n, int K, int mcg, int mul1,
                              void* workspace, size_t ws_bytes, void* stream)
{
    if (!gate || !up || !trellis || !y || !suh || !xh || !svh || m < 0 || K < 1 || K > 8 || k % 128 || n % 128 ||
        k < 128 || n < 128 || ldx < k || ldy < n || ldx % 8 || ldy % 8 || (((uintptr_t) gate) & 15) ||
        (((uintptr_t) up) & 15) || (((uintptr_t) xh) & 15) || (((uintptr_t) y) & 15) || (((uintptr_t) svh) & 15) ||
        (((uintptr_t) trellis) & 15))
        return EXL3_EINVAL;
    if (m == 0) return EXL3_OK;
    uint16_t* yp = (uint16_t*) y;
    return gemm_trellis_common(gate, ldx, &trellis, &yp, ldy, &suh, (uint16_t*) xh, &svh, &n, 1, m, k, K, mcg, mul1,
                               workspace, ws_bytes, (hipStream_t) stream, up);
}

int exl3_gemm(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh, void* A_had,
              const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
              void* stream)
{
    if (m <= 0) return m == 0 ? 1 : EXL3_EINVAL;
    if (m <= EXL3_GEMV_FUSED_MAX_ROWS) {
        const int rc = exl3_gemv_mr(x, ldx, trellis, y, ldy, suh, A_had, svh, m, k, n, K, mcg, mul1, workspace,
                                    ws_bytes, stream);
        return rc == EXL3_OK ? 1 : (rc > 0 ? EXL3_EINVAL : rc);
    }
    const int rc = exl3_gemm_trellis(x, ldx, trellis, y, ldy, suh, A_had, svh, m, k, n, K, mcg, mul1, stream);
    return rc == EXL3_OK ? 2 : rc;
}

}  // extern "C"
