// exl3_gemv.hip -- EXL3 decode / reconstruct / Hadamard / fused small-M GEMV kernels for gfx950.
//
// The GEMV (1 <= M <= 32) is one launch per call:
//   prologue  each workgroup rotates its own k-slice of the input into LDS:
//             A_had = fp16(Had128(fp16(x * suh)))                 (exact float64 butterflies)
//   main loop each wave decodes 2 n-tiles x 4 k-tiles (8 tiles, 2048 weights) per step, one
//             q-block per lane, and feeds the packed fp16 pairs straight into
//             v_mfma_f32_16x16x32_f16 (rows of the MFMA = up to 16 input rows; fp32 accumulate)
//   epilogue split-K partials go to the workspace; the last workgroup of a 128-column block
//             (per-block completion counter, reset by that workgroup) sums them in split order,
//             rounds C to fp16 and applies y = fp16(fp16(Had128(C)) * svh).
// Rows never interact, and the split count depends only on (k, n), so every row of an M-row
// call is bitwise identical to the M == 1 call of that row, grouped or not.
#include "exl3_device.h"
#include "../../include/exl3_mi355x.h"

#include <stdio.h>
#include <stdlib.h>
#include <algorithm>
#include <utility>

using namespace exl3;

// f(integral_constant<int, I>) for I in the sequence: ring slots are indexed by constants in the
// source, so the ring always lives in registers (a loop index here could leave it in scratch memory)
template <class F, int... I>
__device__ __forceinline__ void static_for(std::integer_sequence<int, I...>, F&& f)
{
    (f(std::integral_constant<int, I>{}), ...);
}

// ============================================================================================
// Codebook decode of raw states (reference binding `decode`, tests/test_gpu_parity.py:101-109)
// ============================================================================================
template <int CB>
__device__ __forceinline__ float decode_one(uint32_t s)
{
    const uint32_t x = state_hash<CB, 0>(s, Codebook<CB>::hi << 16, CB == 0 ? Codebook<0>::add : 0u, Codebook<CB>::lo);
    if constexpr (CB == 2) {
        const uint32_t h = __builtin_amdgcn_udot4(x, 0x01010101u, 0x6400u, false);
        const f16 v = __builtin_fmaf16(bits_f16(h), bits_f16(0x1EEEu), bits_f16(0xC931u));
        return (float) v;
    } else {
        const uint32_t y = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
        return (float) (bits_f16(y & 0xFFFFu) + bits_f16(y >> 16));
    }
}

template <int CB>
__global__ void __launch_bounds__(256) decode_kernel(const uint16_t* __restrict__ states, float* __restrict__ out,
                                                     int64_t count)
{
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i < count) out[i] = decode_one<CB>(states[i]);
}

// ============================================================================================
// reconstruct: trellis -> dense fp16 W[k, n_out] for n-tiles [nt0, nt0 + n_out/16)
// One workgroup = one k-tile row x up to 32 n-tiles; one q-block per thread, transposed
// through LDS so global stores are whole rows.
// ============================================================================================
template <int BITS, int CB>
__global__ void __launch_bounds__(256) reconstruct_kernel(const uint32_t* __restrict__ trellis, uint16_t* __restrict__ W,
                                                          int nt_total, int nt0, int nt_out, int64_t ldw)
{
    __shared__ uint16_t tile[16][512 + 8];
    const int kt = blockIdx.y;
    const int strip = blockIdx.x * 32;
    const int t = threadIdx.x;
    const int local_nt = t >> 3, q = t & 7;
    const int nts = min(32, nt_out - strip);
    if (local_nt < nts) {
        gc_u32* tp = as_global(trellis) + ((int64_t) kt * nt_total + nt0 + strip + local_nt) * (8 * BITS);
        uint32_t Wd[BITS + 1];
        load_qblock<BITS>(tp, q, Wd);
        uint32_t P[16];
        decode_qblock<BITS, CB>(Wd, P);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = i >> 2, h = (i >> 1) & 1, rh = i & 1;     // i = 4r + 2h + rh
            const int row = 8 * rh + 2 * r, col = local_nt * 16 + q + 8 * h;
            tile[row][col] = (uint16_t) (P[i] & 0xFFFFu);
            tile[row + 1][col] = (uint16_t) (P[i] >> 16);
        }
    }
    __syncthreads();
    // write-out: 16 rows x (16*nts) columns, 8 halves (16 B) per store
    const int chunks_per_row = nts * 2;            // 16 cols per tile = 2 chunks of 8
    for (int c = t; c < 16 * chunks_per_row; c += 256) {
        const int row = c / chunks_per_row, ch = c % chunks_per_row;
        const u32x4 v = *reinterpret_cast<const u32x4*>(&tile[row][ch * 8]);
        *reinterpret_cast<u32x4*>(W + (int64_t) (kt * 16 + row) * ldw + (int64_t) strip * 16 + ch * 8) = v;
    }
}

// ============================================================================================
// had_r_128: out = fp16(Had128(in [* pre]) * r * scale) [* post]; one 16-lane group per 128-block,
// 4 blocks per wave (reference binding `had_r_128`, vllm_plugin/exl3rocm/ops.py:88,97)
// ============================================================================================
__global__ void __launch_bounds__(256) had_kernel(const uint16_t* __restrict__ in, int64_t ld_in, uint16_t* __restrict__ out,
                                                  int64_t ld_out, int rows, int cols, const uint16_t* __restrict__ pre,
                                                  const uint16_t* __restrict__ post, double scale)
{
    const int blocks_per_row = cols / 128;
    const int64_t job = ((int64_t) blockIdx.x * 256 + threadIdx.x) >> 4;     // one 128-block per 16 lanes
    const bool live = job < (int64_t) rows * blocks_per_row;
    const int r = threadIdx.x & 15;
    const int64_t row = live ? job / blocks_per_row : 0;
    const int col = live ? (int) (job % blocks_per_row) * 128 + 8 * r : 0;
    u32x4 v = {0u, 0u, 0u, 0u}, pv = v, qv = v;
    if (live) {
        v = *reinterpret_cast<const u32x4*>(in + row * ld_in + col);
        if (pre) pv = *reinterpret_cast<const u32x4*>(pre + col);
        if (post) qv = *reinterpret_cast<const u32x4*>(post + col);
    }
    // every lane takes part in the DPP exchanges; only live lanes store
    const u32x4 res = had128_x8(v, pv, pre != nullptr, qv, post != nullptr, R_SCALE * scale);
    if (live) *reinterpret_cast<u32x4*>(out + row * ld_out + col) = res;
}

// ============================================================================================
// Fused GEMV with stream-K balancing
//
// Work unit: (128-column block cb, 128-row k slice ku) == two 64-row k steps == one Hadamard
// block of the input; units are ordered cb-major, U in total, UPB = k / 128 per block.  The grid
// has G workgroups (all resident); workgroup w owns units [w*U/G, (w+1)*U/G).  Wave i of a
// workgroup covers n-tiles 2i, 2i+1 of the block; its lanes = (k-tile g of the step, n-tile,
// q-block).  A workgroup keeps fp32 accumulators across consecutive units of one block and writes
// one partial per block it touches; the block's completion counter counts the contributing
// workgroups and the last one sums the partials in workgroup order (fixed for the shape, hence
// deterministic), rounds C to fp16 and applies the output Hadamard and svh.
// ============================================================================================
struct GemvGroup {
    const uint32_t* trellis;   // tile words
    const uint16_t* suh;
    const uint16_t* svh;
    uint16_t* y;               // output columns of this group (row stride ldy)
};

struct GemvArgs {
    const uint16_t* x;         // [M][ldx] fp16
    int64_t ldx;
    GemvGroup g[EXL3_MAX_GROUPS];
    const int64_t* tab_trellis; // optional device pointer tables (grouped M=1 `mgemm` form)
    const int64_t* tab_suh;
    const int64_t* tab_svh;
    int64_t group_col_stride;  // with tables: group i writes y + i * group_col_stride
    int M, k, n;
    int G, U, UPB, max_seg;    // grid, units, units per block, partial slots per workgroup
    int chunk_units;           // units whose rotated input fits the LDS at once
    int64_t ldy;
    float* part;               // [groups][G][max_seg][M][128] fp32 partials
    uint32_t* counters;        // [groups][NB], zero between calls
};

constexpr int RED_BATCH = 16;                   // partial loads in flight per thread in the reduction
constexpr int A_ROW = 136;                      // LDS row of one rotated 128-block (padded, halves)
constexpr int LDS_BUDGET = 64 * 1024;           // per workgroup: 2 workgroups per CU
constexpr int RING = 8;                         // 64-row k steps in flight per wave (even)
constexpr int WAVES_PER_SIMD = 2;

// s_waitcnt vmcnt(0) (gfx9 encoding: expcnt / lgkmcnt left at their maxima), fenced against
// compiler reordering: every vector-memory store of this wave has completed.
__device__ __forceinline__ void wait_stores_complete()
{
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ int wg_lo(int w, int U, int G) { return (int) ((int64_t) w * U / G); }
// workgroup owning unit u: the largest w with floor(w*U/G) <= u
__device__ __forceinline__ int wg_of_unit(int u, int U, int G) { return (int) (((int64_t) (u + 1) * G - 1) / U); }


// Two workgroups (8 waves) per CU are resident at once: up to 256 registers per lane, enough for
// a ring deep enough that one wave alone keeps its SIMD busy.
template <int BITS, int CB, int MT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WAVES_PER_SIMD, WAVES_PER_SIMD))) gemv_kernel(GemvArgs a)
{
    extern __shared__ __align__(16) uint16_t smem[];
    __shared__ int s_last[256];
    const int w = blockIdx.x, grp = blockIdx.y;
    const int G = a.G, U = a.U, UPB = a.UPB, M = a.M;
    const int NB = a.n / 128, NT = a.n / 16;
    const uint32_t* trel;
    const uint16_t* suh;
    const uint16_t* svh;
    uint16_t* y;
    if (a.tab_trellis) {
        trel = reinterpret_cast<const uint32_t*>(a.tab_trellis[grp]);
        suh = reinterpret_cast<const uint16_t*>(a.tab_suh[grp]);
        svh = reinterpret_cast<const uint16_t*>(a.tab_svh[grp]);
        y = a.g[0].y + grp * a.group_col_stride;
    } else {
        // constant indices only: a runtime index into the kernel-argument struct would copy it to
        // scratch memory, and every later read of it would be a vector-memory load
        const GemvGroup gg = grp == 0 ? a.g[0] : grp == 1 ? a.g[1] : grp == 2 ? a.g[2] : a.g[3];
        trel = gg.trellis;
        suh = gg.suh;
        svh = gg.svh;
        y = gg.y;
    }
    // the trellis as one raw buffer (layers of 4 GiB and more are declined on the host)
    const uint64_t trel_bytes = (uint64_t) a.k * a.n * BITS / 8;
    const __amdgpu_buffer_rsrc_t trsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(trel), 0, (int) (uint32_t) trel_bytes, RAW_BUFFER_FLAGS);
    gc_u16* const gsuh = as_global(suh);
    gc_u16* const gsvh = as_global(svh);
    gc_u16* const gx = as_global(a.x);
    g_u16* const gy = as_global(y);
    // LDS: the rotated input of a chunk of units, M rows per unit followed by one zero row (the A
    // operand of MFMA rows >= M), then the fp16 C of one block for the output transform
    const int UROWS = M + 1;
    uint16_t* lds_a = smem;                                   // [chunk_units][M + 1][A_ROW]
    uint16_t* lds_c = smem + a.chunk_units * UROWS * A_ROW;   // [M][A_ROW]
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int g = lane >> 4, j = lane & 15, q = j & 7;
    const int ulo = wg_lo(w, U, G), uhi = wg_lo(w + 1, U, G);
    if (ulo >= uhi) return;                                   // uniform per workgroup
    const int seg0_cb = ulo / UPB;
    float* part_grp = a.part + (int64_t) grp * G * a.max_seg * M * 128;

    // Trellis addressing.  Step d (0, 1) of unit (cb, ku) covers k-tiles 8ku + 4d .. +3 and n-tiles
    // 8cb .. 8cb + 7; this lane reads q-block q of tile (k-tile + g, n-tile 8cb + 2 wave + (j >> 3)).
    // A uniform byte offset walks the units; the lane adds fixed byte offsets.
    const int tile_lane = (g * NT + wave * 2 + (j >> 3)) * (8 * BITS);            // words
    const uint32_t off_main = (uint32_t) (tile_lane + q * BITS) * 4u;
    const uint32_t off_prev = (uint32_t) (tile_lane + (q == 0 ? 8 * BITS - 1 : q * BITS - 1)) * 4u;
    const uint32_t STEP_D = (uint32_t) (4 * NT * 8 * BITS * 4);   // bytes from step 0 to step 1 of a unit
    const uint32_t STEP_KU = 2 * STEP_D;                          // to the next unit of the same block
    const uint32_t STEP_CB = 8 * 8 * BITS * 4;                    // to the next block, same ku
    const uint32_t STEP_WRAP = STEP_CB - (uint32_t) (UPB - 1) * STEP_KU;   // to ku 0 of the next block (mod 2^32)

    // rotated-input job i of a chunk starting at unit u0: (unit u0 + i / M, row i % M), 16 lanes each
    auto job_src = [&](int u0, int i, int& m, int& col) __attribute__((always_inline)) {
        const int u = u0 + i / M;
        m = i - (i / M) * M;
        col = (u - (u / UPB) * UPB) * 128 + 8 * (threadIdx.x & 15);
    };

    // The prologue and the completion phase sit on every workgroup's critical path while other
    // workgroups on the same SIMDs run VALU-heavy decode loops: give them issue priority.
    __builtin_amdgcn_s_setprio(2);

    // ---- first input chunk: its x / suh loads go out before the trellis ring ----------------
    const int nfirst = min(a.chunk_units, uhi - ulo) * M;
    u32x4 px = {0u, 0u, 0u, 0u}, ps = px;
    {
        const int i = threadIdx.x >> 4;
        if (i < nfirst) {
            int m, col;
            job_src(ulo, i, m, col);
            px = *reinterpret_cast<gc_u32x4*>(gx + (int64_t) m * a.ldx + col);
            ps = *reinterpret_cast<gc_u32x4*>(gsuh + col);
        }
    }
    // ---- the trellis ring: RING steps in flight per wave ----------------------------------------
    // Slot i always holds a step with d == i & 1.  The load cursor (ul, ku_l, lp) is the unit of the
    // next refill; it stops at the last unit, whose steps are reloaded (in bounds, never used).
    uint32_t Wr[RING][BITS + 1];
    int ul = ulo, ku_l = ulo - seg0_cb * UPB;
    uint32_t lp = (uint32_t) seg0_cb * STEP_CB + (uint32_t) ku_l * STEP_KU;
    auto advance_load = [&]() __attribute__((always_inline)) {
        if (ul + 1 < uhi) {
            ++ul;
            if (++ku_l == UPB) {
                ku_l = 0;
                lp += STEP_WRAP;
            } else {
                lp += STEP_KU;
            }
        }
    };
    static_for(std::make_integer_sequence<int, RING>{}, [&](auto I) __attribute__((always_inline)) {
        constexpr int i = decltype(I)::value;
        load_qblock_buf<BITS>(trsrc, off_main, off_prev, lp + (i & 1) * STEP_D, Wr[i]);
        if (i & 1) advance_load();
    });
    // rotated input of units [c0, c1) -> LDS; the first 16-lane job of each lane uses (x0, s0)
    auto rotate_chunk = [&](int c0, int c1, u32x4 x0, u32x4 s0, bool have_first) __attribute__((always_inline)) {
        const int njobs = (c1 - c0) * M;
        const int i = threadIdx.x >> 4;
        if (i - (threadIdx.x & 63) / 16 < njobs) {            // waves with a job (whole 16-lane groups)
            if (!have_first && i < njobs) {
                int m, col;
                job_src(c0, i, m, col);
                x0 = *reinterpret_cast<gc_u32x4*>(gx + (int64_t) m * a.ldx + col);
                s0 = *reinterpret_cast<gc_u32x4*>(gsuh + col);
            }
            const u32x4 r = had128_x8(x0, s0, true, u32x4{0u, 0u, 0u, 0u}, false, R_SCALE);
            if (i < njobs) {
                int m, col;
                job_src(c0, i, m, col);
                *reinterpret_cast<u32x4*>(lds_a + ((i / M) * UROWS + m) * A_ROW + 8 * (threadIdx.x & 15)) = r;
            }
            for (int i2 = i + 16; i2 - (threadIdx.x & 63) / 16 < njobs; i2 += 16) {
                u32x4 xv = {0u, 0u, 0u, 0u}, sv = xv;
                int m = 0, col = 0;
                if (i2 < njobs) {
                    job_src(c0, i2, m, col);
                    xv = *reinterpret_cast<gc_u32x4*>(gx + (int64_t) m * a.ldx + col);
                    sv = *reinterpret_cast<gc_u32x4*>(gsuh + col);
                }
                const u32x4 r2 = had128_x8(xv, sv, true, u32x4{0u, 0u, 0u, 0u}, false, R_SCALE);
                if (i2 < njobs)
                    *reinterpret_cast<u32x4*>(lds_a + ((i2 / M) * UROWS + m) * A_ROW + 8 * (threadIdx.x & 15)) = r2;
            }
        }
    };
    int c0 = ulo, c1 = min(ulo + a.chunk_units, uhi);
    rotate_chunk(c0, c1, px, ps, true);
    // zero rows: never overwritten by later chunks
    for (int t = threadIdx.x; t < a.chunk_units * (A_ROW / 8); t += 256)
        *reinterpret_cast<u32x4*>(lds_a + ((t / (A_ROW / 8)) * UROWS + M) * A_ROW + 8 * (t % (A_ROW / 8))) =
            u32x4{0u, 0u, 0u, 0u};
    __syncthreads();

    // A operand row of this lane (per MFMA row tile) within a unit: rows >= M read the zero row
    int a_lane[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) a_lane[mt] = (mt * 16 + j < M ? mt * 16 + j : M) * A_ROW + 16 * g;

    f32x4 acc[2][MT];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[h][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int colb = wave * 32 + (j >> 3) * 16 + (j & 7);    // + 8h: column of this lane in the block
    auto write_partial = [&](int cb) __attribute__((always_inline)) {
        float* slab = part_grp + ((int64_t) w * a.max_seg + (cb - seg0_cb)) * M * 128;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int m = mt * 16 + 4 * g + v;
                    if (m < M)
                        __hip_atomic_store(&slab[m * 128 + colb + 8 * h], acc[h][mt][v], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                }
    };

    // one k step: decode the slot's q-block, refill the slot from the load cursor (when the ring
    // still has steps to fetch), two MFMAs per tile column half
    auto step = [&](uint32_t (&Wq)[BITS + 1], const uint16_t* unit_a, int d, bool refill) __attribute__((always_inline)) {
        uint32_t P[16];
        decode_qblock<BITS, CB>(Wq, P);
        if (refill) load_qblock_buf<BITS>(trsrc, off_main, off_prev, lp + d * STEP_D, Wq);
        f16x8 A0[MT], A1[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const uint16_t* ap = unit_a + a_lane[mt] + 64 * d;
            A0[mt] = *reinterpret_cast<const f16x8*>(ap);
            A1[mt] = *reinterpret_cast<const f16x8*>(ap + 8);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const u32x4 B0 = {P[2 * h], P[4 + 2 * h], P[8 + 2 * h], P[12 + 2 * h]};
            const u32x4 B1 = {P[2 * h + 1], P[5 + 2 * h], P[9 + 2 * h], P[13 + 2 * h]};
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                acc[h][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0[mt], __builtin_bit_cast(f16x8, B0), acc[h][mt], 0, 0, 0);
                acc[h][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1[mt], __builtin_bit_cast(f16x8, B1), acc[h][mt], 0, 0, 0);
            }
        }
    };

    int cb_cur = seg0_cb;
    int left = UPB - (ulo - seg0_cb * UPB);                   // units of block cb_cur still to come
    // sub-step i of the ring turn starting at unit u0 (slot i, d = i & 1)
    auto sub_step = [&](auto I, int u0, bool refill) __attribute__((always_inline)) {
        constexpr int i = decltype(I)::value;
        if (!(i & 1)) {
            if (left == 0) {                                  // a new 128-column block starts
                write_partial(cb_cur);
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[h][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
                ++cb_cur;
                left = UPB;
            }
            --left;
        }
        step(Wr[i], lds_a + (u0 + i / 2 - c0) * UROWS * A_ROW, i & 1, refill);
        if ((i & 1) && refill) advance_load();
    };
    auto next_chunk = [&](int u0) __attribute__((always_inline)) {      // chunks hold whole ring turns
        if (u0 == c1) {
            c0 = c1;
            c1 = min(c0 + a.chunk_units, uhi);
            __syncthreads();
            rotate_chunk(c0, c1, px, ps, false);
            __syncthreads();
        }
    };

    __builtin_amdgcn_s_setprio(0);
    // Full ring turns run without per-step conditions (a conditional step would make the compiler
    // wait for every load in flight); the last, partial turn only drains the ring.
    const int S = 2 * (uhi - ulo);                            // 64-row k steps of this workgroup
    const int S_full = S - S % RING;
    int s0 = 0;
    for (; s0 < S_full; s0 += RING) {
        const int u0 = ulo + s0 / 2;
        next_chunk(u0);
        static_for(std::make_integer_sequence<int, RING>{}, [&](auto I) __attribute__((always_inline)) { sub_step(I, u0, true); });
    }
    if (s0 < S) {
        const int u0 = ulo + s0 / 2;
        next_chunk(u0);
        static_for(std::make_integer_sequence<int, RING>{}, [&](auto I) __attribute__((always_inline)) {
            if (s0 + decltype(I)::value < S) sub_step(I, u0, false);
        });
    }
    __builtin_amdgcn_s_setprio(2);
    write_partial(cb_cur);

    // ---- completion: count this workgroup into every block it touched, reduce those it completed
    // The partials are device-scope (write-through) stores: once complete (vmcnt(0)) they are
    // visible to device-scope loads from any XCD, so no cache-wide release is needed.
    wait_stores_complete();
    __syncthreads();
    const int nblk = cb_cur - seg0_cb + 1;
    for (int b0 = 0; b0 < nblk; b0 += 256) {
        const int nb = min(256, nblk - b0);
        if ((int) threadIdx.x < nb) {                         // one counter per thread, all in flight
            const int cb = seg0_cb + b0 + threadIdx.x;
            const int wf = wg_of_unit(cb * UPB, U, G), wl = wg_of_unit(cb * UPB + UPB - 1, U, G);
            const uint32_t prev = __hip_atomic_fetch_add(&a.counters[grp * NB + cb], 1u, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            s_last[threadIdx.x] = prev == (uint32_t) (wl - wf) ? 1 : 0;
        }
        __syncthreads();
        for (int bi = 0; bi < nb; ++bi) {
            if (!__builtin_amdgcn_readfirstlane(s_last[bi])) continue;
            const int cb = seg0_cb + b0 + bi;
            // contributor wf holds block cb in its segment cb - first_cb(wf); every later
            // contributor starts inside cb, so its segment is 0.  Loads go out in batches of
            // RED_BATCH; the sum runs in contributor order.
            const int wf = wg_of_unit(cb * UPB, U, G), wl = wg_of_unit(cb * UPB + UPB - 1, U, G);
            const int seg_f = cb - wg_lo(wf, U, G) / UPB;
            const int nc = wl - wf + 1;
            for (int e = threadIdx.x; e < M * 128; e += 256) {
                float sum = 0.f;
                for (int cc0 = 0; cc0 < nc; cc0 += RED_BATCH) {
                    float v[RED_BATCH];
#pragma unroll
                    for (int ii = 0; ii < RED_BATCH; ++ii) {
                        const int c = cc0 + ii;
                        const int64_t slot = c == 0 ? (int64_t) wf * a.max_seg + seg_f : (int64_t) (wf + c) * a.max_seg;
                        v[ii] = c < nc ? __hip_atomic_load(part_grp + slot * M * 128 + e, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT)
                                       : 0.f;
                    }
#pragma unroll
                    for (int ii = 0; ii < RED_BATCH; ++ii)
                        if (cc0 + ii < nc) sum += v[ii];
                }
                lds_c[(e >> 7) * A_ROW + (e & 127)] = f16_bits((f16) sum);
            }
            if (threadIdx.x == 0)                              // ready for the next call (stream order)
                __hip_atomic_store(&a.counters[grp * NB + cb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            // output Hadamard + svh: 16 lanes per row
            const int rr = threadIdx.x & 15;
            const u32x4 sv = *reinterpret_cast<gc_u32x4*>(gsvh + cb * 128 + 8 * rr);
            for (int m0 = 0; m0 < M; m0 += 16) {
                const int m = m0 + (threadIdx.x >> 4);
                const bool live = m < M;
                u32x4 c = {0u, 0u, 0u, 0u};
                if (live) c = *reinterpret_cast<const u32x4*>(lds_c + m * A_ROW + 8 * rr);
                const u32x4 r = had128_x8(c, u32x4{0u, 0u, 0u, 0u}, false, sv, true, R_SCALE);
                if (live) *reinterpret_cast<g_u32x4*>(gy + (int64_t) m * a.ldy + cb * 128 + 8 * rr) = r;
            }
            __syncthreads();                                   // lds_c free for the next block
        }
        __syncthreads();                                       // s_last free for the next batch
    }
}

// ============================================================================================
// Host side
// ============================================================================================
namespace {

int env_int(const char* name, int dflt)
{
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

int codebook_of(int mcg, int mul1) { return mul1 ? 2 : (mcg ? 1 : 0); }

// Stream-K grid: workgroups per group, from (k, n, groups) only -- never from m -- so every row
// of an m-row call is bitwise equal to the m == 1 call, and a module's grouped launches agree
// across row counts.  All workgroups of a launch are resident at once (4 per CU at the kernel's
// register budget), each with at least two 64-row k steps.
constexpr int RESIDENT_WGS = 256 * WAVES_PER_SIMD;   // 256 CUs x workgroups per CU

int choose_grid(int k, int n, int groups)
{
    const int64_t UPB = k / 128, U = (int64_t) (n / 128) * UPB;
    const int forced = env_int("EXL3_GEMV_GRID", 0);
    // all workgroups resident; at most ~max_contrib workgroups sharing one block
    const int max_contrib = env_int("EXL3_GEMV_MAX_CONTRIB", 32);
    const int64_t min_units = std::max<int64_t>(1, (UPB + max_contrib - 1) / max_contrib);
    int64_t G = forced > 0 ? forced : std::min<int64_t>(RESIDENT_WGS / std::max(groups, 1), U / min_units);
    return (int) std::max<int64_t>(1, std::min<int64_t>(G, U));
}

int max_segments(int k, int n, int G)
{
    const int64_t UPB = k / 128, U = (int64_t) (n / 128) * UPB;
    const int64_t per = (U + G - 1) / G;
    return (int) ((per + UPB - 1) / UPB + 1);
}

// units whose rotated input a workgroup stages at once (all of them when they fit)
int chunk_units(int m, int k, int n, int G)
{
    const int64_t U = (int64_t) (n / 128) * (k / 128);
    const int64_t per = (U + G - 1) / G;
    // a chunk that is not the last one holds whole ring turns (RING / 2 units)
    const int64_t fit = std::max<int64_t>(RING / 2, ((LDS_BUDGET / (2 * A_ROW) - m) / (m + 1)) / (RING / 2) * (RING / 2));
    return (int) std::max<int64_t>(1, std::min(per, fit));
}

size_t lds_bytes(int M, int cu) { return ((size_t) cu * (M + 1) + M) * A_ROW * 2; }

template <int BITS, int CB, int MT>
int launch_gemv_t(const GemvArgs& a, int groups, hipStream_t stream)
{
    hipLaunchKernelGGL((gemv_kernel<BITS, CB, MT>), dim3(a.G, groups), dim3(256), lds_bytes(a.M, a.chunk_units),
                       stream, a);
    return hipGetLastError() == hipSuccess ? EXL3_OK : EXL3_ELAUNCH;
}

template <int BITS, int CB>
int launch_gemv_m(const GemvArgs& a, int groups, hipStream_t s)
{
    return a.M <= 16 ? launch_gemv_t<BITS, CB, 1>(a, groups, s) : launch_gemv_t<BITS, CB, 2>(a, groups, s);
}

template <int BITS>
int launch_gemv_cb(const GemvArgs& a, int cb, int groups, hipStream_t s)
{
    switch (cb) {
        case 0: return launch_gemv_m<BITS, 0>(a, groups, s);
        case 1: return launch_gemv_m<BITS, 1>(a, groups, s);
        default: return launch_gemv_m<BITS, 2>(a, groups, s);
    }
}

int launch_gemv(const GemvArgs& a, int bits, int cb, int groups, hipStream_t s)
{
    switch (bits) {
        case 1: return launch_gemv_cb<1>(a, cb, groups, s);
        case 2: return launch_gemv_cb<2>(a, cb, groups, s);
        case 3: return launch_gemv_cb<3>(a, cb, groups, s);
        case 4: return launch_gemv_cb<4>(a, cb, groups, s);
        case 5: return launch_gemv_cb<5>(a, cb, groups, s);
        case 6: return launch_gemv_cb<6>(a, cb, groups, s);
        case 7: return launch_gemv_cb<7>(a, cb, groups, s);
        default: return launch_gemv_cb<8>(a, cb, groups, s);
    }
}

// workspace layout: [counters: fixed EXL3_GEMV_COUNTER_BYTES region][partials: groups*G*max_seg*M*128 f32].
// The counter region has a fixed size so calls of different shapes sharing one workspace never
// see another shape's partial sums where their counters live.
constexpr size_t COUNTER_BYTES = EXL3_GEMV_COUNTER_BYTES;

size_t gemv_ws_bytes(int m, int k, int n, int groups)
{
    const int G = choose_grid(k, n, groups);
    return COUNTER_BYTES + (size_t) groups * G * max_segments(k, n, G) * m * 128 * 4;
}

bool shape_ok(int m, int k, int n, int K)
{
    return m >= 1 && m <= EXL3_GEMV_MAX_ROWS && k >= 128 && n >= 128 && k % 128 == 0 && n % 128 == 0 && K >= 1 && K <= 8;
}

int gemv_common(const void* x, int64_t ldx, const GemvGroup* gs, int groups, const int64_t* const* tabs,
                int64_t col_stride, int64_t ldy, int m, int k, int n, int K, int mcg, int mul1, void* ws,
                size_t ws_bytes, void* stream)
{
    if (!x || groups < 1 || groups > EXL3_MAX_GROUPS || ldx < k || ldy < n) return EXL3_EINVAL;
    // the kernel moves fp16 in 16-byte groups of 8: x rows, y rows, suh and svh 16-byte aligned
    if ((ldx & 7) || (ldy & 7) || (((uintptr_t) x) & 15)) return EXL3_EINVAL;
    // with pointer tables only gs[0].y is given; the table entries are the caller's contract
    for (int i = 0; i < (tabs ? 1 : groups); ++i) {
        if (!gs[i].y || (((uintptr_t) gs[i].y) & 15)) return EXL3_EINVAL;
        if (!tabs && ((((uintptr_t) gs[i].suh) & 15) || (((uintptr_t) gs[i].svh) & 15) ||
                      (((uintptr_t) gs[i].trellis) & 15)))
            return EXL3_EINVAL;
    }
    if (groups > 1 && !tabs && m > 1 && ldy < (int64_t) groups * n) return EXL3_EINVAL;
    if (!shape_ok(m, k, n, K)) return EXL3_DECLINED;
    if ((uint64_t) k * n * K / 8 > 0xFFFFFFFFull) return EXL3_DECLINED;   // one raw buffer per trellis
    if ((size_t) groups * (n / 128) * 4 > COUNTER_BYTES) return EXL3_DECLINED;
    if (ws_bytes < gemv_ws_bytes(m, k, n, groups) || !ws) return EXL3_EWORKSPACE;
    GemvArgs a{};
    a.x = (const uint16_t*) x;
    a.ldx = ldx;
    for (int i = 0; i < groups && !tabs; ++i) a.g[i] = gs[i];
    if (tabs) {
        a.tab_trellis = tabs[0];
        a.tab_suh = tabs[1];
        a.tab_svh = tabs[2];
        a.g[0].y = gs[0].y;
        a.group_col_stride = col_stride;
    }
    a.M = m;
    a.k = k;
    a.n = n;
    a.G = choose_grid(k, n, groups);
    a.UPB = k / 128;
    a.U = (n / 128) * a.UPB;
    a.max_seg = max_segments(k, n, a.G);
    a.chunk_units = chunk_units(m, k, n, a.G);
    a.ldy = ldy;
    a.counters = (uint32_t*) ws;
    a.part = (float*) ((char*) ws + COUNTER_BYTES);
    return launch_gemv(a, K, codebook_of(mcg, mul1), groups, (hipStream_t) stream);
}

}  // namespace

// ============================================================================================
// C ABI
// ============================================================================================
extern "C" {

int exl3_abi_version(void) { return EXL3_ABI_VERSION; }

int exl3_gemv_grid(int k, int n, int groups)
{
    return (k % 128 || k < 128 || n % 128 || n < 128 || groups < 1 || groups > EXL3_MAX_GROUPS) ? 0
                                                                                               : choose_grid(k, n, groups);
}

size_t exl3_gemv_workspace_size(int m, int k, int n, int K, int groups)
{
    (void) K;
    if (!shape_ok(m, k, n, 1) || groups < 1 || groups > EXL3_MAX_GROUPS) return 0;
    return gemv_ws_bytes(m, k, n, groups);
}

int exl3_gemv_mr_supported(int m, int k, int n, int K, int mcg, int mul1)
{
    (void) mcg;
    (void) mul1;
    return shape_ok(m, k, n, K) ? 1 : 0;
}

int exl3_gemv(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh, void* A_had,
              const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
              void* stream)
{
    (void) A_had;
    if (!trellis || !y || !suh || !svh) return EXL3_EINVAL;
    if (m != 1) return EXL3_DECLINED;
    GemvGroup g{(const uint32_t*) trellis, (const uint16_t*) suh, (const uint16_t*) svh, (uint16_t*) y};
    return gemv_common(x, ldx, &g, 1, nullptr, 0, ldy, m, k, n, K, mcg, mul1, workspace, ws_bytes, stream);
}

int exl3_gemv_mr(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh, void* A_had,
                 const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
                 void* stream)
{
    (void) A_had;
    if (!trellis || !y || !suh || !svh) return EXL3_EINVAL;
    GemvGroup g{(const uint32_t*) trellis, (const uint16_t*) suh, (const uint16_t*) svh, (uint16_t*) y};
    return gemv_common(x, ldx, &g, 1, nullptr, 0, ldy, m, k, n, K, mcg, mul1, workspace, ws_bytes, stream);
}

int exl3_gemv_mr_grouped(const void* x, int64_t ldx, const void* const* trellis, void* y, int64_t ldy,
                         const void* const* suh, void* A_had, const void* const* svh, int groups, int m, int k, int n,
                         int K, int mcg, int mul1, int bszm_for_warps, void* workspace, size_t ws_bytes, void* stream)
{
    (void) A_had;
    (void) bszm_for_warps;
    if (!trellis || !suh || !svh || !y || groups < 1 || groups > EXL3_MAX_GROUPS) return EXL3_EINVAL;
    GemvGroup gs[EXL3_MAX_GROUPS];
    for (int i = 0; i < groups; ++i) {
        if (!trellis[i] || !suh[i] || !svh[i]) return EXL3_EINVAL;
        gs[i] = {(const uint32_t*) trellis[i], (const uint16_t*) suh[i], (const uint16_t*) svh[i],
                 (uint16_t*) y + (int64_t) i * n};
    }
    return gemv_common(x, ldx, gs, groups, nullptr, 0, ldy, m, k, n, K, mcg, mul1, workspace, ws_bytes, stream);
}

int exl3_mgemm(const void* x, const int64_t* ptrs_trellis, void* y, const int64_t* ptrs_suh, void* xh,
               const int64_t* ptrs_svh, int groups, int k, int n, int K, int mcg, int mul1, void* workspace,
               size_t ws_bytes, void* stream)
{
    (void) xh;
    if (!ptrs_trellis || !ptrs_suh || !ptrs_svh || !y || groups < 1 || groups > EXL3_MAX_GROUPS) return EXL3_EINVAL;
    GemvGroup g{nullptr, nullptr, nullptr, (uint16_t*) y};
    const int64_t* tabs[3] = {ptrs_trellis, ptrs_suh, ptrs_svh};
    return gemv_common(x, k, &g, groups, tabs, n, (int64_t) groups * n, 1, k, n, K, mcg, mul1, workspace, ws_bytes,
                       stream);
}

int exl3_reconstruct_slice(void* W, int64_t ldw, const void* trellis, int k, int n, int K, int mcg, int mul1, int n0,
                           int n_out, void* stream)
{
    if (!W || !trellis || k % 16 || n % 16 || n0 % 16 || n_out % 16 || n0 < 0 || n_out < 16 || n0 + n_out > n ||
        ldw < n_out || ldw % 8 || (((uintptr_t) W) & 15) || (((uintptr_t) trellis) & 15) || K < 1 || K > 8 || k < 16)
        return EXL3_EINVAL;
    const int cb = codebook_of(mcg, mul1);
    const int nt_out = n_out / 16;
    dim3 grid((nt_out + 31) / 32, k / 16);
    hipStream_t s = (hipStream_t) stream;
#define EXL3_REC(B, C) hipLaunchKernelGGL((reconstruct_kernel<B, C>), grid, dim3(256), 0, s, (const uint32_t*) trellis, \
                                          (uint16_t*) W, n / 16, n0 / 16, nt_out, ldw)
#define EXL3_REC_CB(B) do { if (cb == 0) EXL3_REC(B, 0); else if (cb == 1) EXL3_REC(B, 1); else EXL3_REC(B, 2); } while (0)
    switch (K) {
        case 1: EXL3_REC_CB(1); break;
        case 2: EXL3_REC_CB(2); break;
        case 3: EXL3_REC_CB(3); break;
        case 4: EXL3_REC_CB(4); break;
        case 5: EXL3_REC_CB(5); break;
        case 6: EXL3_REC_CB(6); break;
        case 7: EXL3_REC_CB(7); break;
        default: EXL3_REC_CB(8); break;
    }
#undef EXL3_REC_CB
#undef EXL3_REC
    return hipGetLastError() == hipSuccess ? EXL3_OK : EXL3_ELAUNCH;
}

int exl3_reconstruct(void* W, const void* trellis, int k, int n, int K, int mcg, int mul1, void* stream)
{
    return exl3_reconstruct_slice(W, n, trellis, k, n, K, mcg, mul1, 0, n, stream);
}

int exl3_decode(const void* states, void* out_f32, int64_t count, int mcg, int mul1, void* stream)
{
    if (!states || !out_f32 || count < 0) return EXL3_EINVAL;
    if (count == 0) return EXL3_OK;
    const int cb = codebook_of(mcg, mul1);
    dim3 grid((unsigned) ((count + 255) / 256));
    hipStream_t s = (hipStream_t) stream;
    if (cb == 0) hipLaunchKernelGGL(decode_kernel<0>, grid, dim3(256), 0, s, (const uint16_t*) states, (float*) out_f32, count);
    else if (cb == 1) hipLaunchKernelGGL(decode_kernel<1>, grid, dim3(256), 0, s, (const uint16_t*) states, (float*) out_f32, count);
    else hipLaunchKernelGGL(decode_kernel<2>, grid, dim3(256), 0, s, (const uint16_t*) states, (float*) out_f32, count);
    return hipGetLastError() == hipSuccess ? EXL3_OK : EXL3_ELAUNCH;
}

int exl3_had_r_128(const void* in, int64_t ld_in, void* out, int64_t ld_out, int rows, int cols, const void* pre,
                   const void* post, float scale, void* stream)
{
    if (!in || !out || rows < 0 || cols % 128 || cols < 128 || ld_in < cols || ld_out < cols || ld_in % 8 || ld_out % 8 ||
        (((uintptr_t) in) & 15) || (((uintptr_t) out) & 15) || (((uintptr_t) pre) & 15) || (((uintptr_t) post) & 15))
        return EXL3_EINVAL;
    if (rows == 0) return EXL3_OK;
    const int64_t jobs = (int64_t) rows * (cols / 128);           // 16 lanes each
    hipLaunchKernelGGL(had_kernel, dim3((unsigned) ((jobs + 15) / 16)), dim3(256), 0, (hipStream_t) stream,
                       (const uint16_t*) in, ld_in, (uint16_t*) out, ld_out, rows, cols, (const uint16_t*) pre,
                       (const uint16_t*) post, (double) scale);
    return hipGetLastError() == hipSuccess ? EXL3_OK : EXL3_ELAUNCH;
}

}  // extern "C"
