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
    int n;                     // width (columns)
    int G;                     // workgroups of this group
    int wg0;                   // its first workgroup in the flattened grid
    int max_seg;               // partial slots per workgroup
    int64_t part_off;          // first partial (floats) of this group
    int cnt_off;               // first completion counter of this group
    int h;                     // its workgroups dispatched first on their CU (weight wa; the rest wb)
};

struct GemvArgs {
    const uint16_t* x;         // [M][ldx] fp16
    int64_t ldx;
    GemvGroup g[EXL3_MAX_GROUPS];
    const int64_t* tab_trellis; // optional device pointer tables (grouped M=1 `mgemm` form): they
    const int64_t* tab_suh;     // replace g[i].trellis / suh / svh
    const int64_t* tab_svh;
    int groups, M, k, UPB;
    int wa, wb;                // unit-split weights of first-dispatched / second workgroups on a CU
    int chunk_units;           // units whose rotated input fits the LDS at once
    int64_t ldy;
    float* part;               // per group: [G][max_seg][M][128] fp32 partials
    uint32_t* counters;        // per group: [n / 128], zero between calls
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

// a wave-uniform 64-bit value as a scalar (readfirstlane of both halves)
__device__ __forceinline__ int64_t uniform_i64(int64_t v)
{
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) v);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) ((uint64_t) v >> 32));
    return (int64_t) (((uint64_t) hi << 32) | lo);
}

// Unit split of a group's U units over its G workgroups: workgroup w owns [lo(w), lo(w + 1)),
// lo(w) = floor(U * S(w) / S(G)) with S(w) = wa * min(w, h) + wb * max(w - h, 0).  The first h
// workgroups of the group are dispatched first on their CU; the SIMD arbiter favours their (older)
// waves, so they get the larger weight wa and both waves of a CU finish their units together.  A
// function of the shape only (never of m): rows stay bitwise equal to the m == 1 call.
struct Split {
    int U, G, h, wa, wb;
    __host__ __device__ int64_t S(int w) const
    {
        return (int64_t) wa * (w < h ? w : h) + (int64_t) wb * (w > h ? w - h : 0);
    }
    __host__ __device__ int lo(int w) const { return (int) ((int64_t) U * S(w) / S(G)); }
    // the workgroup owning unit u: the largest w in [0, G) with lo(w) <= u, i.e. S(w) <= T
    __host__ __device__ int owner(int u) const
    {
        const int64_t SG = S(G);
        const int64_t T = ((int64_t) (u + 1) * SG + U - 1) / U - 1;
        const int w = T < (int64_t) wa * h ? (int) (T / wa) : h + (int) ((T - (int64_t) wa * h) / wb);
        return w < G - 1 ? w : G - 1;
    }
    // most units any workgroup owns
    __host__ __device__ int max_units() const
    {
        const int wmax = wa > wb ? wa : wb;
        return (int) (((int64_t) U * wmax + S(G) - 1) / S(G)) + 1;
    }
};


// Two workgroups (8 waves) per CU are resident at once: up to 256 registers per lane, enough for
// a ring deep enough that one wave alone keeps its SIMD busy.
template <int BITS, int CB, int MT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WAVES_PER_SIMD, WAVES_PER_SIMD))) gemv_kernel(GemvArgs a)
{
    extern __shared__ __align__(16) uint16_t smem[];
    __shared__ int s_last[256];
    __shared__ int s_list[256];
    __shared__ int s_nred;
    // the group of this workgroup: a flattened grid, each group its own range of workgroups
    int grp = 0;
    if (a.groups > 1 && (int) blockIdx.x >= a.g[1].wg0) grp = 1;
    if (a.groups > 2 && (int) blockIdx.x >= a.g[2].wg0) grp = 2;
    if (a.groups > 3 && (int) blockIdx.x >= a.g[3].wg0) grp = 3;
    // constant indices only: a runtime index into the kernel-argument struct would copy it to
    // scratch memory, and every later read of it would be a vector-memory load
    const GemvGroup gg = grp == 0 ? a.g[0] : grp == 1 ? a.g[1] : grp == 2 ? a.g[2] : a.g[3];
    const int w = blockIdx.x - gg.wg0;
    const int G = gg.G, UPB = a.UPB, M = a.M;
    const int NB = gg.n / 128, NT = gg.n / 16, U = NB * UPB;
    const Split sp{U, G, gg.h, a.wa, a.wb};
    const uint32_t* trel = gg.trellis;
    const uint16_t* suh = gg.suh;
    const uint16_t* svh = gg.svh;
    uint16_t* y = gg.y;
    if (a.tab_trellis) {
        // table entries are uniform (grp is): keep them in scalar registers, or the trellis buffer
        // resource would look divergent and every buffer load would be wrapped in a waterfall loop
        trel = reinterpret_cast<const uint32_t*>(uniform_i64(a.tab_trellis[grp]));
        suh = reinterpret_cast<const uint16_t*>(uniform_i64(a.tab_suh[grp]));
        svh = reinterpret_cast<const uint16_t*>(uniform_i64(a.tab_svh[grp]));
    }
    uint32_t* const counters = a.counters + gg.cnt_off;
    // the trellis as one raw buffer (layers of 4 GiB and more are declined on the host)
    const uint64_t trel_bytes = (uint64_t) a.k * gg.n * BITS / 8;
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
    const int ulo = sp.lo(w), uhi = sp.lo(w + 1);
    if (ulo >= uhi) return;                                   // uniform per workgroup
    const int seg0_cb = ulo / UPB;
    float* part_grp = a.part + gg.part_off;

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
        float* slab = part_grp + ((int64_t) w * gg.max_seg + (cb - seg0_cb)) * M * 128;
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
    const int RB = M == 1 ? 2 : 1;                            // completed blocks reduced side by side
    for (int b0 = 0; b0 < nblk; b0 += 256) {
        const int nb = min(256, nblk - b0);
        if ((int) threadIdx.x < nb) {                         // one counter per thread, all in flight
            const int cb = seg0_cb + b0 + threadIdx.x;
            const int wf = sp.owner(cb * UPB), wl = sp.owner(cb * UPB + UPB - 1);
            const uint32_t prev = __hip_atomic_fetch_add(&counters[cb], 1u, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            s_last[threadIdx.x] = prev == (uint32_t) (wl - wf) ? 1 : 0;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int c = 0;
            for (int bi = 0; bi < nb; ++bi)
                if (s_last[bi]) s_list[c++] = seg0_cb + b0 + bi;
            s_nred = c;
        }
        __syncthreads();
        const int nred = __builtin_amdgcn_readfirstlane(s_nred);
        for (int r0 = 0; r0 < nred; r0 += RB) {
            const int rb = min(RB, nred - r0);
            // svh of the first output-transform pass, requested before the partial loads so that its
            // round trip overlaps theirs
            const int l16 = threadIdx.x & 15;
            u32x4 sv_first = {0u, 0u, 0u, 0u};
            {
                const int rr = threadIdx.x >> 4;
                if (rr < rb * M) sv_first = *reinterpret_cast<gc_u32x4*>(gsvh + s_list[r0 + rr / M] * 128 + 8 * l16);
            }
            // contributor wf holds block cb in its segment cb - first_cb(wf); every later
            // contributor starts inside cb, so its segment is 0.  Loads go out in batches of
            // RED_BATCH; the sum runs in contributor order.
            for (int e = threadIdx.x; e < rb * M * 128; e += 256) {
                const int r = e / (M * 128), el = e - r * (M * 128);
                const int cb = s_list[r0 + r];
                const int wf = sp.owner(cb * UPB), wl = sp.owner(cb * UPB + UPB - 1);
                const int seg_f = cb - sp.lo(wf) / UPB;
                const int nc = wl - wf + 1;
                float sum = 0.f;
                for (int cc0 = 0; cc0 < nc; cc0 += RED_BATCH) {
                    float v[RED_BATCH];
#pragma unroll
                    for (int ii = 0; ii < RED_BATCH; ++ii) {
                        const int c = cc0 + ii;
                        const int64_t slot = c == 0 ? (int64_t) wf * gg.max_seg + seg_f : (int64_t) (wf + c) * gg.max_seg;
                        v[ii] = c < nc ? __hip_atomic_load(part_grp + slot * M * 128 + el, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT)
                                       : 0.f;
                    }
#pragma unroll
                    for (int ii = 0; ii < RED_BATCH; ++ii)
                        if (cc0 + ii < nc) sum += v[ii];
                }
                lds_c[(r * M + (el >> 7)) * A_ROW + (el & 127)] = f16_bits((f16) sum);
            }
            if ((int) threadIdx.x < rb)                        // ready for the next call (stream order)
                __hip_atomic_store(&counters[s_list[r0 + threadIdx.x]], 0u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            // output Hadamard + svh: 16 lanes per (block, row)
            for (int rr0 = 0; rr0 < rb * M; rr0 += 16) {
                const int rr = rr0 + (threadIdx.x >> 4);
                const bool live = rr < rb * M;
                const int r = live ? rr / M : 0, m = live ? rr - r * M : 0;
                const int cb = s_list[r0 + r];
                u32x4 c = {0u, 0u, 0u, 0u}, sv = c;
                if (live) {
                    c = *reinterpret_cast<const u32x4*>(lds_c + rr * A_ROW + 8 * l16);
                    sv = rr0 == 0 ? sv_first : *reinterpret_cast<gc_u32x4*>(gsvh + cb * 128 + 8 * l16);
                }
                const u32x4 res = had128_x8(c, u32x4{0u, 0u, 0u, 0u}, false, sv, true, R_SCALE);
                if (live) *reinterpret_cast<g_u32x4*>(gy + (int64_t) m * a.ldy + cb * 128 + 8 * l16) = res;
            }
            __syncthreads();                                   // lds_c free for the next blocks
        }
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

// Stream-K grid plan of one launch: workgroups per group from (k, widths) only -- never from m --
// so every row of an m-row call is bitwise equal to the m == 1 call, and a module's grouped
// launches agree across row counts.  The groups share the resident workgroup slots in proportion
// to their units; each keeps its own workgroup range, partial slots and completion counters.
constexpr int NUM_CUS = 256;                          // MI355X
constexpr int RESIDENT_WGS = NUM_CUS * WAVES_PER_SIMD;   // workgroups per CU x CUs

struct GridPlan {
    int groups;
    int G[EXL3_MAX_GROUPS], wg0[EXL3_MAX_GROUPS], max_seg[EXL3_MAX_GROUPS], cnt_off[EXL3_MAX_GROUPS];
    int64_t slot_off[EXL3_MAX_GROUPS];   // first partial slot (one slot = m * 128 floats)
    int total_wgs, counters;
    int64_t slots;
    int max_per;                         // most units any workgroup owns
    int h[EXL3_MAX_GROUPS], wa, wb;      // unit-split weights (Split)
};

// Unit-split weights of first-dispatched / second workgroups on a CU: the measured issue share of
// an older wave on a SIMD shared by two (EXL3_GEMV_WEIGHTS="a,b" overrides, for measurement)
void split_weights(int& wa, int& wb)
{
    wa = 3;
    wb = 2;
    const char* e = getenv("EXL3_GEMV_WEIGHTS");
    int a = 0, b = 0;
    if (e && sscanf(e, "%d,%d", &a, &b) == 2 && a >= 1 && b >= 1 && a <= 64 && b <= 64) {
        wa = a;
        wb = b;
    }
}

GridPlan plan_grid(int k, const int* widths, int groups)
{
    GridPlan p{};
    p.groups = groups;
    const int UPB = k / 128;
    int64_t Utot = 0;
    for (int i = 0; i < groups; ++i) Utot += (int64_t) (widths[i] / 128) * UPB;
    const int forced = env_int("EXL3_GEMV_GRID", 0);
    // at most ~max_contrib workgroups sharing one block
    const int max_contrib = env_int("EXL3_GEMV_MAX_CONTRIB", 32);
    const int64_t min_units = std::max<int64_t>(1, (UPB + max_contrib - 1) / max_contrib);
    int64_t Gt = forced > 0 ? (int64_t) forced * groups : std::min<int64_t>(RESIDENT_WGS, Utot / min_units);
    Gt = std::max<int64_t>(Gt, groups);
    split_weights(p.wa, p.wb);
    int Gs[EXL3_MAX_GROUPS], gsum = 0;
    for (int i = 0; i < groups; ++i) {
        const int64_t Ui = (int64_t) (widths[i] / 128) * UPB;
        Gs[i] = (int) std::max<int64_t>(1, std::min<int64_t>(Ui, (Gt * Ui + Utot / 2) / Utot));
        gsum += Gs[i];
    }
    // workgroups [0, NUM_CUS) of the grid are the first on their CU; with at most one per CU all
    // are, and the split is uniform
    const int first = gsum > NUM_CUS ? NUM_CUS : gsum;
    int wg = 0, cnt = 0;
    int64_t slots = 0;
    for (int i = 0; i < groups; ++i) {
        const int Ui = (widths[i] / 128) * UPB;
        p.G[i] = Gs[i];
        p.wg0[i] = wg;
        // weighted only where every workgroup still gets a unit (U * min(wa, wb) >= max(wa, wb) * G;
        // the completion count assumes each workgroup between a block's first and last owner
        // contributes to it)
        const bool weighted = (int64_t) Ui * std::min(p.wa, p.wb) >= (int64_t) std::max(p.wa, p.wb) * Gs[i];
        p.h[i] = weighted ? std::min(std::max(first - wg, 0), Gs[i]) : Gs[i];
        const Split sp{Ui, Gs[i], p.h[i], p.wa, p.wb};
        const int per = sp.max_units();
        p.max_seg[i] = (per + UPB - 1) / UPB + 1;
        p.cnt_off[i] = cnt;
        p.slot_off[i] = slots;
        p.max_per = std::max(p.max_per, per);
        wg += p.G[i];
        cnt += widths[i] / 128;
        slots += (int64_t) p.G[i] * p.max_seg[i];
    }
    p.total_wgs = wg;
    p.counters = cnt;
    p.slots = slots;
    return p;
}

// units whose rotated input a workgroup stages at once (all of them when they fit); a chunk that
// is not the last one holds whole ring turns (RING / 2 units)
int chunk_units(int m, int max_per)
{
    const int64_t fit = std::max<int64_t>(RING / 2, ((LDS_BUDGET / (2 * A_ROW) - 2 * m) / (m + 1)) / (RING / 2) * (RING / 2));
    return (int) std::max<int64_t>(1, std::min<int64_t>(max_per, fit));
}

// LDS: chunk_units x (m + 1) input rows, then the C rows of the blocks reduced side by side
size_t lds_bytes(int M, int cu) { return ((size_t) cu * (M + 1) + (M == 1 ? 2 : M)) * A_ROW * 2; }

template <int BITS, int CB, int MT>
int launch_gemv_t(const GemvArgs& a, int wgs, hipStream_t stream)
{
    hipLaunchKernelGGL((gemv_kernel<BITS, CB, MT>), dim3(wgs), dim3(256), lds_bytes(a.M, a.chunk_units), stream, a);
    return hipGetLastError() == hipSuccess ? EXL3_OK : EXL3_ELAUNCH;
}

template <int BITS, int CB>
int launch_gemv_m(const GemvArgs& a, int wgs, hipStream_t s)
{
    return a.M <= 16 ? launch_gemv_t<BITS, CB, 1>(a, wgs, s) : launch_gemv_t<BITS, CB, 2>(a, wgs, s);
}

template <int BITS>
int launch_gemv_cb(const GemvArgs& a, int cb, int wgs, hipStream_t s)
{
    switch (cb) {
        case 0: return launch_gemv_m<BITS, 0>(a, wgs, s);
        case 1: return launch_gemv_m<BITS, 1>(a, wgs, s);
        default: return launch_gemv_m<BITS, 2>(a, wgs, s);
    }
}

int launch_gemv(const GemvArgs& a, int bits, int cb, int wgs, hipStream_t s)
{
    switch (bits) {
        case 1: return launch_gemv_cb<1>(a, cb, wgs, s);
        case 2: return launch_gemv_cb<2>(a, cb, wgs, s);
        case 3: return launch_gemv_cb<3>(a, cb, wgs, s);
        case 4: return launch_gemv_cb<4>(a, cb, wgs, s);
        case 5: return launch_gemv_cb<5>(a, cb, wgs, s);
        case 6: return launch_gemv_cb<6>(a, cb, wgs, s);
        case 7: return launch_gemv_cb<7>(a, cb, wgs, s);
        default: return launch_gemv_cb<8>(a, cb, wgs, s);
    }
}

// workspace layout: [counters: fixed EXL3_GEMV_COUNTER_BYTES region][partials: slots * m * 128 f32].
// The counter region has a fixed size so calls of different shapes sharing one workspace never
// see another shape's partial sums where their counters live.
constexpr size_t COUNTER_BYTES = EXL3_GEMV_COUNTER_BYTES;

size_t gemv_ws_bytes(int m, int k, const int* widths, int groups)
{
    const GridPlan p = plan_grid(k, widths, groups);
    return COUNTER_BYTES + (size_t) p.slots * m * 128 * 4;
}

bool shape_ok(int m, int k, int n, int K)
{
    return m >= 1 && m <= EXL3_GEMV_MAX_ROWS && k >= 128 && n >= 128 && k % 128 == 0 && n % 128 == 0 && K >= 1 && K <= 8;
}

// gs[i].y: group i's first output column (rows ldy apart); with pointer tables only gs[i].y is
// read from gs, the table entries are the caller's contract
int gemv_common(const void* x, int64_t ldx, const GemvGroup* gs, const int* widths, int groups,
                const int64_t* const* tabs, int64_t ldy, int m, int k, int K, int mcg, int mul1, void* ws,
                size_t ws_bytes, void* stream)
{
    if (!x || groups < 1 || groups > EXL3_MAX_GROUPS || ldx < k) return EXL3_EINVAL;
    // the kernel moves fp16 in 16-byte groups of 8: x rows, y rows, suh and svh 16-byte aligned
    if ((ldx & 7) || (ldy & 7) || (((uintptr_t) x) & 15)) return EXL3_EINVAL;
    int64_t total = 0;
    for (int i = 0; i < groups; ++i) {
        if (!gs[i].y || (((uintptr_t) gs[i].y) & 15)) return EXL3_EINVAL;
        if (!tabs && (!gs[i].trellis || !gs[i].suh || !gs[i].svh || (((uintptr_t) gs[i].suh) & 15) ||
                      (((uintptr_t) gs[i].svh) & 15) || (((uintptr_t) gs[i].trellis) & 15)))
            return EXL3_EINVAL;
        if (widths[i] < 1) return EXL3_EINVAL;
        total += widths[i];
    }
    if (ldy < widths[0] || (m > 1 && ldy < total)) return EXL3_EINVAL;
    for (int i = 0; i < groups; ++i) {
        if (!shape_ok(m, k, widths[i], K)) return EXL3_DECLINED;
        if ((uint64_t) k * widths[i] * K / 8 > 0xFFFFFFFFull) return EXL3_DECLINED;   // one raw buffer per trellis
    }
    const GridPlan p = plan_grid(k, widths, groups);
    if ((size_t) p.counters * 4 > COUNTER_BYTES) return EXL3_DECLINED;
    if (!ws || ws_bytes < COUNTER_BYTES + (size_t) p.slots * m * 128 * 4) return EXL3_EWORKSPACE;
    GemvArgs a{};
    a.x = (const uint16_t*) x;
    a.ldx = ldx;
    for (int i = 0; i < groups; ++i) {
        a.g[i] = gs[i];
        a.g[i].n = widths[i];
        a.g[i].G = p.G[i];
        a.g[i].wg0 = p.wg0[i];
        a.g[i].max_seg = p.max_seg[i];
        a.g[i].part_off = p.slot_off[i] * m * 128;
        a.g[i].cnt_off = p.cnt_off[i];
        a.g[i].h = p.h[i];
    }
    a.wa = p.wa;
    a.wb = p.wb;
    if (tabs) {
        a.tab_trellis = tabs[0];
        a.tab_suh = tabs[1];
        a.tab_svh = tabs[2];
    }
    a.groups = groups;
    a.M = m;
    a.k = k;
    a.UPB = k / 128;
    a.chunk_units = chunk_units(m, p.max_per);
    a.ldy = ldy;
    a.counters = (uint32_t*) ws;
    a.part = (float*) ((char*) ws + COUNTER_BYTES);
    return launch_gemv(a, K, codebook_of(mcg, mul1), p.total_wgs, (hipStream_t) stream);
}

}  // namespace

// ============================================================================================
// C ABI
// ============================================================================================
extern "C" {

int exl3_abi_version(void) { return EXL3_ABI_VERSION; }

int exl3_gemv_grid(int k, int n, int groups)
{
    if (k % 128 || k < 128 || n % 128 || n < 128 || groups < 1 || groups > EXL3_MAX_GROUPS) return 0;
    const int widths[EXL3_MAX_GROUPS] = {n, n, n, n};
    return plan_grid(k, widths, groups).G[0];
}

size_t exl3_gemv_workspace_size(int m, int k, int n, int K, int groups)
{
    (void) K;
    if (!shape_ok(m, k, n, 1) || groups < 1 || groups > EXL3_MAX_GROUPS) return 0;
    const int widths[EXL3_MAX_GROUPS] = {n, n, n, n};
    return gemv_ws_bytes(m, k, widths, groups);
}

size_t exl3_gemv_workspace_size_widths(int m, int k, const int* widths, int groups)
{
    if (!widths || groups < 1 || groups > EXL3_MAX_GROUPS) return 0;
    for (int i = 0; i < groups; ++i)
        if (!shape_ok(m, k, widths[i], 1)) return 0;
    return gemv_ws_bytes(m, k, widths, groups);
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
    return gemv_common(x, ldx, &g, &n, 1, nullptr, ldy, m, k, K, mcg, mul1, workspace, ws_bytes, stream);
}

int exl3_gemv_mr(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh, void* A_had,
                 const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
                 void* stream)
{
    (void) A_had;
    if (!trellis || !y || !suh || !svh) return EXL3_EINVAL;
    GemvGroup g{(const uint32_t*) trellis, (const uint16_t*) suh, (const uint16_t*) svh, (uint16_t*) y};
    return gemv_common(x, ldx, &g, &n, 1, nullptr, ldy, m, k, K, mcg, mul1, workspace, ws_bytes, stream);
}

int exl3_gemv_mr_grouped(const void* x, int64_t ldx, const void* const* trellis, void* y, int64_t ldy,
                         const void* const* suh, void* A_had, const void* const* svh, int groups, int m, int k, int n,
                         int K, int mcg, int mul1, int bszm_for_warps, void* workspace, size_t ws_bytes, void* stream)
{
    (void) A_had;
    (void) bszm_for_warps;
    if (!trellis || !suh || !svh || !y || groups < 1 || groups > EXL3_MAX_GROUPS) return EXL3_EINVAL;
    GemvGroup gs[EXL3_MAX_GROUPS];
    int widths[EXL3_MAX_GROUPS];
    for (int i = 0; i < groups; ++i) {
        gs[i] = {(const uint32_t*) trellis[i], (const uint16_t*) suh[i], (const uint16_t*) svh[i],
                 (uint16_t*) y + (int64_t) i * n};
        widths[i] = n;
    }
    return gemv_common(x, ldx, gs, widths, groups, nullptr, ldy, m, k, K, mcg, mul1, workspace, ws_bytes, stream);
}

int exl3_gemv_mr_grouped_widths(const void* x, int64_t ldx, const void* const* trellis, void* y, int64_t ldy,
                                const void* const* suh, const void* const* svh, const int* widths, int groups, int m,
                                int k, int K, int mcg, int mul1, void* workspace, size_t ws_bytes, void* stream)
{
    if (!trellis || !suh || !svh || !y || !widths || groups < 1 || groups > EXL3_MAX_GROUPS) return EXL3_EINVAL;
    GemvGroup gs[EXL3_MAX_GROUPS];
    int64_t n0 = 0;
    for (int i = 0; i < groups; ++i) {
        gs[i] = {(const uint32_t*) trellis[i], (const uint16_t*) suh[i], (const uint16_t*) svh[i], (uint16_t*) y + n0};
        n0 += widths[i];
    }
    if (ldy < n0) return EXL3_EINVAL;
    return gemv_common(x, ldx, gs, widths, groups, nullptr, ldy, m, k, K, mcg, mul1, workspace, ws_bytes, stream);
}

int exl3_mgemm(const void* x, const int64_t* ptrs_trellis, void* y, const int64_t* ptrs_suh, void* xh,
               const int64_t* ptrs_svh, int groups, int k, int n, int K, int mcg, int mul1, void* workspace,
               size_t ws_bytes, void* stream)
{
    (void) xh;
    if (!ptrs_trellis || !ptrs_suh || !ptrs_svh || !y || groups < 1 || groups > EXL3_MAX_GROUPS) return EXL3_EINVAL;
    GemvGroup gs[EXL3_MAX_GROUPS];
    int widths[EXL3_MAX_GROUPS];
    for (int i = 0; i < groups; ++i) {
        gs[i] = {nullptr, nullptr, nullptr, (uint16_t*) y + (int64_t) i * n};
        widths[i] = n;
    }
    const int64_t* tabs[3] = {ptrs_trellis, ptrs_suh, ptrs_svh};
    return gemv_common(x, k, gs, widths, groups, tabs, (int64_t) groups * n, 1, k, K, mcg, mul1, workspace, ws_bytes,
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
