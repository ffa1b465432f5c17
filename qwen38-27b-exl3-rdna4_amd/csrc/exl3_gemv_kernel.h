// exl3_gemv_kernel.h -- the fused stream-K GEMV kernel template, shared by exl3_gemv.hip (plain
// launches) and exl3_gemv_gated.hip (gate / up launches with the SiLU-and-mul epilogue), so the two
// sets of instantiations compile in parallel and the plain kernels are unaffected by the gated one.
#pragma once
#include "exl3_device.h"
#include "../../include/exl3_mi355x.h"

#include <utility>

using namespace exl3;

typedef int i32x4 __attribute__((ext_vector_type(4)));

// f(integral_constant<int, I>) for I in the sequence: ring slots are indexed by constants in the
// source, so the ring always lives in registers (a loop index here could leave it in scratch memory)
template <class F, int... I>
__device__ __forceinline__ void static_for(std::integer_sequence<int, I...>, F&& f)
{
    (f(std::integral_constant<int, I>{}), ...);
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
// n / d for 32-bit unsigned n and an invariant divisor d >= 1 in a multiply-high, a subtract and
// two shifts (Granlund and Montgomery, "Division by invariant integers using multiplication",
// PLDI 1994, figure 4.1): m = floor(2^32 (2^l - d) / d) + 1 with l = ceil(log2 d).  The unit
// split's divisions run on the completion path of every launch; 64-bit divisions there cost
// hundreds of instructions each.
struct UDiv {
    uint32_t m, s1, s2;
    static UDiv of(uint32_t d)
    {
        int l = 0;
        while ((1ull << l) < d) ++l;
        UDiv r;
        r.m = (uint32_t) (((1ull << 32) * ((1ull << l) - d)) / d + 1);
        r.s1 = l > 0 ? 1u : 0u;
        r.s2 = l > 0 ? (uint32_t) (l - 1) : 0u;
        return r;
    }
    __host__ __device__ uint32_t div(uint32_t n) const
    {
        const uint32_t t = (uint32_t) (((uint64_t) m * n) >> 32);
        return (t + ((n - t) >> s1)) >> s2;
    }
};

struct GemvGroup {
    const uint32_t* trellis;   // tile words
    const uint16_t* suh;
    const uint16_t* svh;
    uint16_t* y;               // output columns of this group (row stride ldy)
    int n;                     // width (columns)
    int G;                     // workgroups of this group
    int o0, nold, y0;          // its workgroups: grid slots [o0, o0 + nold) among the first
                               // `first` (dispatched first on their CU), then [y0, y0 + G - nold)
    int max_seg;               // partial slots per workgroup
    int64_t part_off;          // first partial (floats) of this group
    int cnt_off;               // first completion counter of this group
    int h;                     // its workgroups dispatched first on their CU (weight wa; the rest wb)
    UDiv d_sg, d_u;            // its split's divisions by S(G) and U
};

struct GemvArgs {
    const uint16_t* x;         // [M][ldx] fp16
    const uint16_t* xr;        // or, when set, every group's rotated input fp16(Had128(fp16(x * suh))):
                               // group i's rows at xr + i * M * k, k apart (computed by one pass per
                               // group before the launch)
    const uint16_t* x_up;      // FORM_SILU_IN: the input rows are fp16(fp16(silu(x)) * x_up), x_up rows
                               // ldx apart as x's (a gated MLP's activation, computed here)
    int64_t ldx;
    GemvGroup g[EXL3_MAX_GROUPS];
    const int64_t* tab_trellis; // optional device pointer tables (grouped M=1 `mgemm` form): they
    const int64_t* tab_suh;     // replace g[i].trellis / suh / svh
    const int64_t* tab_svh;
    int groups, M, k, UPB;
    int first;                 // grid slots dispatched first on their CU (one per CU)
    i32x4 slot_o, slot_y;      // g[i].o0 and g[i].y0 as vectors, read whole by every workgroup
    int wa, wb;                // unit-split weights of first-dispatched / second workgroups on a CU
    UDiv d_wa, d_wb;
    int chunk_units;           // units whose rotated input fits the LDS at once
    int max_per;               // most units any workgroup owns (one LDS chunk when chunk_units == max_per)
    int64_t ldy;
    float* part;               // per group: [G][max_seg][M][128] fp32 partials
    uint32_t* counters;        // per group: [n / 128], zero between calls
};

// partial loads in flight per thread in the reduction (config-1 step: 8 measured +0.8 us, 32 +3.0 us;
// outputs bitwise equal)
constexpr int RED_BATCH = 16;
// completion counters one per 128-byte line: every contributor of every block increments its block's
// counter at about the same time, and atomics to one line serialize at its L2 channel (64- and
// 256-byte spacing measured within 0.1 us of it on the config-1 step)
constexpr int CNT_STRIDE = 32;
constexpr int A_ROW = 136;                      // LDS row of one rotated 128-block (padded, halves)
constexpr int LDS_BUDGET = 64 * 1024;           // per workgroup: 2 workgroups per CU
// 64-row k steps in flight per wave (even).  4 measured faster than 8 (+2 % config 1; gate, down
// and o -1.7, -1.2 and -0.3 us alone): at launch every wave of every CU requests its first ring
// half at once, and the CUs' load queues stall each wave's issue until early data returns, so a
// shallower ring starts the first decode sooner (the first step of gate/up completed ~5 us after
// launch with 8 in flight).  2 and 6 measured slower too: config-1 step 67.1 and 66.1 us against
// 65.3 (one process, outputs bitwise equal).
constexpr int RING = 4;
constexpr int WAVES_PER_SIMD = 2;

// Phase timeline (tracing builds only: -DEXL3_TIMELINE, libexl3_mi355x_timeline.so).  Thread 0 of
// every workgroup writes the 100 MHz s_memrealtime counter at each phase boundary into
// exl3_tl[workgroup][phase] (a vector store; phases a workgroup does not reach keep their last
// value, so a reader clears the array first); exl3_timeline_read copies it out.  The product build
// compiles EXL3_TL to nothing.
enum { TL_ENTRY = 0, TL_ISSUED, TL_LOOP, TL_LOOP_END, TL_STORED, TL_COUNTED, TL_SUMMED, TL_END, TL_HWID, TL_PHASES };
constexpr int TL_MAX_WGS = 4096;
#ifdef EXL3_TIMELINE
__device__ unsigned long long exl3_tl[TL_MAX_WGS * TL_PHASES];
#define EXL3_TL(k)                                                                                        \
    do {                                                                                                  \
        __builtin_amdgcn_sched_barrier(0);                                                                \
        if (threadIdx.x == 0 && blockIdx.x < TL_MAX_WGS)                                                  \
            exl3_tl[blockIdx.x * TL_PHASES + (k)] = __builtin_amdgcn_s_memrealtime();                     \
        __builtin_amdgcn_sched_barrier(0);                                                                \
    } while (0)
#else
#define EXL3_TL(k) ((void) 0)
#endif
// the workgroup's placement, stamped at entry in the tracing build: HW_ID (CU, SH, SE in its low
// 16 bits) and XCC_ID in the high word
#ifdef EXL3_TIMELINE
#define EXL3_TL_HWID()                                                                                    \
    do {                                                                                                  \
        if (threadIdx.x == 0 && blockIdx.x < TL_MAX_WGS)                                                  \
            exl3_tl[blockIdx.x * TL_PHASES + TL_HWID] =                                                   \
                (unsigned long long) __builtin_amdgcn_s_getreg((31 << 11) | 4) |                          \
                ((unsigned long long) __builtin_amdgcn_s_getreg((15 << 11) | 20) << 32);                  \
    } while (0)
#else
#define EXL3_TL_HWID() ((void) 0)
#endif

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
// workgroups of the group are dispatched first on their CU (weight wa = 2); the others are the
// second workgroup on their CU, run their loop at the higher wave priority (the SIMD arbiter
// otherwise favours the older waves) and take the larger weight wb = 3.  A function of the shape
// only (never of m): rows stay bitwise equal to the m == 1 call.
struct Split {
    int U, G, h, wa, wb;
    UDiv d_sg, d_u, d_wa, d_wb;          // divisions by S(G), U, wa and wb
    static Split make(int U, int G, int h, int wa, int wb)
    {
        Split s{U, G, h, wa, wb, {}, {}, {}, {}};
        s.d_sg = UDiv::of(s.S(G));
        s.d_u = UDiv::of((uint32_t) U);
        s.d_wa = UDiv::of((uint32_t) wa);
        s.d_wb = UDiv::of((uint32_t) wb);
        return s;
    }
    __host__ __device__ uint32_t S(int w) const
    {
        return (uint32_t) wa * (uint32_t) (w < h ? w : h) + (uint32_t) wb * (uint32_t) (w > h ? w - h : 0);
    }
    __host__ __device__ int lo(int w) const { return (int) d_sg.div((uint32_t) U * S(w)); }
    // the workgroup owning unit u: the largest w in [0, G) with lo(w) <= u, i.e. S(w) <= T
    __host__ __device__ int owner(int u) const
    {
        const uint32_t T = d_u.div((uint32_t) (u + 1) * S(G) + (uint32_t) (U - 1)) - 1u;
        const uint32_t wah = (uint32_t) wa * (uint32_t) h;
        const int w = T < wah ? (int) d_wa.div(T) : h + (int) d_wb.div(T - wah);
        return w < G - 1 ? w : G - 1;
    }
    // the 32-bit forms above hold: every numerator is at most U * S(G) + U - 1
    bool fits32() const { return (uint64_t) U * S(G) + (uint64_t) U < (1ull << 32); }
    // most units any workgroup owns
    int max_units() const
    {
        const int wmax = wa > wb ? wa : wb;
        return (int) (((int64_t) U * wmax + S(G) - 1) / S(G)) + 1;
    }
};


// Two workgroups (8 waves) per CU are resident at once: up to 256 registers per lane, enough for
// a ring deep enough that one wave alone keeps its SIMD busy.
// MT: 16-row MFMA tiles of the input rows (0: exactly one row, a compile-time M; 1 to 4; 5 and 6:
// one tile, like 1, with the 16-byte-load reduction of the multi-tile forms, 6 with one quad of
// loads in flight per contributor batch instead of four; 7: two tiles, like 2, with two quads).
// FORM:
//   FORM_PLAIN   the EXL3 linear of each group;
//   FORM_GATED   groups 0 (gate) and 1 (up) of equal width; the workgroup completing a block of
//                both writes fp16(fp16(silu(gate)) * up) to g[0].y instead of the two outputs;
//   FORM_SILU_IN the input rows are fp16(fp16(silu(x)) * x_up), formed as they load;
//   FORM_F32OUT  the plain linear with an fp32 output (single row only): C stays fp32 (no fp16
//                rounding) and y = (float) (H C r) * svh.
enum { FORM_PLAIN = 0, FORM_GATED = 1, FORM_SILU_IN = 2, FORM_F32OUT = 3 };

template <int BITS, int CB, int MT_, int FORM>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WAVES_PER_SIMD, WAVES_PER_SIMD))) gemv_kernel(GemvArgs a)
{
    constexpr bool GATED = FORM == FORM_GATED;
    extern __shared__ __align__(16) uint16_t smem[];
    EXL3_TL(TL_ENTRY);
    EXL3_TL_HWID();
    {
        // Request every 64-byte line of the argument struct at once: the argument reads that
        // depend on earlier ones (the group's fields after the group index, then the input
        // pointers) hit the scalar cache instead of each costing a memory round trip before the
        // first trellis request.
        const uint32_t __attribute__((address_space(4)))* kp =
            (const uint32_t __attribute__((address_space(4)))*) __builtin_amdgcn_kernarg_segment_ptr();
        uint32_t touch = 0;
#pragma unroll
        for (int l = 0; l < (int) ((sizeof(GemvArgs) + 63) / 64); ++l) touch += kp[l * 16];
        asm volatile("" ::"s"(touch));
    }
    __shared__ int s_last[256];
    __shared__ int s_list[256];
    __shared__ int s_nred;
    // per block of a counting batch: first contributor, contributor count, the first contributor's
    // segment holding the block (gated: for gate, then up)
    __shared__ int s_own[GATED ? 6 : 3][256];
    // the group of this workgroup: a flattened grid, each group its own range of workgroups
    // Every group owns slots among the first-dispatched workgroups (older waves, favoured by the
    // SIMD arbiter) and among the second ones, in proportion to its size, so the weighted unit
    // split balances each group's two kinds of workgroups.
    // (The thresholds come as two vectors selected element-wise: a select between two scalar
    // argument loads would become one load from a selected address, a dependent round trip at
    // the start of every workgroup.)
    const int b = blockIdx.x;
    const bool older = b < a.first;
    const i32x4 so = a.slot_o, sy = a.slot_y;
    const int t1 = older ? so[1] : sy[1], t2 = older ? so[2] : sy[2], t3 = older ? so[3] : sy[3];
    int grp = 0;
    if (a.groups > 1 && b >= t1) grp = 1;
    if (a.groups > 2 && b >= t2) grp = 2;
    if (a.groups > 3 && b >= t3) grp = 3;
    // constant indices only: a runtime index into the kernel-argument struct would copy it to
    // scratch memory, and every later read of it would be a vector-memory load
    const GemvGroup gg = grp == 0 ? a.g[0] : grp == 1 ? a.g[1] : grp == 2 ? a.g[2] : a.g[3];
    const int w = older ? b - gg.o0 : gg.nold + (b - gg.y0);
    constexpr int MT = MT_ == 0 || MT_ == 5 || MT_ == 6 ? 1 : MT_ == 7 ? 2 : MT_;
    // approximate mul1 routes (CB 3: affine, CB 4: int8 activations): the decoder emits 1024 + s
    // unscaled; per (unit, row) the input rotation leaves in the LDS row's padding the row's input
    // sum (affine) or its int8 scale q and integer sum (int8)
    constexpr bool AFF = CB == 3, I8 = CB == 4;
    constexpr float MUL1_K_INV = 0.00676727294921875f, MUL1_K_BIAS = -10.3828125f;   // fp16 0x1EEE, 0xC931
    constexpr float MUL1_K_SUM = 1024.0f * MUL1_K_INV + MUL1_K_BIAS;                    // -3.453125, exact
    const int G = gg.G, UPB = a.UPB, M = MT_ == 0 ? 1 : a.M;
    const int NB = gg.n / 128, NT = gg.n / 16, U = NB * UPB;
    const Split sp{U, G, gg.h, a.wa, a.wb, gg.d_sg, gg.d_u, a.d_wa, a.d_wb};
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
    // a gated launch counts both groups' contributions to block cb in group 0's counter cb
    constexpr bool gated = GATED;
    uint32_t* const counters = a.counters + (int64_t) (gated ? a.g[0].cnt_off : gg.cnt_off) * CNT_STRIDE;
    // the trellis as one raw buffer (layers of 4 GiB and more are declined on the host)
    const uint64_t trel_bytes = (uint64_t) a.k * gg.n * BITS / 8;
    const __amdgpu_buffer_rsrc_t trsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(trel), 0, (int) (uint32_t) trel_bytes, RAW_BUFFER_FLAGS);
    gc_u16* const gsuh = as_global(suh);
    // svh is read only after the completion counters, as device-scope (sc1) raw-buffer loads like
    // the partial sums around it: every load after a counter atomic then carries sc1, which a check
    // of the built code can require without telling the two apart
    auto sc1_rsrc = [](const uint16_t* p) __attribute__((always_inline)) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p), 0, 0x7FFFFFFF, RAW_BUFFER_FLAGS);
    };
    auto sv32 = [](__amdgpu_buffer_rsrc_t r, int e) __attribute__((always_inline)) {
        return (uint32_t) __builtin_amdgcn_raw_buffer_load_b32(r, (uint32_t) (2 * e), 0, SC1);
    };
    auto sv128 = [](__amdgpu_buffer_rsrc_t r, int e) __attribute__((always_inline)) {
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t) (2 * e), 0, SC1));
    };
    const __amdgpu_buffer_rsrc_t svsrc = sc1_rsrc(svh);
    // the input rows: x (rotated here, per workgroup) or the group's pre-rotated rows
    const bool pre = MT_ != 0 && a.xr != nullptr;
    gc_u16* const gx = as_global(pre ? a.xr + (int64_t) grp * M * a.k : a.x);
    // gated-MLP input: the activation silu(gate) * up is formed from the two rows as they load
    constexpr bool silu_in = FORM == FORM_SILU_IN;
    gc_u16* const gxu = as_global(a.x_up);
    const int64_t ldx = pre ? (int64_t) a.k : a.ldx;
    // outputs go out as write-through (device-scope) stores: no dirty output lines are left in L2
    // for the end-of-kernel writeback (~0.2 us off the small launches)
    const __amdgpu_buffer_rsrc_t ysrc = __builtin_amdgcn_make_buffer_rsrc(y, 0, 0x7FFFFFFF, RAW_BUFFER_FLAGS);
    const __amdgpu_buffer_rsrc_t y0src = __builtin_amdgcn_make_buffer_rsrc(a.g[0].y, 0, 0x7FFFFFFF, RAW_BUFFER_FLAGS);
    // LDS: the rotated input of a chunk of units, M rows per unit followed by one zero row (the A
    // operand of MFMA rows >= M), then the fp16 C of one block for the output transform
    const int UROWS = M + 1;
    uint16_t* lds_a = smem;                                   // [chunk_units][M + 1][A_ROW]
    uint16_t* lds_c = smem + a.chunk_units * UROWS * A_ROW;   // [2 M][A_ROW]: two blocks side by side
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

    // Transforms run float64 butterflies (the pre-rotation pass too, so every layout gives the same
    // values): the rotated input and y are then the correctly rounded fp16 of the exact transforms,
    // which the reference's strict M = 1 gates assume (a last-place flip of one large output alone
    // is ~3e-3 of the output RMS).  Float32 butterflies measured no faster here: the prologue waits
    // on memory, not on the rotation's VALU work.
    // Approximate routes: the row's input values (8 a lane, `width` lanes a row) -> the values the
    // MFMA consumes, with the row's scalars written to the padding of its LDS row (lds_row: the
    // row's first half, live: this lane group stores).  Every lane of the group takes part in the
    // reductions.
    auto approx_row = [&](u32x4 r, int width, uint16_t* lds_row, bool live) __attribute__((always_inline)) {
        if constexpr (AFF || I8) {
            const f16x8 h = __builtin_bit_cast(f16x8, r);
            auto red = [&](float v, bool mx) __attribute__((always_inline)) {
                for (int o = 1; o < width; o <<= 1) {
                    const float w = __shfl_xor(v, o, width);
                    v = mx ? fmaxf(v, w) : v + w;
                }
                return v;
            };
            float* pad = reinterpret_cast<float*>(lds_row + 128);
            const bool leader = live && ((int) threadIdx.x & (width - 1)) == 0;
            if constexpr (AFF) {
                // pairwise in the lane, then across lanes: the 64-lane form (2 values a lane, the
                // rest zero) adds in exactly the 16-lane form's order, so a row's sum, and with it
                // every output, is the same bitwise in both
                const float p0 = (float) h[0] + (float) h[1], p1 = (float) h[2] + (float) h[3];
                const float p2 = (float) h[4] + (float) h[5], p3 = (float) h[6] + (float) h[7];
                float sum = (p0 + p1) + (p2 + p3);
                sum = red(sum, false);
                if (leader) pad[0] = sum;
                return r;
            } else {
                // symmetric int8 of the slice: q = max(|a|, 1e-8) / 127, v = clamp(rint(a / q))
                float mx = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) mx = fmaxf(mx, __builtin_fabsf((float) h[i]));
                const float q = fmaxf(red(mx, true), 1e-8f) / 127.f;
                f16x8 v;
                float sum = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float t = fminf(fmaxf(__builtin_rintf((float) h[i] / q), -127.f), 127.f);
                    v[i] = (f16) t;
                    sum += t;
                }
                sum = red(sum, false);
                if (leader) {
                    pad[0] = q;
                    pad[1] = sum;
                }
                return __builtin_bit_cast(u32x4, v);
            }
        } else {
            (void) width; (void) lds_row; (void) live;
            return r;
        }
    };

    // The prologue and the completion phase sit on every workgroup's critical path while other
    // workgroups on the same SIMDs run VALU-heavy decode loops: give them issue priority.
    __builtin_amdgcn_s_setprio(2);

    // ---- first input chunk: the x / suh loads of its first two 16-lane job passes go out before
    // the trellis ring (a pass requested after the ring waits behind every workgroup's ring)
    const int nfirst = min(a.chunk_units, uhi - ulo) * M;
    u32x4 px = {0u, 0u, 0u, 0u}, ps = px, px2 = px, ps2 = px, pu = px, pu2 = px;
    // a single row of at most 4 jobs: one job per wave, two columns a lane (had128_x2, a fourth
    // of the 16-lane transform's latency)
    const bool wide = MT_ == 0 && nfirst <= 4;
    // The loads are unconditional: a job past nfirst reads job 0's (in-bounds) input, and its
    // results are never stored (the 16 lanes of a job exchange data only among themselves).  A
    // load under a condition would merge with the zero-initialised register after the branch, and
    // that copy would wait for the load before the trellis requests below could issue.
    if (wide) {
        const int u = ulo + (wave < nfirst ? wave : 0);
        const int col = (u - (u / UPB) * UPB) * 128 + 2 * lane;
        px.x = *reinterpret_cast<gc_u32*>(gx + col);
        if (silu_in) pu.x = *reinterpret_cast<gc_u32*>(gxu + col);
        ps.x = *reinterpret_cast<gc_u32*>(gsuh + col);
    } else {
        const int i = threadIdx.x >> 4;
        {
            int m, col;
            job_src(ulo, i < nfirst ? i : 0, m, col);
            px = *reinterpret_cast<gc_u32x4*>(gx + (int64_t) m * ldx + col);
            if (silu_in) pu = *reinterpret_cast<gc_u32x4*>(gxu + (int64_t) m * ldx + col);
            if (!pre) ps = *reinterpret_cast<gc_u32x4*>(gsuh + col);
        }
        if (nfirst > 16) {
            int m, col;
            job_src(ulo, i + 16 < nfirst ? i + 16 : 0, m, col);
            px2 = *reinterpret_cast<gc_u32x4*>(gx + (int64_t) m * ldx + col);
            if (silu_in) pu2 = *reinterpret_cast<gc_u32x4*>(gxu + (int64_t) m * ldx + col);
            if (!pre) ps2 = *reinterpret_cast<gc_u32x4*>(gsuh + col);
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
    // the first half of the ring goes out now, the second after the first input rotation: a wave
    // stalls at issue once its CU's load queue is full, so the rotation's VALU work would otherwise
    // wait for the whole ring to be issued
    auto fill = [&](auto I) __attribute__((always_inline)) {
        constexpr int i = decltype(I)::value;
        load_qblock_buf<BITS>(trsrc, off_main, off_prev, lp + (i & 1) * STEP_D, Wr[i]);
        if (i & 1) advance_load();
    };
    static_for(std::make_integer_sequence<int, RING / 2>{}, fill);
    EXL3_TL(TL_ISSUED);
    // rotated input of units [c0, c1) -> LDS; with have_first the lane's first two 16-lane jobs use
    // (x0, s0, u0) and (x1, s1, u1) (u: the up rows of a gated-MLP input)
    auto rotate_chunk = [&](int c0, int c1, u32x4 x0, u32x4 s0, u32x4 x1, u32x4 s1, u32x4 u0, u32x4 u1,
                            bool have_first) __attribute__((always_inline)) {
        const int njobs = (c1 - c0) * M;
        const int i = threadIdx.x >> 4;
        if (MT_ != 0 && pre) {
            // pre-rotated rows: a plain copy into LDS, PRE_BATCH passes of loads in flight before
            // their stores (one round trip per batch instead of one per 16-job pass)
            constexpr int PRE_BATCH = 8;
            for (int b0 = i; b0 - (threadIdx.x & 63) / 16 < njobs; b0 += 16 * PRE_BATCH) {
                u32x4 buf[PRE_BATCH];
#pragma unroll
                for (int p = 0; p < PRE_BATCH; ++p) {
                    const int i3 = b0 + 16 * p;
                    buf[p] = u32x4{0u, 0u, 0u, 0u};
                    if (i3 < njobs) {
                        int m3, col3;
                        job_src(c0, i3, m3, col3);
                        buf[p] = *reinterpret_cast<gc_u32x4*>(gx + (int64_t) m3 * ldx + col3);
                    }
                }
#pragma unroll
                for (int p = 0; p < PRE_BATCH; ++p) {
                    const int i3 = b0 + 16 * p;
                    if (i3 - (threadIdx.x & 63) / 16 >= njobs) break;   // whole 16-lane groups of the wave
                    int m3 = 0, col3;
                    if (i3 < njobs) job_src(c0, i3, m3, col3);
                    uint16_t* row3 = lds_a + ((i3 < njobs ? i3 / M : 0) * UROWS + m3) * A_ROW;
                    const u32x4 r3 = approx_row(buf[p], 16, row3, i3 < njobs);
                    if (i3 < njobs) *reinterpret_cast<u32x4*>(row3 + 8 * (threadIdx.x & 15)) = r3;
                }
            }
            return;
        }
        if (i - (threadIdx.x & 63) / 16 < njobs) {            // waves with a job (whole 16-lane groups)
            if (!have_first && i < njobs) {
                int m, col;
                job_src(c0, i, m, col);
                x0 = *reinterpret_cast<gc_u32x4*>(gx + (int64_t) m * ldx + col);
                if (silu_in) u0 = *reinterpret_cast<gc_u32x4*>(gxu + (int64_t) m * ldx + col);
                if (!pre) s0 = *reinterpret_cast<gc_u32x4*>(gsuh + col);
            }
            if (silu_in) x0 = silu_mul_x8(x0, u0);
            u32x4 r = pre ? x0 : had128_x8<double>(x0, s0, true, u32x4{0u, 0u, 0u, 0u}, false, r_scale<double>());
            {
                int m = 0, col;
                if (i < njobs) job_src(c0, i, m, col);
                uint16_t* row = lds_a + ((i < njobs ? i / M : 0) * UROWS + m) * A_ROW;
                r = approx_row(r, 16, row, i < njobs);
                if (i < njobs) *reinterpret_cast<u32x4*>(row + 8 * (threadIdx.x & 15)) = r;
            }
            for (int i2 = i + 16; i2 - (threadIdx.x & 63) / 16 < njobs; i2 += 16) {
                u32x4 xv = {0u, 0u, 0u, 0u}, sv = xv, uv = xv;
                int m = 0, col = 0;
                if (i2 < njobs) {
                    job_src(c0, i2, m, col);
                    if (have_first && i2 == i + 16) {
                        xv = x1;
                        sv = s1;
                        uv = u1;
                    } else {
                        xv = *reinterpret_cast<gc_u32x4*>(gx + (int64_t) m * ldx + col);
                        if (silu_in) uv = *reinterpret_cast<gc_u32x4*>(gxu + (int64_t) m * ldx + col);
                        if (!pre) sv = *reinterpret_cast<gc_u32x4*>(gsuh + col);
                    }
                }
                if (silu_in) xv = silu_mul_x8(xv, uv);
                u32x4 r2 = pre ? xv : had128_x8<double>(xv, sv, true, u32x4{0u, 0u, 0u, 0u}, false, r_scale<double>());
                uint16_t* row2 = lds_a + ((i2 < njobs ? i2 / M : 0) * UROWS + m) * A_ROW;
                r2 = approx_row(r2, 16, row2, i2 < njobs);
                if (i2 < njobs) *reinterpret_cast<u32x4*>(row2 + 8 * (threadIdx.x & 15)) = r2;
            }
        }
    };
    int c0 = ulo, c1 = min(ulo + a.chunk_units, uhi);
    if (wide) {
        if (wave < nfirst) {
            const uint32_t xin = silu_in ? silu_mul_x2(px.x, pu.x) : px.x;
            uint32_t r = had128_x2<double>(xin, ps.x, true, 0u, false, r_scale<double>());
            if constexpr (AFF || I8) {
                // one row of 128 per wave, 2 values a lane: the same helper on a 64-lane group
                const u32x4 r8 = approx_row(u32x4{r, 0u, 0u, 0u}, 64, lds_a + (wave * UROWS) * A_ROW, true);
                r = r8.x;
            }
            *reinterpret_cast<uint32_t*>(lds_a + (wave * UROWS) * A_ROW + 2 * lane) = r;
        }
    } else {
        rotate_chunk(c0, c1, px, ps, px2, ps2, pu, pu2, true);
    }
    static_for(std::make_integer_sequence<int, RING / 2>{}, [&](auto I) __attribute__((always_inline)) {
        fill(std::integral_constant<int, RING / 2 + decltype(I)::value>{});
    });
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
    // approximate routes: the block segment's input sums per accumulator row (affine), or the
    // segment's folded sum of finished units (int8: acc holds one unit at a time)
    float asum_seg[MT][4];
    f32x4 acc_seg[2][MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) asum_seg[mt][v] = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc_seg[h][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // the padding scalars of unit row mt * 16 + 4 g + v of this lane (rows >= M: the zero row)
    auto pad_of = [&](const uint16_t* unit_a, int mt, int v) __attribute__((always_inline)) {
        const int row = mt * 16 + 4 * g + v;
        return reinterpret_cast<const float*>(unit_a + (row < M ? row : M) * A_ROW + 128);
    };

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
                    float val = acc[h][mt][v];
                    if constexpr (AFF) val = MUL1_K_INV * acc[h][mt][v] + MUL1_K_BIAS * asum_seg[mt][v];
                    if constexpr (I8) val = acc_seg[h][mt][v];
                    if (m < M)
                        __hip_atomic_store(&slab[m * 128 + colb + 8 * h], val, __ATOMIC_RELAXED,
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
        const uint16_t* unit_a = lds_a + (u0 + i / 2 - c0) * UROWS * A_ROW;
        if (!(i & 1)) {
            if (left == 0) {                                  // a new 128-column block starts
                write_partial(cb_cur);
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        acc[h][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
                        acc_seg[h][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
                    }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int v = 0; v < 4; ++v) asum_seg[mt][v] = 0.f;
                ++cb_cur;
                left = UPB;
            }
            --left;
            if constexpr (AFF) {                              // the unit's input sums join the segment
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int v = 0; v < 4; ++v) asum_seg[mt][v] += pad_of(unit_a, mt, v)[0];
            }
        }
        step(Wr[i], unit_a, i & 1, refill);
        if constexpr (I8) {
            if (i & 1) {                                      // unit done: fold q (k_inv acc + (1024 k_inv + k_bias) sum v)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const float* pd = pad_of(unit_a, mt, v);
                        const float q = pd[0], sv = pd[1];
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            acc_seg[h][mt][v] += q * (MUL1_K_INV * acc[h][mt][v] + MUL1_K_SUM * sv);
                            acc[h][mt][v] = 0.f;
                        }
                    }
            }
        }
        if ((i & 1) && refill) advance_load();
    };
    auto next_chunk = [&](int u0) __attribute__((always_inline)) {      // chunks hold whole ring turns
        if (u0 == c1) {
            c0 = c1;
            c1 = min(c0 + a.chunk_units, uhi);
            __syncthreads();
            rotate_chunk(c0, c1, px, ps, px2, ps2, pu, pu2, false);
            __syncthreads();
        }
    };

    // In the loop the second-dispatched workgroup of a CU runs at the higher priority (and takes
    // the larger unit share, weights 2 : 3): it starts later, and at equal priority the arbiter
    // favours the older wave, so the younger one's loop ended last (timeline probe).
    EXL3_TL(TL_LOOP);
    if (older) __builtin_amdgcn_s_setprio(0);
    else __builtin_amdgcn_s_setprio(1);
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
    EXL3_TL(TL_LOOP_END);
    __builtin_amdgcn_s_setprio(2);
    write_partial(cb_cur);

    // ---- completion: count this workgroup into every block it touched, reduce those it completed
    // The partials are device-scope (write-through) stores: once complete (vmcnt(0)) they are
    // visible to device-scope loads from any XCD, so no cache-wide release is needed.
    wait_stores_complete();
    EXL3_TL(TL_STORED);
    __syncthreads();
    const int nblk = cb_cur - seg0_cb + 1;
    // completed blocks (gated: block pairs, 2M rows each: gate, then up) reduced side by side
    // blocks reduced side by side: two up to 8 rows (one round trip of partial loads for both;
    // measured slower from 16 rows, where one block already fills the passes)
    // (MT 5 and 6, up to 16 rows: two blocks side by side, one pass (MT 5; MT 6 at up to 4 rows) of
    // 16-byte loads for both: a second pass of partial loads cost 16-row launches ~5 us)
    const int RB = gated && M > 1 ? 1 : (M <= (MT_ >= 5 ? 16 : 8) ? 2 : 1);
    const int RM = gated ? 2 * M : M;
    const Split sp0{U, a.g[0].G, a.g[0].h, a.wa, a.wb, a.g[0].d_sg, a.g[0].d_u, a.d_wa, a.d_wb};
    const Split sp1{U, a.g[1].G, a.g[1].h, a.wa, a.wb, a.g[1].d_sg, a.g[1].d_u, a.d_wa, a.d_wb};
    for (int b0 = 0; b0 < nblk; b0 += 256) {
        const int nb = min(256, nblk - b0);
        if ((int) threadIdx.x < nb) {                         // one counter per thread, all in flight
            const int t = threadIdx.x;
            const int cb = seg0_cb + b0 + t;
            const uint32_t prev = __hip_atomic_fetch_add(&counters[cb * CNT_STRIDE], 1u, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            // the block's contributors (integer divisions) while the counter round trip is in flight
            __builtin_amdgcn_sched_barrier(0);
            const int uf = cb * UPB, ul = cb * UPB + UPB - 1;
            int before;                                       // contributors before the last one
            if constexpr (GATED) {
                const int wf0 = sp0.owner(uf), wl0 = sp0.owner(ul), wf1 = sp1.owner(uf), wl1 = sp1.owner(ul);
                s_own[0][t] = wf0;
                s_own[1][t] = wl0 - wf0 + 1;
                s_own[2][t] = cb - sp0.lo(wf0) / UPB;
                s_own[3][t] = wf1;
                s_own[4][t] = wl1 - wf1 + 1;
                s_own[5][t] = cb - sp1.lo(wf1) / UPB;
                before = wl0 - wf0 + wl1 - wf1 + 1;
            } else {
                const int wf = sp.owner(uf), wl = sp.owner(ul);
                s_own[0][t] = wf;
                s_own[1][t] = wl - wf + 1;
                s_own[2][t] = cb - sp.lo(wf) / UPB;
                before = wl - wf;
            }
            s_last[t] = prev == (uint32_t) before ? 1 : 0;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int c = 0;
            for (int bi = 0; bi < nb; ++bi)
                if (s_last[bi]) s_list[c++] = bi;             // index in the batch (block seg0_cb + b0 + bi)
            s_nred = c;
        }
        __syncthreads();
        const int nred = __builtin_amdgcn_readfirstlane(s_nred);
        EXL3_TL(TL_COUNTED);
        for (int r0 = 0; r0 < nred; r0 += RB) {
            const int rb = min(RB, nred - r0);
            // svh of the first output-transform pass, requested before the partial loads so that its
            // round trip overlaps theirs
            const int l16 = threadIdx.x & 15;
            u32x4 sv_first = {0u, 0u, 0u, 0u}, sv_first_u = sv_first;
            {
                const int rr = threadIdx.x >> 4;
                if (gated && MT_ == 0) {
                    // single row: pair r goes to wave r, two columns a lane
                    if (wave < rb) {
                        const int cb = seg0_cb + b0 + s_list[r0 + wave];
                        sv_first.x = sv32(sc1_rsrc(a.g[0].svh), cb * 128 + 2 * lane);
                        sv_first_u.x = sv32(sc1_rsrc(a.g[1].svh), cb * 128 + 2 * lane);
                    }
                } else if (gated) {
                    if (rr < rb * M) {
                        const int cb = seg0_cb + b0 + s_list[r0 + rr / M];
                        sv_first = sv128(sc1_rsrc(a.g[0].svh), cb * 128 + 8 * l16);
                        sv_first_u = sv128(sc1_rsrc(a.g[1].svh), cb * 128 + 8 * l16);
                    }
                } else if (MT_ == 0) {
                    // single row: block r of the pair goes to wave r, two columns a lane
                    if (wave < rb)
                        sv_first.x = sv32(svsrc, (seg0_cb + b0 + s_list[r0 + wave]) * 128 + 2 * lane);
                } else if (rr < rb * M) {
                    sv_first = sv128(svsrc, (seg0_cb + b0 + s_list[r0 + rr / M]) * 128 + 8 * l16);
                }
            }
            // contributor wf holds block cb in its segment cb - first_cb(wf); every later
            // contributor starts inside cb, so its segment is 0.  Loads go out in batches of
            // RED_BATCH and each sum runs in contributor order; the gated form sums two elements at
            // a time with both elements' loads in flight together (its passes hold twice the rows).
            const int total = rb * RM * 128;
            // both groups' partial-slot geometry as scalars: a per-element choice between two
            // argument fields would otherwise become a vector load from a per-lane argument address
            const int ms0 = __builtin_amdgcn_readfirstlane(a.g[0].max_seg);
            const int ms1 = __builtin_amdgcn_readfirstlane(a.g[1].max_seg);
            const float* const pg0 = a.part + uniform_i64(a.g[0].part_off);
            const float* const pg1 = a.part + uniform_i64(a.g[1].part_off);
            // element e of the pass: contributor 0's partial, contributor 1's (the rest follow
            // cstride floats apart), the contributor count and the element's LDS slot
            auto elem = [&](int e, const float*& p0, const float*& p1, int64_t& cstride, int& nc, int& lofs)
                __attribute__((always_inline)) {
                const int r = e / (RM * 128);
                int el = e - r * (RM * 128);
                const int bi = s_list[r0 + r];
                // the group whose partials hold element el: this workgroup's, or gate / up rows
                const bool up = gated && el >= M * 128;
                if (up) el -= M * 128;
                const int max_seg = !gated ? gg.max_seg : up ? ms1 : ms0;
                const float* pr = !gated ? part_grp : up ? pg1 : pg0;
                const int wf = s_own[up ? 3 : 0][bi], seg_f = s_own[up ? 5 : 2][bi];
                nc = s_own[up ? 4 : 1][bi];
                cstride = (int64_t) max_seg * M * 128;
                p0 = pr + ((int64_t) wf * max_seg + seg_f) * M * 128 + el;
                p1 = pr + (int64_t) (wf + 1) * cstride + el;
                lofs = (r * RM + (up ? M : 0) + (el >> 7)) * A_ROW + (el & 127);
            };
            auto part_load = [&](const float* p0, const float* p1, int64_t cstride, int c) __attribute__((always_inline)) {
                return __hip_atomic_load(c == 0 ? p0 : p1 + (int64_t) (c - 1) * cstride, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
            };
            if (GATED && MT_ != 0 && M > 1) {
                // a pair per pass: gate rows then up rows, each group's contributors shared by its
                // elements; 4 elements x 8 contributors of loads in flight per thread
                const int bi = s_list[r0];
                const int half = M * 128;
                const int64_t csa = (int64_t) a.g[0].max_seg * M * 128, csb = (int64_t) a.g[1].max_seg * M * 128;
                const int nca = s_own[1][bi], ncb = s_own[4][bi];
                const float* a0 = a.part + a.g[0].part_off + ((int64_t) s_own[0][bi] * a.g[0].max_seg + s_own[2][bi]) * M * 128;
                const float* b0 = a.part + a.g[1].part_off + ((int64_t) s_own[3][bi] * a.g[1].max_seg + s_own[5][bi]) * M * 128;
                const float* a1 = a.part + a.g[0].part_off + (int64_t) (s_own[0][bi] + 1) * csa;
                const float* b1 = a.part + a.g[1].part_off + (int64_t) (s_own[3][bi] + 1) * csb;
                const int ncmax = nca > ncb ? nca : ncb;
                for (int e0 = threadIdx.x; e0 < total; e0 += 1024) {
                    float sum[4] = {0.f, 0.f, 0.f, 0.f};
                    for (int c0 = 0; c0 < ncmax; c0 += 8) {
                        float v[4][8];
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const int e = e0 + 256 * j;
                            const bool up = e >= half;
                            const int el = up ? e - half : e;
                            const int nc = e < total ? (up ? ncb : nca) : 0;
#pragma unroll
                            for (int cc = 0; cc < 8; ++cc) {
                                const int c = c0 + cc;
                                const float* src = (c == 0 ? (up ? b0 : a0)
                                                           : (up ? b1 + (int64_t) (c - 1) * csb : a1 + (int64_t) (c - 1) * csa)) + el;
                                v[j][cc] = c < nc ? __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
                            }
                        }
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const int e = e0 + 256 * j;
                            const int nc = e < total ? (e >= half ? ncb : nca) : 0;
#pragma unroll
                            for (int cc = 0; cc < 8; ++cc)
                                if (c0 + cc < nc) sum[j] += v[j][cc];
                        }
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int e = e0 + 256 * j;
                        if (e < total) lds_c[(e >> 7) * A_ROW + (e & 127)] = f16_bits((f16) sum[j]);
                    }
                }
            } else if (!GATED && MT_ == 1 && M > 1 && rb == 2) {
                // up to 16 rows, two blocks side by side up to 8: 4-byte loads, a thread keeping 4
                // elements x 8 contributors in flight.  (The 16-byte form below in this
                // instantiation too took 8 and 16 rows 1-3 us faster but 2 and 4 rows 1-1.9 us
                // slower: its registers changed the whole kernel's allocation.)
                {
                    // two blocks side by side (M <= 8): a thread keeps 4 elements x 8 contributors of
                    // loads in flight, each element summing its block's contributors in order (one
                    // round trip for both blocks: -1.5 to -2 us at M = 2 / 4 on gate; the one-block
                    // pass below stays from 16 rows, where its hoisted pointers measured faster)
                    const int half = M * 128;
                    const int bi0 = s_list[r0], bi1 = s_list[r0 + 1];
                    const int64_t cs = (int64_t) gg.max_seg * M * 128;
                    const int nc0 = s_own[1][bi0], nc1 = s_own[1][bi1];
                    const float* const q0 = part_grp + ((int64_t) s_own[0][bi0] * gg.max_seg + s_own[2][bi0]) * M * 128;
                    const float* const q1 = part_grp + (int64_t) (s_own[0][bi0] + 1) * cs;
                    const float* const r0p = part_grp + ((int64_t) s_own[0][bi1] * gg.max_seg + s_own[2][bi1]) * M * 128;
                    const float* const r1p = part_grp + (int64_t) (s_own[0][bi1] + 1) * cs;
                    const int ncmax = nc0 > nc1 ? nc0 : nc1;
                    for (int e0 = threadIdx.x; e0 < total; e0 += 1024) {
                        float sum[4] = {0.f, 0.f, 0.f, 0.f};
                        for (int c0 = 0; c0 < ncmax; c0 += 8) {
                            float v[4][8];
    #pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                const int e = e0 + 256 * j;
                                const bool second = e >= half;
                                const int el = second ? e - half : e;
                                const int nc = e < total ? (second ? nc1 : nc0) : 0;
    #pragma unroll
                                for (int cc = 0; cc < 8; ++cc) {
                                    const int c = c0 + cc;
                                    const float* src = (c == 0 ? (second ? r0p : q0)
                                                               : (second ? r1p : q1) + (int64_t) (c - 1) * cs) + el;
                                    v[j][cc] = c < nc ? __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
                                }
                            }
    #pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                const int e = e0 + 256 * j;
                                const int nc = e < total ? (e >= half ? nc1 : nc0) : 0;
    #pragma unroll
                                for (int cc = 0; cc < 8; ++cc)
                                    if (c0 + cc < nc) sum[j] += v[j][cc];
                            }
                        }
    #pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const int e = e0 + 256 * j;
                            if (e < total) lds_c[(e >> 7) * A_ROW + (e & 127)] = f16_bits((f16) sum[j]);
                        }
                    }
                }
            } else if (!GATED && MT_ == 1 && M > 1) {
                {
                    // one block per pass (rb == 1): every element shares the block's contributors, so a
                    // thread keeps 4 elements x 8 contributors of loads in flight (sums in contributor order)
                    const int bi = s_list[r0];
                    const int wf = s_own[0][bi], nc = s_own[1][bi];
                    const int64_t cs = (int64_t) gg.max_seg * M * 128;
                    const float* p0 = part_grp + ((int64_t) wf * gg.max_seg + s_own[2][bi]) * M * 128;
                    const float* p1 = part_grp + (int64_t) (wf + 1) * cs;
                    for (int e0 = threadIdx.x; e0 < total; e0 += 1024) {
                        float sum[4] = {0.f, 0.f, 0.f, 0.f};
                        for (int c0 = 0; c0 < nc; c0 += 8) {
                            float v[4][8];
    #pragma unroll
                            for (int j = 0; j < 4; ++j)
    #pragma unroll
                                for (int cc = 0; cc < 8; ++cc) {
                                    const int c = c0 + cc, e = e0 + 256 * j;
                                    const float* src = (c == 0 ? p0 : p1 + (int64_t) (c - 1) * cs) + e;
                                    v[j][cc] = c < nc && e < total
                                                   ? __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                                   : 0.f;
                                }
    #pragma unroll
                            for (int j = 0; j < 4; ++j)
    #pragma unroll
                                for (int cc = 0; cc < 8; ++cc)
                                    if (c0 + cc < nc) sum[j] += v[j][cc];
                        }
    #pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const int e = e0 + 256 * j;
                            if (e < total) lds_c[(e >> 7) * A_ROW + (e & 127)] = f16_bits((f16) sum[j]);
                        }
                    }
                }
            } else if (!GATED && MT_ != 0 && M > 1) {
                // MT 5 / 6 and 17 to 64 rows (two blocks side by side up to 16, else one block per pass): partials as
                // 16-byte device-scope loads, a thread summing 4 consecutive elements of one row per
                // load, each element over its block's contributors in order (the order of every
                // other form), J x 8 loads in flight per thread.  Scalar 4-byte loads carried 4 x fewer elements per round trip:
                // at 32 rows the reduction was the critical workgroup's longest phase (down 8 us, at
                // 64 rows 35 us); with these loads down takes 41.1 against 48.9 us at 32 rows, 67.3
                // against 83.3 at 64.  MT 6 keeps one quad per thread (J = 1: the 1024 elements of two
                // blocks of up to 4 rows in one pass, more rows in further passes): the 128 VGPRs of
                // four quads would raise the whole kernel's allocation (MT 5: 220, MT 6: 172; MT 2:
                // 220, MT 7 with two quads: 155)
                constexpr int J = MT_ == 6 ? 1 : MT_ == 7 ? 2 : 4;
                const int half = M * 128;
                const int bi0 = s_list[r0], bi1 = s_list[r0 + (rb == 2 ? 1 : 0)];
                const uint32_t cs4 = (uint32_t) gg.max_seg * (uint32_t) M * 512u;   // bytes between slots
                const uint32_t f00 = (uint32_t) ((s_own[0][bi0] * gg.max_seg + s_own[2][bi0]) * M) * 512u;
                const uint32_t f01 = (uint32_t) (s_own[0][bi0] + 1) * cs4;
                const uint32_t f10 = (uint32_t) ((s_own[0][bi1] * gg.max_seg + s_own[2][bi1]) * M) * 512u;
                const uint32_t f11 = (uint32_t) (s_own[0][bi1] + 1) * cs4;
                const int nc0 = s_own[1][bi0], nc1 = rb == 2 ? s_own[1][bi1] : 0;
                const int ncmax = nc0 > nc1 ? nc0 : nc1;
                const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(part_grp), 0, 0x7FFFFFFF,
                                                                                     RAW_BUFFER_FLAGS);
                for (int e0 = 4 * (int) threadIdx.x; e0 < total; e0 += 1024 * J) {
                    f32x4 sum[J];
#pragma unroll
                    for (int j = 0; j < J; ++j) sum[j] = f32x4{0.f, 0.f, 0.f, 0.f};
                    for (int c0 = 0; c0 < ncmax; c0 += 8) {
                        f32x4 v[J][8];
#pragma unroll
                        for (int j = 0; j < J; ++j) {
                            const int e = e0 + 1024 * j;
                            const bool second = e >= half;
                            const int el = second ? e - half : e;
                            const int nc = e < total ? (second ? nc1 : nc0) : 0;
#pragma unroll
                            for (int cc = 0; cc < 8; ++cc) {
                                const int c = c0 + cc;
                                const uint32_t off = (c == 0 ? (second ? f10 : f00) : (second ? f11 : f01) + (uint32_t) (c - 1) * cs4) +
                                                     (uint32_t) el * 4u;
                                v[j][cc] = c < nc ? __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, off, 0, SC1))
                                                  : f32x4{0.f, 0.f, 0.f, 0.f};
                            }
                        }
#pragma unroll
                        for (int j = 0; j < J; ++j) {
                            const int e = e0 + 1024 * j;
                            const int nc = e < total ? (e >= half ? nc1 : nc0) : 0;
#pragma unroll
                            for (int cc = 0; cc < 8; ++cc)
                                if (c0 + cc < nc) sum[j] += v[j][cc];
                        }
                    }
#pragma unroll
                    for (int j = 0; j < J; ++j) {
                        const int e = e0 + 1024 * j;
                        if (e < total) {
                            // the 4 elements share a row (rows are 128 wide): one 8-byte LDS store
                            const uint32_t lo = f16_bits((f16) sum[j][0]) | (f16_bits((f16) sum[j][1]) << 16);
                            const uint32_t hi = f16_bits((f16) sum[j][2]) | (f16_bits((f16) sum[j][3]) << 16);
                            *reinterpret_cast<u32x2*>(&lds_c[(e >> 7) * A_ROW + (e & 127)]) = u32x2{lo, hi};
                        }
                    }
                }
            } else if constexpr (!GATED) {
                for (int e = threadIdx.x; e < total; e += 256) {
                    const int r = e / (M * 128), el = e - r * (M * 128);
                    const int bi = s_list[r0 + r];
                    const int wf = s_own[0][bi], nc = s_own[1][bi], seg_f = s_own[2][bi];
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
                    if constexpr (FORM == FORM_F32OUT)
                        reinterpret_cast<float*>(lds_c)[r * 128 + el] = sum;          // single row: el < 128
                    else
                        lds_c[(r * M + (el >> 7)) * A_ROW + (el & 127)] = f16_bits((f16) sum);
                }
            } else {
                for (int e0 = threadIdx.x; e0 < total; e0 += 512) {
                    const bool has_b = e0 + 256 < total;
                    const float *pa0, *pa1, *pb0 = nullptr, *pb1 = nullptr;
                    int64_t csa, csb = 0;
                    int na, nb = 0, la, lb = 0;
                    elem(e0, pa0, pa1, csa, na, la);
                    if (has_b) elem(e0 + 256, pb0, pb1, csb, nb, lb);
                    float sa = 0.f, sb = 0.f;
                    const int nmax = na > nb ? na : nb;
                    for (int cc0 = 0; cc0 < nmax; cc0 += RED_BATCH) {
                        float va[RED_BATCH], vb[RED_BATCH];
#pragma unroll
                        for (int ii = 0; ii < RED_BATCH; ++ii) {
                            const int c = cc0 + ii;
                            va[ii] = c < na ? part_load(pa0, pa1, csa, c) : 0.f;
                            vb[ii] = c < nb ? part_load(pb0, pb1, csb, c) : 0.f;
                        }
#pragma unroll
                        for (int ii = 0; ii < RED_BATCH; ++ii) {
                            if (cc0 + ii < na) sa += va[ii];
                            if (cc0 + ii < nb) sb += vb[ii];
                        }
                    }
                    lds_c[la] = f16_bits((f16) sa);
                    if (has_b) lds_c[lb] = f16_bits((f16) sb);
                }
            }
            EXL3_TL(TL_SUMMED);
            if ((int) threadIdx.x < rb)                        // ready for the next call (stream order)
                __hip_atomic_store(&counters[(seg0_cb + b0 + s_list[r0 + threadIdx.x]) * CNT_STRIDE], 0u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            if (gated && MT_ == 0) {
                // single row: pair r on wave r, two columns a lane (gate and up transforms
                // interleave), SiLU-and-mul into g[0].y
                if (wave < rb) {
                    const int cb = seg0_cb + b0 + s_list[r0 + wave];
                    const uint32_t cg = *reinterpret_cast<const uint32_t*>(lds_c + (wave * RM) * A_ROW + 2 * lane);
                    const uint32_t cu = *reinterpret_cast<const uint32_t*>(lds_c + (wave * RM + 1) * A_ROW + 2 * lane);
                    const uint32_t rg = had128_x2<double>(cg, 0u, false, sv_first.x, true, r_scale<double>());
                    const uint32_t ru = had128_x2<double>(cu, 0u, false, sv_first_u.x, true, r_scale<double>());
                    __builtin_amdgcn_raw_buffer_store_b32(silu_mul_x2(rg, ru), y0src, (uint32_t) ((cb * 128 + 2 * lane) * 2), 0,
                                                          SC1);
                }
                __syncthreads();
                continue;
            }
            if (gated) {
                // gate and up rows m of pair r: output Hadamard + svh each, then SiLU-and-mul
                // into g[0].y
                for (int rr0 = 0; rr0 < rb * M; rr0 += 16) {
                    const int rr = rr0 + (threadIdx.x >> 4);
                    const bool live = rr < rb * M;
                    const int r = live ? rr / M : 0, m = live ? rr - r * M : 0;
                    const int cb = seg0_cb + b0 + s_list[r0 + r];
                    u32x4 cg = {0u, 0u, 0u, 0u}, cu = cg, svg = cg, svu = cg;
                    if (live) {
                        cg = *reinterpret_cast<const u32x4*>(lds_c + (r * RM + m) * A_ROW + 8 * l16);
                        cu = *reinterpret_cast<const u32x4*>(lds_c + (r * RM + M + m) * A_ROW + 8 * l16);
                        svg = rr0 == 0 ? sv_first : sv128(sc1_rsrc(a.g[0].svh), cb * 128 + 8 * l16);
                        svu = rr0 == 0 ? sv_first_u : sv128(sc1_rsrc(a.g[1].svh), cb * 128 + 8 * l16);
                    }
                    const u32x4 rg = had128_x8<double>(cg, u32x4{0u, 0u, 0u, 0u}, false, svg, true, r_scale<double>());
                    const u32x4 ru = had128_x8<double>(cu, u32x4{0u, 0u, 0u, 0u}, false, svu, true, r_scale<double>());
                    if (live)
                        __builtin_amdgcn_raw_buffer_store_b128(silu_mul_x8(rg, ru), y0src,
                                                               (uint32_t) (((int64_t) m * a.ldy + cb * 128 + 8 * l16) * 2), 0, SC1);
                }
                __syncthreads();
                continue;
            }
            if constexpr (MT_ == 0 && FORM == FORM_F32OUT) {
                // fp32 output: the block's fp32 C, float64 butterflies, (float) (v r) * svh
                if (wave < rb) {
                    const int cb = seg0_cb + b0 + s_list[r0 + wave];
                    const float* cf = reinterpret_cast<const float*>(lds_c) + wave * 128 + 2 * lane;
                    float o0, o1;
                    had128_x2_f32(cf[0], cf[1], sv_first.x, r_scale<double>(), o0, o1);
                    __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(o0), __float_as_uint(o1)}, ysrc,
                                                          (uint32_t) ((cb * 128 + 2 * lane) * 4), 0, SC1);
                }
                __syncthreads();                               // lds_c free for the next blocks
                continue;
            } else if constexpr (MT_ == 0) {
                // output Hadamard + svh of a single row: one wave per block, two columns a lane
                if (wave < rb) {
                    const int cb = seg0_cb + b0 + s_list[r0 + wave];
                    const uint32_t c = *reinterpret_cast<const uint32_t*>(lds_c + wave * A_ROW + 2 * lane);
                    __builtin_amdgcn_raw_buffer_store_b32(had128_x2<double>(c, 0u, false, sv_first.x, true, r_scale<double>()), ysrc,
                                                          (uint32_t) ((cb * 128 + 2 * lane) * 2), 0, SC1);
                }
                __syncthreads();                               // lds_c free for the next blocks
                continue;
            }
            // output Hadamard + svh: 16 lanes per (block, row)
            for (int rr0 = 0; rr0 < rb * M; rr0 += 16) {
                const int rr = rr0 + (threadIdx.x >> 4);
                const bool live = rr < rb * M;
                const int r = live ? rr / M : 0, m = live ? rr - r * M : 0;
                const int cb = seg0_cb + b0 + s_list[r0 + r];
                u32x4 c = {0u, 0u, 0u, 0u}, sv = c;
                if (live) {
                    c = *reinterpret_cast<const u32x4*>(lds_c + rr * A_ROW + 8 * l16);
                    sv = rr0 == 0 ? sv_first : sv128(svsrc, cb * 128 + 8 * l16);
                }
                const u32x4 res = had128_x8<double>(c, u32x4{0u, 0u, 0u, 0u}, false, sv, true, r_scale<double>());
                if (live)
                    __builtin_amdgcn_raw_buffer_store_b128(res, ysrc, (uint32_t) (((int64_t) m * a.ldy + cb * 128 + 8 * l16) * 2), 0, SC1);
            }
            __syncthreads();                                   // lds_c free for the next blocks
        }
    }
    EXL3_TL(TL_END);
}

// LDS: chunk_units x (m + 1) input rows, then the C rows of the blocks reduced side by side (the
// fp32-output form: two fp32 rows of 128, the room of four fp16 rows)
inline size_t lds_bytes(int M, int cu, bool gated, bool f32out = false, bool pair16 = false)
{
    // blocks (gated: pairs) reduced side by side x rows: as RB in the kernel
    const int c_rows = gated || f32out ? (M == 1 ? 4 : 2 * M) : (M <= (pair16 ? 16 : 8) ? 2 * M : M);
    return ((size_t) cu * (M + 1) + c_rows) * A_ROW * 2;
}

template <int BITS, int CB, int MT_, int FORM>
int launch_gemv_t(const GemvArgs& a, int wgs, hipStream_t stream)
{
    hipLaunchKernelGGL((gemv_kernel<BITS, CB, MT_, FORM>), dim3(wgs), dim3(256),
                       lds_bytes(a.M, a.chunk_units, FORM == FORM_GATED, FORM == FORM_F32OUT, MT_ >= 5), stream, a);
    return hipGetLastError() == hipSuccess ? EXL3_OK : EXL3_ELAUNCH;
}

// 16-row MFMA tiles of the rows: one exact row, <= 16, <= 32, and for the plain faithful forms (the
// only ones the host lets past EXL3_GEMV_FUSED_MAX_ROWS) <= 48 and <= 64.  Up to 16 rows the plain
// and SiLU-input forms take a one-tile instantiation with the 16-byte-load reduction: MT 6 (one
// quad in flight, 172 VGPRs) when the workgroups stage their input in one LDS chunk, up to 8 rows
// on a grid of two workgroups per CU and up to 16 on a smaller one; else MT 5 (four quads, 220
// VGPRs) from 5 rows on the full grid and from 9 on a smaller one.  Against the 4-byte-load MT 1:
// MT 6 0.5-2.7 us faster at 2-8 rows on every shape measured (o at 4 rows 14.1 -> 12.1 us, q/k/v at
// 2 rows 16.0 -> 13.7), ~1 us at 9-16 rows on the 320-workgroup k/v pair; MT 5 up to 1.2 us faster
// than MT 6 at 9-16 rows on full grids.  With two LDS chunks (gate/up at 8 rows: 27 units per
// workgroup, 24 fit) the 172-VGPR forms lose 4 us to the chunk reload and MT 5 keeps them.
template <int BITS, int CB, int FORM>
int launch_gemv_m(const GemvArgs& a, int wgs, hipStream_t s)
{
    if (a.M == 1) return launch_gemv_t<BITS, CB, 0, FORM>(a, wgs, s);
    if constexpr ((FORM == FORM_PLAIN || FORM == FORM_SILU_IN) && CB <= 2) {
        const bool full = wgs >= 256 * WAVES_PER_SIMD;
        if (a.M <= (full ? 8 : 16) && a.chunk_units >= a.max_per) return launch_gemv_t<BITS, CB, 6, FORM>(a, wgs, s);
        if (a.M >= (full ? 5 : 9) && a.M <= 16) return launch_gemv_t<BITS, CB, 5, FORM>(a, wgs, s);
    }
    if (a.M <= 16) return launch_gemv_t<BITS, CB, 1, FORM>(a, wgs, s);
    if constexpr (FORM == FORM_PLAIN && CB <= 2) {
        if (a.M > 48) return launch_gemv_t<BITS, CB, 4, FORM>(a, wgs, s);
        if (a.M > 32) return launch_gemv_t<BITS, CB, 3, FORM>(a, wgs, s);
        // 17-32 rows: two quads of partial loads in flight (MT 7, 155 VGPRs against MT 2's 220)
        // when every block has at most 8 contributors (one batch of loads per pass: the second
        // pass is one round trip); with more, the extra pass costs more than the registers save
        // (A/B in one call: gate/up, ~3 contributors, 1.4-2.3 us faster at 17-32 rows, gate, ~5,
        // up to 1 us; down, q/k/v and the k/v pair, 10-21, up to 1.7 us slower)
        int wpb = 0;
        for (int i = 0; i < a.groups; ++i) {
            const int w = (a.g[i].G * 128 + a.g[i].n - 1) / a.g[i].n;     // workgroups per block
            wpb = w > wpb ? w : wpb;
        }
        if (wpb + 1 <= 8) return launch_gemv_t<BITS, CB, 7, FORM>(a, wgs, s);
    }
    return launch_gemv_t<BITS, CB, 2, FORM>(a, wgs, s);
}

template <int BITS, int FORM>
int launch_gemv_cb(const GemvArgs& a, int cb, int wgs, hipStream_t s)
{
    switch (cb) {
        case 0: return launch_gemv_m<BITS, 0, FORM>(a, wgs, s);
        case 1: return launch_gemv_m<BITS, 1, FORM>(a, wgs, s);
        default: return launch_gemv_m<BITS, 2, FORM>(a, wgs, s);
    }
}

// the kernel instantiation for (bits, codebook, rows) of one form
template <int FORM>
int launch_gemv_impl(const GemvArgs& a, int bits, int cb, int wgs, hipStream_t s)
{
    switch (bits) {
        case 1: return launch_gemv_cb<1, FORM>(a, cb, wgs, s);
        case 2: return launch_gemv_cb<2, FORM>(a, cb, wgs, s);
        case 3: return launch_gemv_cb<3, FORM>(a, cb, wgs, s);
        case 4: return launch_gemv_cb<4, FORM>(a, cb, wgs, s);
        case 5: return launch_gemv_cb<5, FORM>(a, cb, wgs, s);
        case 6: return launch_gemv_cb<6, FORM>(a, cb, wgs, s);
        case 7: return launch_gemv_cb<7, FORM>(a, cb, wgs, s);
        default: return launch_gemv_cb<8, FORM>(a, cb, wgs, s);
    }
}

// gated instantiations live in exl3_gemv_gated.hip, SiLU-input ones in exl3_gemv_silu.hip
int launch_gemv_gated(const GemvArgs& a, int bits, int cb, int wgs, hipStream_t s);
int launch_gemv_silu_in(const GemvArgs& a, int bits, int cb, int wgs, hipStream_t s);
// the fp32-output single-row instantiations live in exl3_gemv_f32.hip
int launch_gemv_f32out(const GemvArgs& a, int bits, int cb, int wgs, hipStream_t s);
// approximate mul1 instantiations (codebook ids 3 and 4) live in exl3_gemv_approx.hip
int launch_gemv_approx(const GemvArgs& a, int bits, int cb, int wgs, hipStream_t s);
