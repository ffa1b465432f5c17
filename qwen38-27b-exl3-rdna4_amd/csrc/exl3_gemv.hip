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
#include "exl3_gemv_kernel.h"

#include <stdio.h>
#include <stdlib.h>
#include <algorithm>

using namespace exl3;


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
// had_r_128: out = fp16(Had128(in [* pre]) * r * scale) [* post]; one 8-lane group per 128-block,
// 8 blocks per wave (reference binding `had_r_128`, vllm_plugin/exl3rocm/ops.py:88,97)
// ============================================================================================

// The exact transform (exl3_had_r_128 and the GEMV's pre-rotation: the same values as the GEMV's
// in-kernel transforms), T = double butterflies; the float32 transform is had_mfma_kernel
// (exl3_had.hip).
// in_up (may be null): the input rows are fp16(fp16(silu(in)) * in_up) (a gated MLP's activation)
// Every group's output of a block comes from one read of the input block (a fused module's groups
// differ only in their pre-scale).
template <class T>
__global__ void __launch_bounds__(256) had_kernel(const uint16_t* __restrict__ in, const uint16_t* __restrict__ in_up,
                                                  int64_t ld_in, HadGroups hg, int groups, int64_t ld_out, int rows,
                                                  int cols, const uint16_t* __restrict__ post, T scale)
{
    const int blocks_per_row = cols / 128;
    const int64_t job = ((int64_t) blockIdx.x * 256 + threadIdx.x) >> 3;     // one 128-block per 8 lanes
    const bool live = job < (int64_t) rows * blocks_per_row;
    const int r = threadIdx.x & 7;
    const int64_t row = live ? job / blocks_per_row : 0;
    const int col = live ? (int) (job % blocks_per_row) * 128 + 16 * r : 0;
    u32x4 v[2], qv[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) v[c] = qv[c] = u32x4{0u, 0u, 0u, 0u};
    if (live) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            v[c] = *reinterpret_cast<const u32x4*>(in + row * ld_in + col + 8 * c);
            if (in_up) v[c] = silu_mul_x8(v[c], *reinterpret_cast<const u32x4*>(in_up + row * ld_in + col + 8 * c));
            if (post) qv[c] = *reinterpret_cast<const u32x4*>(post + col + 8 * c);
        }
    }
    for (int g = 0; g < groups; ++g) {
        // constant indices into the argument struct (a runtime index would copy it to scratch)
        const uint16_t* pre = g == 0 ? hg.pre[0] : g == 1 ? hg.pre[1] : g == 2 ? hg.pre[2] : hg.pre[3];
        uint16_t* out = g == 0 ? hg.out[0] : g == 1 ? hg.out[1] : g == 2 ? hg.out[2] : hg.out[3];
        u32x4 pv[2] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};
        if (live && pre) {
#pragma unroll
            for (int c = 0; c < 2; ++c) pv[c] = *reinterpret_cast<const u32x4*>(pre + col + 8 * c);
        }
        // every lane takes part in the DPP exchanges; only live lanes store
        u32x4 res[2];
        had128_x16<T>(v, pv, pre != nullptr, qv, post != nullptr, scale, res);
        if (live) {
#pragma unroll
            for (int c = 0; c < 2; ++c) *reinterpret_cast<u32x4*>(out + row * ld_out + col + 8 * c) = res[c];
        }
    }
}

// The same exact transform with one 128-block per wave, two elements a lane (had128_x2): the
// latency form, for launches of at most EXL3_GEMV_MAX_ROWS rows (the GEMV's pre-rotation pass).
// There had_kernel's grid of one 8-lane group per block leaves most CUs idle (16 rows x 40
// blocks: 20 workgroups) and each lane's 16-element butterflies are the critical path.  The
// same values bit for bit: both sum exactly in float64 and round once (scaled_f16), with the
// same fp16 products for pre, post and the SiLU input.  A wave reads its whole block before any
// lane writes, so in == out is safe.
template <class T>
__global__ void __launch_bounds__(256) had_kernel_x2(const uint16_t* __restrict__ in, const uint16_t* __restrict__ in_up,
                                                     int64_t ld_in, HadGroups hg, int groups, int64_t ld_out, int rows,
                                                     int cols, const uint16_t* __restrict__ post, T scale)
{
    const int blocks_per_row = cols / 128;
    const int64_t job = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);       // one 128-block per wave
    if (job >= (int64_t) rows * blocks_per_row) return;                      // whole waves leave together
    const int lane = threadIdx.x & 63;
    const int64_t row = job / blocks_per_row;
    const int col = (int) (job % blocks_per_row) * 128 + 2 * lane;
    uint32_t v = *reinterpret_cast<const uint32_t*>(in + row * ld_in + col);
    if (in_up) v = silu_mul_x2(v, *reinterpret_cast<const uint32_t*>(in_up + row * ld_in + col));
    const uint32_t q = post ? *reinterpret_cast<const uint32_t*>(post + col) : 0u;
    for (int g = 0; g < groups; ++g) {
        // constant indices into the argument struct (a runtime index would copy it to scratch)
        const uint16_t* pre = g == 0 ? hg.pre[0] : g == 1 ? hg.pre[1] : g == 2 ? hg.pre[2] : hg.pre[3];
        uint16_t* out = g == 0 ? hg.out[0] : g == 1 ? hg.out[1] : g == 2 ? hg.out[2] : hg.out[3];
        const uint32_t p = pre ? *reinterpret_cast<const uint32_t*>(pre + col) : 0u;
        *reinterpret_cast<uint32_t*>(out + row * ld_out + col) = had128_x2<T>(v, p, pre != nullptr, q, post != nullptr, scale);
    }
}

// the float transform's launch (exl3_had.hip)
void launch_had_mfma(const uint16_t* in, const uint16_t* up, int64_t ld_in, const HadGroups& hg, int groups,
                     int64_t ld_out, int rows, int cols, const uint16_t* post, float scale, bool has_pre, hipStream_t s);

// had_r_128 of one input into `groups` outputs, group i scaled by pre[i] (may be null; the float32
// form takes a pre for every group or for none): one launch (the prefill's input transforms of a
// fused module); exact: float64 butterflies, else float32 sums on the matrix cores (the prefill's
// input transforms and epilogue values)
int launch_had(const void* in, int64_t ld_in, void* const* out, int64_t ld_out, int rows, int cols, const void* const* pre,
               int groups, const void* post, float scale, void* stream, bool exact, const void* in_up)
{
    if (((uintptr_t) in_up) & 15) return EXL3_EINVAL;
    if (!in || !out || rows < 0 || cols % 128 || cols < 128 || ld_in < cols || ld_out < cols || ld_in % 8 || ld_out % 8 ||
        groups < 1 || groups > EXL3_MAX_GROUPS || (((uintptr_t) in) & 15) || (((uintptr_t) post) & 15))
        return EXL3_EINVAL;
    HadGroups hg{};
    for (int i = 0; i < groups; ++i) {
        const void* p = pre ? pre[i] : nullptr;
        if (!out[i] || (((uintptr_t) out[i]) & 15) || (((uintptr_t) p) & 15)) return EXL3_EINVAL;
        hg.pre[i] = (const uint16_t*) p;
        hg.out[i] = (uint16_t*) out[i];
    }
    if (rows == 0) return EXL3_OK;
    const int64_t jobs = (int64_t) rows * (cols / 128);           // 8 lanes each
    const dim3 grid((unsigned) ((jobs + 31) / 32));
    if (!exact) {
        const int64_t waves = ((int64_t) rows + 15) / 16 * (cols / 128);
        if (waves >= (1ll << 31)) return EXL3_EINVAL;
        const float sc = (float) (R_SCALE * (double) scale);
        int n_pre = 0;
        for (int i = 0; i < groups; ++i) n_pre += hg.pre[i] != nullptr;
        if (n_pre != 0 && n_pre != groups) return EXL3_EINVAL;      // pre for every group or for none
        launch_had_mfma((const uint16_t*) in, (const uint16_t*) in_up, ld_in, hg, groups, ld_out, rows, cols,
                        (const uint16_t*) post, sc, n_pre != 0, (hipStream_t) stream);
    } else if (rows <= EXL3_GEMV_MAX_ROWS) {
        // the latency form: one block per wave, four waves a workgroup
        hipLaunchKernelGGL(had_kernel_x2<double>, dim3((unsigned) ((jobs + 3) / 4)), dim3(256), 0, (hipStream_t) stream,
                           (const uint16_t*) in, (const uint16_t*) in_up, ld_in, hg, groups, ld_out, rows, cols,
                           (const uint16_t*) post, R_SCALE * (double) scale);
    } else {
        hipLaunchKernelGGL(had_kernel<double>, grid, dim3(256), 0, (hipStream_t) stream, (const uint16_t*) in,
                           (const uint16_t*) in_up, ld_in, hg, groups, ld_out, rows, cols, (const uint16_t*) post,
                           R_SCALE * (double) scale);
    }
    return hipGetLastError() == hipSuccess ? EXL3_OK : EXL3_ELAUNCH;
}

// SiLU-and-mul of fp16 rows: out[r][c] = fp16(fp16(silu(gate[r][c])) * up[r][c]), 8 columns a thread
__global__ void __launch_bounds__(256) silu_mul_kernel(const uint16_t* __restrict__ gate, const uint16_t* __restrict__ up,
                                                       int64_t ld_in, uint16_t* __restrict__ out, int64_t ld_out,
                                                       int rows, int n8)
{
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t) rows * n8) return;
    const int64_t r = i / n8;
    const int64_t c = (i - r * n8) * 8;
    const u32x4 g = *reinterpret_cast<gc_u32x4*>(as_global(gate) + r * ld_in + c);
    const u32x4 u = *reinterpret_cast<gc_u32x4*>(as_global(up) + r * ld_in + c);
    *reinterpret_cast<g_u32x4*>(as_global(out) + r * ld_out + c) = silu_mul_x8(g, u);
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
    int G[EXL3_MAX_GROUPS], o0[EXL3_MAX_GROUPS], nold[EXL3_MAX_GROUPS], y0[EXL3_MAX_GROUPS];
    int max_seg[EXL3_MAX_GROUPS], cnt_off[EXL3_MAX_GROUPS], first;
    int64_t slot_off[EXL3_MAX_GROUPS];   // first partial slot (one slot = m * 128 floats)
    int total_wgs, counters;
    int64_t slots;
    int max_per;                         // most units any workgroup owns
    int h[EXL3_MAX_GROUPS], wa, wb;      // unit-split weights (Split)
    Split split[EXL3_MAX_GROUPS];
};

// Unit-split weights of first-dispatched / second workgroups on a CU: the second runs its loop at
// the higher wave priority and takes the larger share (EXL3_GEMV_WEIGHTS="a,b" overrides, for
// measurement)
void split_weights(int& wa, int& wb)
{
    wa = 2;
    wb = 3;
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
    // at most ~max_contrib workgroups sharing one block (EXL3_GEMV_MAX_CONTRIB below 1: the default)
    const int mc = env_int("EXL3_GEMV_MAX_CONTRIB", 32);
    const int max_contrib = mc >= 1 ? mc : 32;
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
    // grid slots [0, NUM_CUS) are the first workgroups on their CU (with at most one per CU all
    // are, and the split is uniform); each group gets a share of them in proportion to its size
    const int first = gsum > NUM_CUS ? NUM_CUS : gsum;
    p.first = first;
    int given = 0;
    for (int i = 0; i < groups; ++i) {
        p.nold[i] = (int) ((int64_t) first * Gs[i] / gsum);
        given += p.nold[i];
    }
    for (int i = 0; i < groups && given < first; ++i)
        if (p.nold[i] < Gs[i]) {
            ++p.nold[i];
            ++given;
        }
    int cnt = 0, o = 0, y = first;
    int64_t slots = 0;
    for (int i = 0; i < groups; ++i) {
        const int Ui = (widths[i] / 128) * UPB;
        p.G[i] = Gs[i];
        p.o0[i] = o;
        p.y0[i] = y;
        o += p.nold[i];
        y += Gs[i] - p.nold[i];
        // weighted only where every workgroup still gets a unit (U * min(wa, wb) >= max(wa, wb) * G;
        // the completion count assumes each workgroup between a block's first and last owner
        // contributes to it)
        const bool weighted = (int64_t) Ui * std::min(p.wa, p.wb) >= (int64_t) std::max(p.wa, p.wb) * Gs[i];
        p.h[i] = weighted ? p.nold[i] : Gs[i];
        const Split sp = Split::make(Ui, Gs[i], p.h[i], p.wa, p.wb);
        p.split[i] = sp;
        const int per = sp.max_units();
        p.max_seg[i] = (per + UPB - 1) / UPB + 1;
        p.cnt_off[i] = cnt;
        p.slot_off[i] = slots;
        p.max_per = std::max(p.max_per, per);
        cnt += widths[i] / 128;
        slots += (int64_t) p.G[i] * p.max_seg[i];
    }
    p.total_wgs = gsum;
    p.counters = cnt;
    p.slots = slots;
    return p;
}

// units whose rotated input a workgroup stages at once (all of them when they fit); a chunk that
// is not the last one holds whole ring turns (RING / 2 units)
int chunk_units(int m, int max_per)
{
    // the C rows of the output transform: at most max(2m, 4) (gated pairs side by side at m == 1)
    const int c_rows = std::max(2 * m, 4);
    const int64_t fit = std::max<int64_t>(RING / 2, ((LDS_BUDGET / (2 * A_ROW) - c_rows) / (m + 1)) / (RING / 2) * (RING / 2));
    return (int) std::max<int64_t>(1, std::min<int64_t>(max_per, fit));
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
// The input is rotated either by every workgroup for its own k-range, in LDS (work ~ rows x the
// units a workgroup owns), or once per group by a separate pass into the caller's A_had scratch
// (a launch and one rotated copy per group: a fixed cost that grows with the groups).  The pass
// pays from rows x max_per >= unit_rows x (groups + 1): unit_rows falls as the workgroups own more
// units (60 below PREROT_SMALL_PER units, 42 up to PREROT_LARGE_PER, 36 from there; launches of a
// few units per workgroup measured their in-LDS rotation cheaper per row-unit).  Measured crossovers with the
// one-block-per-wave pass (rows where the pass first wins, max_per): gate 6 (14), down 5-6 (14),
// gate/up 4 (27), 6144 x 5120 14 (6), the 3-group q/k/v 24 (7); o 24 (5), the 2-group 1024-wide
// k/v pair 40 (4).  Outputs are bitwise the same either way.  EXL3_GEMV_PREROT_M, when set, fixes
// one row count for every shape.
constexpr int PREROT_SMALL_PER = 6;
constexpr int PREROT_LARGE_PER = 20;

int prerot_override()
{
    static const int v = env_int("EXL3_GEMV_PREROT_M", 0);
    return v;
}

bool prerot(int m, int max_per, int groups)
{
    const int o = prerot_override();
    if (o > 0) return m >= o;
    const int unit_rows = max_per >= PREROT_LARGE_PER ? 36 : max_per >= PREROT_SMALL_PER ? 42 : 60;
    return m > 1 && (int64_t) m * max_per >= (int64_t) unit_rows * (groups + 1);
}

// the fewest rows at which any shape may be pre-rotated: callers pass A_had from there on
int prerot_rows()
{
    const int o = prerot_override();
    return o > 0 ? o : 2;
}

// The same for a SiLU input (EXL3_GEMV_SILU_PREROT_M overrides): there the pass takes the place
// of the activation kernel the caller would otherwise run, while rotating in LDS repeats the SiLU
// in every workgroup sharing a k-range (config-1 down projection, MLP time against the
// two-launch form: in LDS -2.4% at 2 rows, +0.8% at 4, +2.5% at 8; the pass +0.8% at 4, -2.2% at 8).
int silu_prerot_rows()
{
    static const int v = env_int("EXL3_GEMV_SILU_PREROT_M", 4);
    return v;
}

// xr: the caller's scratch of groups * m * k fp16 for pre-rotated input (may be null)
int gemv_common(const void* x, int64_t ldx, const GemvGroup* gs, const int* widths, int groups,
                const int64_t* const* tabs, int64_t ldy, int m, int k, int K, int mcg, int mul1, void* ws,
                size_t ws_bytes, void* stream, bool gated = false, void* xr = nullptr, int approx = 0,
                const void* x_up = nullptr, bool f32out = false)
{
    if (f32out && (m != 1 || gated || tabs || approx || x_up)) return EXL3_EINVAL;
    // the fused-epilogue forms take up to EXL3_GEMV_FUSED_MAX_ROWS rows (16-row tiles 1 and 2 only)
    if ((gated || x_up || approx) && m > EXL3_GEMV_FUSED_MAX_ROWS) return EXL3_DECLINED;
    if (x_up && (gated || tabs || approx || (((uintptr_t) x_up) & 15))) return EXL3_EINVAL;
    if (approx && (gated || approx > 2)) return EXL3_EINVAL;
    if (gated && (groups != 2 || tabs || widths[0] != widths[1] || ldy < widths[0])) return EXL3_EINVAL;
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
    if (ldy < widths[0] || (m > 1 && !gated && ldy < total)) return EXL3_EINVAL;
    for (int i = 0; i < groups; ++i) {
        if (!shape_ok(m, k, widths[i], K)) return EXL3_DECLINED;
        if ((uint64_t) k * widths[i] * K / 8 > 0xFFFFFFFFull) return EXL3_DECLINED;   // one raw buffer per trellis
    }
    const GridPlan p = plan_grid(k, widths, groups);
    if ((size_t) p.counters * 4 * CNT_STRIDE > COUNTER_BYTES) return EXL3_DECLINED;
    for (int i = 0; i < groups; ++i)
        if (!p.split[i].fits32()) return EXL3_DECLINED;   // unreachable below the 4 GiB trellis limit
    if (!ws || ws_bytes < COUNTER_BYTES + (size_t) p.slots * m * 128 * 4) return EXL3_EWORKSPACE;
    GemvArgs a{};
    a.x = (const uint16_t*) x;
    a.ldx = ldx;
    a.x_up = (const uint16_t*) x_up;
    if (xr && !tabs && m > 1 && (x_up ? m >= silu_prerot_rows() : prerot(m, p.max_per, groups))) {
        if (((uintptr_t) xr) & 15) return EXL3_EINVAL;
        // every group's rotated rows in one launch
        void* outs[EXL3_MAX_GROUPS];
        const void* pres[EXL3_MAX_GROUPS];
        for (int i = 0; i < groups; ++i) {
            outs[i] = (uint16_t*) xr + (int64_t) i * m * k;
            pres[i] = gs[i].suh;
        }
        const int rc = launch_had(x, ldx, outs, k, m, k, pres, groups, nullptr, 1.0f, stream, true, x_up);
        if (rc != EXL3_OK) return rc;
        a.xr = (const uint16_t*) xr;
        a.x_up = nullptr;                       // the activation is in the pre-rotated rows
    }
    for (int i = 0; i < groups; ++i) {
        a.g[i] = gs[i];
        a.g[i].n = widths[i];
        a.g[i].G = p.G[i];
        a.g[i].o0 = p.o0[i];
        a.g[i].nold = p.nold[i];
        a.g[i].y0 = p.y0[i];
        a.slot_o[i] = p.o0[i];
        a.slot_y[i] = p.y0[i];
        a.g[i].max_seg = p.max_seg[i];
        a.g[i].part_off = p.slot_off[i] * m * 128;
        a.g[i].cnt_off = p.cnt_off[i];
        a.g[i].h = p.h[i];
        a.g[i].d_sg = p.split[i].d_sg;
        a.g[i].d_u = p.split[i].d_u;
    }
    a.first = p.first;
    a.wa = p.wa;
    a.wb = p.wb;
    a.d_wa = UDiv::of((uint32_t) p.wa);
    a.d_wb = UDiv::of((uint32_t) p.wb);
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
    a.max_per = p.max_per;
    a.ldy = ldy;
    a.counters = (uint32_t*) ws;
    a.part = (float*) ((char*) ws + COUNTER_BYTES);
    if (f32out) return launch_gemv_f32out(a, K, codebook_of(mcg, mul1), p.total_wgs, (hipStream_t) stream);
    if (approx) return launch_gemv_approx(a, K, 2 + approx, p.total_wgs, (hipStream_t) stream);
    if (a.x_up) return launch_gemv_silu_in(a, K, codebook_of(mcg, mul1), p.total_wgs, (hipStream_t) stream);
    return gated ? launch_gemv_gated(a, K, codebook_of(mcg, mul1), p.total_wgs, (hipStream_t) stream)
                 : launch_gemv_impl<FORM_PLAIN>(a, K, codebook_of(mcg, mul1), p.total_wgs, (hipStream_t) stream);
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

int exl3_gemv_prerot_rows(void) { return prerot_rows(); }

int exl3_gemv_silu_prerot_rows(void) { return silu_prerot_rows(); }

#ifdef EXL3_TIMELINE
// Tracing build only (include/exl3_mi355x_timeline.h): the GEMV's per-workgroup phase stamps.
int exl3_timeline_shape(int* max_wgs, int* phases)
{
    if (max_wgs) *max_wgs = TL_MAX_WGS;
    if (phases) *phases = TL_PHASES;
    return EXL3_OK;
}

int exl3_timeline_clear(void)
{
    static const unsigned long long zeros[TL_MAX_WGS * TL_PHASES] = {};
    return hipMemcpyToSymbol(HIP_SYMBOL(exl3_tl), zeros, sizeof(zeros)) == hipSuccess ? EXL3_OK : EXL3_ELAUNCH;
}

int exl3_timeline_read(void* host, size_t bytes)
{
    if (!host || bytes > sizeof(unsigned long long) * TL_MAX_WGS * TL_PHASES) return EXL3_EINVAL;
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(exl3_tl), bytes, 0, hipMemcpyDeviceToHost) == hipSuccess ? EXL3_OK
                                                                                                         : EXL3_ELAUNCH;
}
#endif

int exl3_gemv_split_check(int U, int G, int h, int wa, int wb)
{
    if (U < 1 || G < 1 || h < 0 || h > G || wa < 1 || wb < 1) return -1;
    const Split sp = Split::make(U, G, h, wa, wb);
    if (!sp.fits32()) return -1;
    // 64-bit restatement: lo(w) = floor(U S(w) / S(G)), owner(u) = the largest w < G with lo(w) <= u
    auto S64 = [&](int w) { return (int64_t) wa * std::min(w, h) + (int64_t) wb * std::max(w - h, 0); };
    auto lo64 = [&](int w) { return (int) ((int64_t) U * S64(w) / S64(G)); };
    int bad = 0;
    for (int w = 0; w <= G; ++w) bad += sp.lo(w) != lo64(w);
    int w = 0;
    for (int u = 0; u < U; ++u) {
        while (w + 1 < G && lo64(w + 1) <= u) ++w;
        bad += sp.owner(u) != w;
    }
    // the divider at the edges of its range for each divisor
    const UDiv ds[4] = {sp.d_sg, sp.d_u, sp.d_wa, sp.d_wb};
    const uint32_t dv[4] = {sp.S(G), (uint32_t) U, (uint32_t) wa, (uint32_t) wb};
    for (int i = 0; i < 4; ++i) {
        const uint32_t d = dv[i];
        const uint32_t ns[] = {0u, 1u, d - 1u, d, d + 1u, 2u * d - 1u, 2u * d, 0x7FFFFFFFu, 0x80000000u, 0xFFFFFFFEu, 0xFFFFFFFFu,
                               0xFFFFFFFFu / d * d, 0xFFFFFFFFu / d * d - 1u};
        for (uint32_t n : ns) bad += ds[i].div(n) != n / d;
    }
    return bad;
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

int exl3_gemv_f32(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh, void* A_had,
                  const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
                  void* stream)
{
    (void) A_had;
    if (!trellis || !y || !suh || !svh) return EXL3_EINVAL;
    if (m != 1) return EXL3_DECLINED;
    GemvGroup g{(const uint32_t*) trellis, (const uint16_t*) suh, (const uint16_t*) svh, (uint16_t*) y};
    return gemv_common(x, ldx, &g, &n, 1, nullptr, ldy, m, k, K, mcg, mul1, workspace, ws_bytes, stream, false, nullptr, 0,
                       nullptr, true);
}

int exl3_gemv_mr(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh, void* A_had,
                 const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
                 void* stream)
{
    if (!trellis || !y || !suh || !svh) return EXL3_EINVAL;
    GemvGroup g{(const uint32_t*) trellis, (const uint16_t*) suh, (const uint16_t*) svh, (uint16_t*) y};
    return gemv_common(x, ldx, &g, &n, 1, nullptr, ldy, m, k, K, mcg, mul1, workspace, ws_bytes, stream, false, A_had);
}

int exl3_gemv_mr_approx(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh,
                        void* A_had, const void* svh, int m, int k, int n, int K, int mode, void* workspace,
                        size_t ws_bytes, void* stream)
{
    if (!trellis || !y || !suh || !svh || mode < 1 || mode > 2) return EXL3_EINVAL;
    GemvGroup g{(const uint32_t*) trellis, (const uint16_t*) suh, (const uint16_t*) svh, (uint16_t*) y};
    return gemv_common(x, ldx, &g, &n, 1, nullptr, ldy, m, k, K, 0, 1, workspace, ws_bytes, stream, false, A_had, mode);
}

int exl3_gemv_silu_in(const void* gate, const void* up, int64_t ld_in, const void* trellis, void* y, int64_t ldy,
                      const void* suh, void* A_had, const void* svh, int m, int k, int n, int K, int mcg, int mul1,
                      void* workspace, size_t ws_bytes, void* stream)
{
    if (!gate || !up || !trellis || !y || !suh || !svh) return EXL3_EINVAL;
    GemvGroup g{(const uint32_t*) trellis, (const uint16_t*) suh, (const uint16_t*) svh, (uint16_t*) y};
    return gemv_common(gate, ld_in, &g, &n, 1, nullptr, ldy, m, k, K, mcg, mul1, workspace, ws_bytes, stream, false, A_had,
                       0, up);
}

int exl3_gemv_mr_grouped(const void* x, int64_t ldx, const void* const* trellis, void* y, int64_t ldy,
                         const void* const* suh, void* A_had, const void* const* svh, int groups, int m, int k, int n,
                         int K, int mcg, int mul1, int bszm_for_warps, void* workspace, size_t ws_bytes, void* stream)
{
    (void) bszm_for_warps;
    if (!trellis || !suh || !svh || !y || groups < 1 || groups > EXL3_MAX_GROUPS) return EXL3_EINVAL;
    GemvGroup gs[EXL3_MAX_GROUPS];
    int widths[EXL3_MAX_GROUPS];
    for (int i = 0; i < groups; ++i) {
        gs[i] = {(const uint32_t*) trellis[i], (const uint16_t*) suh[i], (const uint16_t*) svh[i],
                 (uint16_t*) y + (int64_t) i * n};
        widths[i] = n;
    }
    return gemv_common(x, ldx, gs, widths, groups, nullptr, ldy, m, k, K, mcg, mul1, workspace, ws_bytes, stream,
                       false, A_had);
}

int exl3_gemv_mr_grouped_widths(const void* x, int64_t ldx, const void* const* trellis, void* y, int64_t ldy,
                                const void* const* suh, void* A_had, const void* const* svh, const int* widths,
                                int groups, int m, int k, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
                                void* stream)
{
    if (!trellis || !suh || !svh || !y || !widths || groups < 1 || groups > EXL3_MAX_GROUPS) return EXL3_EINVAL;
    GemvGroup gs[EXL3_MAX_GROUPS];
    int64_t n0 = 0;
    for (int i = 0; i < groups; ++i) {
        gs[i] = {(const uint32_t*) trellis[i], (const uint16_t*) suh[i], (const uint16_t*) svh[i], (uint16_t*) y + n0};
        n0 += widths[i];
    }
    if (ldy < n0) return EXL3_EINVAL;
    return gemv_common(x, ldx, gs, widths, groups, nullptr, ldy, m, k, K, mcg, mul1, workspace, ws_bytes, stream,
                       false, A_had);
}

int exl3_gemv_silu_mul(const void* x, int64_t ldx, const void* const* trellis, void* y, int64_t ldy,
                       const void* const* suh, void* A_had, const void* const* svh, int m, int k, int n, int K, int mcg,
                       int mul1, void* workspace, size_t ws_bytes, void* stream)
{
    if (!trellis || !suh || !svh || !y) return EXL3_EINVAL;
    GemvGroup gs[2];
    const int widths[2] = {n, n};
    for (int i = 0; i < 2; ++i)
        gs[i] = {(const uint32_t*) trellis[i], (const uint16_t*) suh[i], (const uint16_t*) svh[i], (uint16_t*) y};
    return gemv_common(x, ldx, gs, widths, 2, nullptr, ldy, m, k, K, mcg, mul1, workspace, ws_bytes, stream, true,
                       A_had);
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

int exl3_silu_mul(const void* gate, const void* up, int64_t ld_in, void* out, int64_t ld_out, int rows, int n,
                  void* stream)
{
    if (!gate || !up || !out || rows < 0 || n < 8 || n % 8 || ld_in < n || ld_out < n || ld_in % 8 || ld_out % 8 ||
        (((uintptr_t) gate) & 15) || (((uintptr_t) up) & 15) || (((uintptr_t) out) & 15))
        return EXL3_EINVAL;
    if (rows == 0) return EXL3_OK;
    const int64_t jobs = (int64_t) rows * (n / 8);
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned) ((jobs + 255) / 256)), dim3(256), 0, (hipStream_t) stream,
                       (const uint16_t*) gate, (const uint16_t*) up, ld_in, (uint16_t*) out, ld_out, rows, n / 8);
    return hipGetLastError() == hipSuccess ? EXL3_OK : EXL3_ELAUNCH;
}

int exl3_had_r_128(const void* in, int64_t ld_in, void* out, int64_t ld_out, int rows, int cols, const void* pre,
                   const void* post, float scale, void* stream)
{
    void* const outs[1] = {out};
    const void* const pres[1] = {pre};
    return launch_had(in, ld_in, outs, ld_out, rows, cols, pres, 1, post, scale, stream, true, nullptr);
}

int exl3_had_r_128_f32(const void* in, int64_t ld_in, void* out, int64_t ld_out, int rows, int cols, const void* pre,
                       const void* post, float scale, void* stream)
{
    void* const outs[1] = {out};
    const void* const pres[1] = {pre};
    return launch_had(in, ld_in, outs, ld_out, rows, cols, pres, 1, post, scale, stream, false, nullptr);
}

}  // extern "C"
