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
#include <mutex>

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
        const uint32_t* tp = trellis + ((int64_t) kt * nt_total + nt0 + strip + local_nt) * (8 * BITS);
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
// had_r_128: out = fp16(Had128(in [* pre]) * r * scale) [* post], one wave per 128-block
// (reference binding `had_r_128`, vllm_plugin/exl3rocm/ops.py:88,97)
// ============================================================================================
__global__ void __launch_bounds__(256) had_kernel(const uint32_t* __restrict__ in, int64_t ld_in, uint32_t* __restrict__ out,
                                                  int64_t ld_out, int rows, int cols, const uint32_t* __restrict__ pre,
                                                  const uint32_t* __restrict__ post, double scale)
{
    const int blocks_per_row = cols / 128;
    const int64_t job = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (job >= (int64_t) rows * blocks_per_row) return;
    const int lane = threadIdx.x & 63;
    const int64_t row = job / blocks_per_row;
    const int blk = (int) (job % blocks_per_row);
    const int64_t e2 = (int64_t) blk * 64 + lane;      // index in half2 units within the row
    const uint32_t v = in[row * (ld_in / 2) + e2];
    const uint32_t r = had128_pair(v, pre ? pre[e2] : 0u, pre != nullptr, post ? post[e2] : 0u, post != nullptr,
                                   R_SCALE * scale);
    out[row * (ld_out / 2) + e2] = r;
}

// ============================================================================================
// Fused GEMV
// ============================================================================================
struct GemvGroup {
    const uint32_t* trellis;   // tile words
    const uint32_t* suh;       // fp16 pairs
    const uint32_t* svh;       // fp16 pairs
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
    int M, k, n, S;
    int64_t ldy;
    float* part;               // [groups][NB][S][M][128] fp32 partials (S > 1)
    uint32_t* counters;        // [groups][NB], zero between calls
    int xcd_remap;
};

template <int MT>
__device__ __forceinline__ void gemv_load_a(const uint16_t* lds_a, int lda, int M, int j, int col, f16x8 (&A)[MT])
{
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + j;
        f16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
        if (m < M) v = *reinterpret_cast<const f16x8*>(lds_a + m * lda + col);
        A[mt] = v;
    }
}

template <int BITS, int CB, int MT>
__global__ void __launch_bounds__(256) gemv_kernel(GemvArgs a)
{
    extern __shared__ __align__(16) uint16_t smem[];
    __shared__ int s_last;
    const int NB = a.n / 128;
    const int S = a.S;
    int cb, sp;
    {
        const int b = blockIdx.x;
        if (a.xcd_remap) {
            const int per_xcd = (NB * S) / 8;
            const int u = (b & 7) * per_xcd + (b >> 3);
            cb = u / S;
            sp = u % S;
        } else {
            cb = b / S;
            sp = b % S;
        }
    }
    const int grp = blockIdx.y;
    const uint32_t* trel;
    const uint32_t* suh;
    const uint32_t* svh;
    uint16_t* y;
    if (a.tab_trellis) {
        trel = reinterpret_cast<const uint32_t*>(a.tab_trellis[grp]);
        suh = reinterpret_cast<const uint32_t*>(a.tab_suh[grp]);
        svh = reinterpret_cast<const uint32_t*>(a.tab_svh[grp]);
        y = a.g[0].y + grp * a.group_col_stride;
    } else {
        trel = a.g[grp].trellis;
        suh = a.g[grp].suh;
        svh = a.g[grp].svh;
        y = a.g[grp].y;
    }
    const int M = a.M;
    const int KR = a.k / S;
    const int k0 = sp * KR;
    const int lda = KR + 8;                       // padded LDS row (halves): rows land on distinct banks
    uint16_t* lds_a = smem;                       // [M][lda]
    uint16_t* lds_c = smem + M * lda;             // [M][136]
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;

    // ---- prologue: rotated input slice ------------------------------------------------------
    const int nblk = KR / 128;
    for (int job = wave; job < M * nblk; job += 4) {
        const int m = job / nblk, blk = job % nblk;
        const uint32_t xv = reinterpret_cast<const uint32_t*>(a.x + (int64_t) m * a.ldx + k0 + blk * 128)[lane];
        const uint32_t sv = suh[(k0 + blk * 128) / 2 + lane];
        reinterpret_cast<uint32_t*>(lds_a + m * lda + blk * 128)[lane] = had128_pair(xv, sv, true, 0u, false, R_SCALE);
    }
    __syncthreads();

    // ---- main loop -----------------------------------------------------------------------------
    const int g = lane >> 4, j = lane & 15, q = j & 7;
    const int NT = a.n / 16;
    const int nt = cb * 8 + wave * 2 + (j >> 3);
    const int kt0 = (k0 >> 4) + g;
    const int64_t tstride = (int64_t) 4 * NT * (8 * BITS);      // 4 k-tiles further
    const uint32_t* tp = trel + ((int64_t) kt0 * NT + nt) * (8 * BITS);
    const int steps = KR / 64;

    f32x4 acc[2][MT];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[h][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    uint32_t Wn[BITS + 1];
    load_qblock<BITS>(tp, q, Wn);
    for (int st = 0; st < steps; ++st) {
        uint32_t Wc[BITS + 1];
#pragma unroll
        for (int i = 0; i <= BITS; ++i) Wc[i] = Wn[i];
        if (st + 1 < steps) load_qblock<BITS>(tp + (int64_t) (st + 1) * tstride, q, Wn);
        uint32_t P[16];
        decode_qblock<BITS, CB>(Wc, P);
        const int col = (st * 4 + g) * 16;
        f16x8 A0[MT], A1[MT];
        gemv_load_a<MT>(lds_a, lda, M, j, col, A0);
        gemv_load_a<MT>(lds_a, lda, M, j, col + 8, A1);
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
    }

    // ---- epilogue ------------------------------------------------------------------------------
    // lane holds rows mt*16 + 4*g + v (v = 0..3) of MFMA column j; MFMA h covers tile columns +8h
    const int colb = wave * 32 + (j >> 3) * 16 + (j & 7);        // + 8h
    if (S == 1) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int m = mt * 16 + 4 * g + v;
                    if (m < M) lds_c[m * 136 + colb + 8 * h] = f16_bits((f16) acc[h][mt][v]);
                }
    } else {
        float* slab = a.part + ((int64_t) (grp * NB + cb) * S + sp) * M * 128;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int m = mt * 16 + 4 * g + v;
                    if (m < M) slab[m * 128 + colb + 8 * h] = acc[h][mt][v];
                }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __syncthreads();
        if (threadIdx.x == 0) {
            const uint32_t prev = __hip_atomic_fetch_add(&a.counters[grp * NB + cb], 1u, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            s_last = prev == (uint32_t) (S - 1);
        }
        __syncthreads();
        if (!s_last) return;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        const float* base = a.part + (int64_t) (grp * NB + cb) * S * M * 128;
        for (int e = threadIdx.x; e < M * 128; e += 256) {
            float s = 0.f;
            for (int i = 0; i < S; ++i) s += __builtin_nontemporal_load(base + (int64_t) i * M * 128 + e);
            lds_c[(e >> 7) * 136 + (e & 127)] = f16_bits((f16) s);
        }
        if (threadIdx.x == 0) a.counters[grp * NB + cb] = 0u;    // ready for the next call (stream order)
    }
    __syncthreads();
    // output Hadamard + svh for every row of this 128-column block
    const uint32_t sv = svh[cb * 64 + lane];
    for (int m = wave; m < M; m += 4) {
        const uint32_t c2 = reinterpret_cast<const uint32_t*>(lds_c + m * 136)[lane];
        const uint32_t r = had128_pair(c2, 0u, false, sv, true, R_SCALE);
        reinterpret_cast<uint32_t*>(y + (int64_t) m * a.ldy + cb * 128)[lane] = r;
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

// Split count over k: depends on (k, n) only (never on m or the group count), so rows and groups
// stay bitwise equal to the single-row, single-group call.
int choose_splits(int k, int n)
{
    const int kb = k / 128, nb = n / 128;
    const int forced = env_int("EXL3_GEMV_SPLITS", 0);
    if (forced > 0 && kb % forced == 0) return forced;
    const int target = env_int("EXL3_GEMV_TARGET_WGS", 512);
    int best = kb;
    for (int d = 1; d <= kb; ++d) {
        if (kb % d) continue;
        if (kb / d > 16) continue;                 // k-slice <= 2048 (LDS budget at M = 32)
        best = d;
        if ((int64_t) nb * d >= target) break;
    }
    return best;
}

size_t lds_bytes(int M, int KR) { return (size_t) M * (KR + 8) * 2 + (size_t) M * 136 * 2; }

template <int BITS, int CB, int MT>
int launch_gemv_t(const GemvArgs& a, int groups, hipStream_t stream)
{
    const int NB = a.n / 128;
    const size_t lds = lds_bytes(a.M, a.k / a.S);
    static std::once_flag once;
    std::call_once(once, [] {
        (void) hipFuncSetAttribute((const void*) gemv_kernel<BITS, CB, MT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            150 * 1024);
    });
    hipLaunchKernelGGL((gemv_kernel<BITS, CB, MT>), dim3(NB * a.S, groups), dim3(256), lds, stream, a);
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

// workspace layout: [counters: fixed EXL3_GEMV_COUNTER_BYTES region][partials: groups*NB*S*M*128 f32].
// The counter region has a fixed size so calls of different shapes sharing one workspace never
// see another shape's partial sums where their counters live.
constexpr size_t COUNTER_BYTES = EXL3_GEMV_COUNTER_BYTES;

size_t gemv_ws_bytes(int m, int k, int n, int groups)
{
    const int S = choose_splits(k, n), NB = n / 128;
    if (S == 1) return COUNTER_BYTES;
    return COUNTER_BYTES + (size_t) groups * NB * S * m * 128 * 4;
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
    // the kernel moves fp16 pairs: x rows, y rows, suh and svh must be 4-byte aligned
    if ((ldx & 1) || (ldy & 1) || (((uintptr_t) x) & 3)) return EXL3_EINVAL;
    // with pointer tables only gs[0].y is given; the table entries are the caller's contract
    for (int i = 0; i < (tabs ? 1 : groups); ++i) {
        if (!gs[i].y || (((uintptr_t) gs[i].y) & 3)) return EXL3_EINVAL;
        if (!tabs && ((((uintptr_t) gs[i].suh) & 3) || (((uintptr_t) gs[i].svh) & 3) || (((uintptr_t) gs[i].trellis) & 15)))
            return EXL3_EINVAL;
    }
    if (groups > 1 && !tabs && m > 1 && ldy < (int64_t) groups * n) return EXL3_EINVAL;
    if (!shape_ok(m, k, n, K)) return EXL3_DECLINED;
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
    a.S = choose_splits(k, n);
    a.ldy = ldy;
    const int NB = n / 128;
    if ((size_t) groups * NB * 4 > COUNTER_BYTES) return EXL3_DECLINED;
    a.counters = (uint32_t*) ws;
    a.part = (float*) ((char*) ws + COUNTER_BYTES);
    a.xcd_remap = (NB * a.S) % 8 == 0 && NB % 8 == 0;
    return launch_gemv(a, K, codebook_of(mcg, mul1), groups, (hipStream_t) stream);
}

}  // namespace

// ============================================================================================
// C ABI
// ============================================================================================
extern "C" {

int exl3_abi_version(void) { return EXL3_ABI_VERSION; }

int exl3_gemv_splits(int k, int n) { return (k % 128 || k < 128) ? 0 : choose_splits(k, n); }

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
    GemvGroup g{(const uint32_t*) trellis, (const uint32_t*) suh, (const uint32_t*) svh, (uint16_t*) y};
    return gemv_common(x, ldx, &g, 1, nullptr, 0, ldy, m, k, n, K, mcg, mul1, workspace, ws_bytes, stream);
}

int exl3_gemv_mr(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh, void* A_had,
                 const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
                 void* stream)
{
    (void) A_had;
    if (!trellis || !y || !suh || !svh) return EXL3_EINVAL;
    GemvGroup g{(const uint32_t*) trellis, (const uint32_t*) suh, (const uint32_t*) svh, (uint16_t*) y};
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
        gs[i] = {(const uint32_t*) trellis[i], (const uint32_t*) suh[i], (const uint32_t*) svh[i],
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
    if (!in || !out || rows < 0 || cols % 128 || cols < 128 || ld_in < cols || ld_out < cols || ld_in % 2 || ld_out % 2 ||
        (((uintptr_t) in) & 3) || (((uintptr_t) out) & 3) || (((uintptr_t) pre) & 3) || (((uintptr_t) post) & 3))
        return EXL3_EINVAL;
    if (rows == 0) return EXL3_OK;
    const int64_t jobs = (int64_t) rows * (cols / 128);
    hipLaunchKernelGGL(had_kernel, dim3((unsigned) ((jobs + 3) / 4)), dim3(256), 0, (hipStream_t) stream,
                       (const uint32_t*) in, ld_in, (uint32_t*) out, ld_out, rows, cols, (const uint32_t*) pre,
                       (const uint32_t*) post, (double) scale);
    return hipGetLastError() == hipSuccess ? EXL3_OK : EXL3_ELAUNCH;
}

}  // extern "C"
