/*
 * exl3_mi355x.h -- C ABI of the MI355X (gfx950) EXL3 quantized-linear library
 * (libexl3_mi355x.so).
 *
 * Every entry point replaces one call of the reference's kernel extension (`exllamav3_ext`,
 * bound by pybind11 in the un-vendored exllamav3 ROCm fork) as it is called from the vLLM
 * plugin's custom ops (vllm_plugin/exl3rocm/ops.py) and tests.  Arguments are raw device
 * pointers, element counts and strides (in elements), plus a hipStream_t passed as void*.
 * No torch types cross this boundary.
 *
 * Conventions
 *   - fp16 tensors are IEEE binary16; the trellis is the checkpoint's (k/16, n/16, 16*K) int16
 *     tensor, read as little-endian 16-bit words; suh [k], svh [n] are fp16.
 *   - Alignment: trellis, x, y, suh, svh 16 bytes, row strides multiples of 8 elements (fp16
 *     moves in 16-byte groups of 8); violations return EXL3_EINVAL before any launch.
 *   - Codebook flags: mul1 != 0 -> mul1 (cb 2), else mcg != 0 -> mcg (cb 1), else 3inst (cb 0).
 *   - K is the bitrate (bits per weight, 1..8).
 *   - Return status: 0 done; > 0 declined (ineligible but valid call, outputs untouched);
 *     < 0 invalid arguments or launch failure.
 *   - All buffers are caller-owned.  Nothing here allocates device memory.  Launches are
 *     asynchronous on `stream`; no call synchronizes or reads back.  Calls are graph-capturable.
 *   - The GEMV entry points need a caller workspace of exl3_gemv_workspace_size() bytes whose
 *     first EXL3_GEMV_COUNTER_BYTES (completion counters) are zero before the first call; every
 *     call leaves them zero again.  One workspace may serve calls of any shape in stream order;
 *     calls that overlap on one workspace race: give concurrent streams their own.
 *   - Results are deterministic: repeat calls and different streams give bitwise-equal output,
 *     and each row of an m-row call equals the m == 1 call of that row.
 */
#ifndef EXL3_MI355X_H
#define EXL3_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EXL3_ABI_VERSION 3       /* 2: exl3_gemv_f32, exl3_gemm_trellis_silu_in; 3: exl3_gemv_silu_prerot_rows,
                                    exl3_gemm_trellis_workspace_bound, the plain GEMV up to 64 rows */
#define EXL3_MAX_GROUPS 4       /* groups per grouped launch (reference EXL3_GEMV_MRG_MAX) */
#define EXL3_GEMV_MAX_ROWS 64   /* rows the plain fused GEMV takes (exl3_gemv_mr and its grouped forms) */
#define EXL3_GEMV_FUSED_MAX_ROWS 32 /* rows of the fused-epilogue forms (SiLU input, gated, approximate) */
#define EXL3_GEMV_COUNTER_BYTES 262144 /* workspace head reserved for completion counters (one per 128-byte line) */
#define EXL3_NOALLOC_SCRATCH_BYTES 17039360 /* 16.25 MiB: exl3_gemv_mr_noalloc's per-GPU device array */

#define EXL3_OK 0
#define EXL3_DECLINED 1
#define EXL3_EINVAL (-1)
#define EXL3_ELAUNCH (-2)
#define EXL3_EWORKSPACE (-3)

int exl3_abi_version(void);

/* Codebook decode of raw 16-bit states to fp32 values.
 * Replaces `decode(codes int16[16,256], out fp32[16,256], mcg, mul1)`
 * (reference tests/test_gpu_parity.py:101-109). */
int exl3_decode(const void* states, void* out_f32, int64_t count, int mcg, int mul1, void* stream);

/* Dense fp16 W[k, n] from the trellis.
 * Replaces `reconstruct(W, trellis, K, mcg, mul1)` (reference vllm_plugin/exl3rocm/ops.py:93). */
int exl3_reconstruct(void* W, const void* trellis, int k, int n, int K, int mcg, int mul1, void* stream);

/* Columns [n0, n0 + n_out) of W into a [k, n_out] buffer with row stride ldw (multiples of 16).
 * Replaces `reconstruct_slice(W, trellis, K, mcg, mul1, n0)` (reference ops.py:95). */
int exl3_reconstruct_slice(void* W, int64_t ldw, const void* trellis, int k, int n, int K, int mcg, int mul1, int n0,
                           int n_out, void* stream);

/* Blockwise 128-point Hadamard over rows: out = fp16(H128(in [* pre]) * r * scale) [* post],
 * r = 0.088388347648; pre / post may be NULL; in == out is allowed.  float64 butterflies: exact
 * (bit-equal to the oracle's float64 product) unless a 128-block spans more than 35 binades.
 * Replaces `had_r_128(in, out, pre, post, scale)` (reference ops.py:88,97). */
int exl3_had_r_128(const void* in, int64_t ld_in, void* out, int64_t ld_out, int rows, int cols, const void* pre,
                   const void* post, float scale, void* stream);

/* The same transform with float32 accumulation on the matrix cores (fp16 products, fp32 sums):
 * bitwise the values the prefill GEMM uses for its input transforms (pre) and in its epilogue
 * (post), which can differ from exl3_had_r_128's exact float64 result in the last fp16 place (by
 * at most the error of an fp32 summation of a block's 128 terms before that rounding).  (The fused
 * GEMV's transforms are float64, exl3_had_r_128's values.)
 * No counterpart of its own in the reference (whose had_r_128 serves both roles, ops.py:88,97).
 * Callers: exl3rocm's reconstruct + hgemm_recon prefill route, so that it stays bitwise equal to
 * the fused prefill route. */
int exl3_had_r_128_f32(const void* in, int64_t ld_in, void* out, int64_t ld_out, int rows, int cols, const void* pre,
                       const void* post, float scale, void* stream);

/* Workgroups per group of the fused GEMV's stream-K grid for a (k, n) layer launched with
 * `groups` groups (diagnostic; a function of the shape only, never of m). */
int exl3_gemv_grid(int k, int n, int groups);

/* Workspace bytes the fused GEMV needs for m rows and `groups` groups.
 * Has no reference counterpart: the reference fork allocates its counters inside the extension
 * (vllm_plugin/patches/exl3-fork/0003-fused-had-graph-capture.patch:17-40); here the caller owns them. */
size_t exl3_gemv_workspace_size(int m, int k, int n, int K, int groups);

/* Eligibility of the fused multi-row GEMV.
 * Replaces `exl3_gemv_mr_supported(m, k, n, K, mcg, mul1)`
 * (reference vllm_plugin/patches/exl3-fork/0002-gemv-multirow.patch:334-338).  Unlike the
 * reference (mul1 only), every codebook is supported; 1 <= m <= EXL3_GEMV_MAX_ROWS (64), k and n multiples
 * of 128. */
int exl3_gemv_mr_supported(int m, int k, int n, int K, int mcg, int mul1);

/* M == 1 EXL3 linear, y = fp16(H(fp16(H(x*suh)) . W) * svh) with fused input and output
 * Hadamards.  m != 1 declines (returns 1) without touching y.
 * Replaces `exl3_gemv(A, B, C, suh, A_had, svh, mcg, mul1)` (reference tests/test_gpu_parity.py:160)
 * and the M == 1 route of `exl3_gemm` (reference ops.py:80-82).  A_had is accepted for
 * signature parity; the rotated input lives in LDS and A_had is not written. */
int exl3_gemv(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh, void* A_had,
              const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
              void* stream);

/* exl3_gemv with an fp32 output y[n]: C = H(x*suh) . W stays fp32 (no fp16 rounding) and
 * y = (float) (H(C) * r) * svh (float64 butterflies over the fp32 C).  m != 1 declines (returns 1)
 * without touching y.  Replaces `exl3_gemv(A, B, C, ...)` called with a float32 C (reference
 * tests/test_fused_had.py:59-65,153-158; the fused epilogue's c_fp32 form,
 * patches/experimental-full.patch:638-653). */
int exl3_gemv_f32(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh, void* A_had,
                  const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
                  void* stream);

/* 1 <= m <= EXL3_GEMV_MAX_ROWS (64) EXL3 linear, output rows with stride ldy.
 * A_had: optional fp16 scratch of m * k elements (groups * m * k for the grouped forms).  When
 * given and the launch takes the pre-rotation pass (m x the most units one workgroup owns >=
 * u x (groups + 1), u = 60 below 6 units per workgroup, 42 from 6, 36 from 20; or m >=
 * EXL3_GEMV_PREROT_M when that is set; exl3_gemv_prerot_rows), the input
 * is rotated once per group into it,
 * A_had = fp16(Had128(fp16(x * suh))) as in the reference, and the GEMV reads those rows; otherwise
 * every workgroup rotates its own k-range in LDS.  Either way the output is the same, bitwise.
 * Replaces `exl3_gemv_mr(A, B, C, suh, A_had, svh, K, mcg, mul1)` (reference ops.py:85;
 * 0002-gemv-multirow.patch:409-422). */
int exl3_gemv_mr(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh, void* A_had,
                 const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
                 void* stream);

/* Approximate mul1 EXL3 linear for 1 <= m <= 32 (opt-in; outputs are not the faithful staging's):
 *   mode 1 (affine): C = k_inv * sum_k a_k (1024 + s_k) + k_bias * sum_k a_k, i.e. the mul1 weights
 *     before their fp16 rounding (rel-L2 ~5e-4 from the faithful output);
 *   mode 2 (int8 activations): the rotated input quantized per (row, 128-input slice) as
 *     v = clamp(rint(a / q), -127, 127), q = max(|a|, 1e-8) / 127, and C = sum over slices of
 *     q (k_inv sum v s + (1024 k_inv + k_bias) sum v) -- the reference's int8 path (integer
 *     products, affine epilogue), with one scale per slice.  A slice's sum v s is exact
 *     (|v s| <= 127 * 1020, 128 terms: below 2^24, so its fp32 MFMA accumulation never rounds).
 * C is rounded to fp16 and transformed as in exl3_gemv_mr.  Arguments, workspace and A_had as
 * exl3_gemv_mr (mul1 codebook implied).  Returns EXL3_EINVAL for another mode.
 * Replaces the reference's opt-in int8 GEMV behind exl3_gemm (EXL3_ROCM_GFX1201_INT8,
 * vllm_plugin/patches/exl3-fork/0001-int8-port-gfx1201-compat.patch:153-523; oracle
 * reference/exl3_oracle.py:357-412); mode 1 has no counterpart (the same epilogue on fp16
 * activations).  On gfx950 the dot products run on fp16 MFMA in both modes (the quantized values
 * and 1024 + s are exact fp16 integers): the saving is the per-weight fp16 scale of the decode. */
int exl3_gemv_mr_approx(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh,
                        void* A_had, const void* svh, int m, int k, int n, int K, int mode, void* workspace,
                        size_t ws_bytes, void* stream);

/* Up to 4 groups sharing x (equal k, n, K): group i writes columns [i*n, (i+1)*n) of y.
 * trellis / suh / svh are host arrays of device pointers.
 * Replaces `exl3_gemv_mr_grouped(A, [B], C, [suh], A_had, [svh], K, mcg, mul1, bszm)`
 * (reference ops.py:164-165; 0002-gemv-multirow.patch:424-440).  bszm_for_warps is accepted for
 * signature parity: the split choice here never depends on it. */
int exl3_gemv_mr_grouped(const void* x, int64_t ldx, const void* const* trellis, void* y, int64_t ldy,
                         const void* const* suh, void* A_had, const void* const* svh, int groups, int m, int k, int n,
                         int K, int mcg, int mul1, int bszm_for_warps, void* workspace, size_t ws_bytes, void* stream);

/* Up to 4 groups sharing x and K but of any widths (q / k / v projections): group i writes the
 * widths[i] columns of y that follow groups 0 .. i-1; rows ldy apart (ldy >= sum of widths).
 * No counterpart in the reference: its linear_groups launches unequal widths one by one
 * (reference ops.py:157-169).  Callers: exl3rocm's linear_groups for mixed-width runs.  The
 * groups share one stream-K grid, so a module pays one launch, prologue and completion. */
int exl3_gemv_mr_grouped_widths(const void* x, int64_t ldx, const void* const* trellis, void* y, int64_t ldy,
                                const void* const* suh, void* A_had, const void* const* svh, const int* widths,
                                int groups, int m, int k, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
                                void* stream);

/* Workspace bytes exl3_gemv_mr_grouped_widths needs (0 for an ineligible shape).  No reference
 * counterpart, as exl3_gemv_workspace_size. */
size_t exl3_gemv_workspace_size_widths(int m, int k, const int* widths, int groups);

/* Rows from which the multi-row GEMV entry points may rotate the input once per group into A_had;
 * callers need not provide A_had below it.  2 by default: the library pre-rotates a launch when
 * rows x the most units one workgroup owns >= u x (groups + 1), u = 60 below 6 units per
 * workgroup, 42 from 6, 36 from 20 (gate and down at 6 rows, gate/up at 4, q/k/v at 24, o at 24)
 * and rotates in LDS otherwise, with the same outputs bitwise.  EXL3_GEMV_PREROT_M
 * fixes one row count for every shape instead and is returned.  No reference counterpart.
 * Callers: exl3rocm's kernel wrappers. */
int exl3_gemv_prerot_rows(void);

/* Rows from which exl3_gemv_silu_in forms and rotates its SiLU input once, by a separate pass into
 * A_had, instead of in every workgroup (EXL3_GEMV_SILU_PREROT_M, default 4); below it A_had is not
 * read.  No reference counterpart.  Callers: exl3rocm's kernel wrappers, which pass no scratch
 * below it. */
int exl3_gemv_silu_prerot_rows(void);

/* Self-check of the GEMV's stream-K unit split (host only, no GPU): the kernels' 32-bit
 * multiply-high division forms of lo(w) and owner(u) against 64-bit arithmetic and brute force for
 * U units over G workgroups (h of them weighted wa, the rest wb), plus the divider at its range
 * edges.  Returns the number of mismatches (0), or -1 for arguments outside the split's domain.
 * No reference counterpart.  Callers: the CPU tests. */
int exl3_gemv_split_check(int U, int G, int h, int wa, int wb);

/* Gated MLP input, 1 <= m <= 32: the gate (group 0) and up (group 1) linears of one module, equal
 * K and width n, share x and one stream-K launch; y[m, n] (rows ldy apart, ldy >= n) receives
 * fp16(fp16(silu(gate)) * up), where gate and up are exactly what exl3_gemv_mr_grouped writes
 * (fp16 C, output Hadamard, svh) and silu is g / (1 + exp(-g)) in fp32 (the SiluAndMul
 * roundings).  trellis / suh / svh: host arrays of 2 device pointers; A_had as exl3_gemv_mr
 * (2 * m * k).  Workspace as
 * exl3_gemv_workspace_size(m, k, n, K, 2).  No counterpart in the reference: its gated MLP runs
 * the gate/up linear_groups, then a separate SiLU-and-mul (reference
 * docs/EFFICIENCY_INVESTIGATION.md:36-66 proposes this fusion).  Callers: model code that owns
 * the gate/up module and its activation (exl3rocm's linear_silu_mul op).  Removes the [m, 2n]
 * intermediate and the activation launch. */
int exl3_gemv_silu_mul(const void* x, int64_t ldx, const void* const* trellis, void* y, int64_t ldy,
                       const void* const* suh, void* A_had, const void* const* svh, int m, int k, int n, int K, int mcg,
                       int mul1, void* workspace, size_t ws_bytes, void* stream);

/* Elementwise SiLU-and-mul: out[r][c] = fp16(fp16(silu(gate[r][c])) * up[r][c]) for r < rows,
 * c < n (n % 8 == 0; gate and up rows ld_in apart, out rows ld_out apart; 16-byte aligned).
 * No counterpart in the reference (vLLM's SiluAndMul does this there).  Callers: exl3rocm's
 * linear_silu_mul op for m > 32, after the grouped prefill. */
int exl3_silu_mul(const void* gate, const void* up, int64_t ld_in, void* out, int64_t ld_out, int rows, int n,
                  void* stream);

/* Gated MLP output, 1 <= m <= 32: exl3_gemv_mr over the input x = fp16(fp16(silu(gate)) * up)
 * (the exl3_silu_mul roundings), formed as the rows load; gate and up rows ld_in apart (a gated
 * module's grouped [m, 2n] output: gate = y, up = y + n, ld_in = 2n).  Bitwise equal to
 * exl3_silu_mul followed by exl3_gemv_mr.  A_had (m * k, optional) as exl3_gemv_mr, but from
 * m >= 4 (EXL3_GEMV_SILU_PREROT_M): it receives the rotated activation.  No counterpart in the reference: its down
 * projection reads the SiluAndMul output (reference docs/EFFICIENCY_INVESTIGATION.md:36-66
 * proposes fusing the activation).  Callers: exl3rocm's silu_mul_linear op (the down projection
 * of a decode step).  Removes the activation launch and its [m, n] round trip. */
int exl3_gemv_silu_in(const void* gate, const void* up, int64_t ld_in, const void* trellis, void* y, int64_t ldy,
                      const void* suh, void* A_had, const void* svh, int m, int k, int n, int K, int mcg, int mul1,
                      void* workspace, size_t ws_bytes, void* stream);

/* Grouped M == 1 linear over device int64 pointer tables (one entry per group), output
 * (groups, 1, n) == the concatenated row.
 * Replaces `exl3_mgemm(x, ptrs_trellis, y, ptrs_suh, xh, ptrs_svh, ...)` (reference ops.py:137-138). */
int exl3_mgemm(const void* x, const int64_t* ptrs_trellis, void* y, const int64_t* ptrs_suh, void* xh,
               const int64_t* ptrs_svh, int groups, int k, int n, int K, int mcg, int mul1, void* workspace,
               size_t ws_bytes, void* stream);

/* Dense fp16 GEMM y[m, n] = fp16(x[m, k] . W[k, n]) with fp32 accumulation (MFMA).
 * Replaces `hgemm_recon(xh, W, y)` (reference ops.py:96), which accumulates in fp16. */
int exl3_hgemm_recon(const void* x, int64_t ldx, const void* W, int64_t ldw, void* y, int64_t ldy, int m, int k, int n,
                     void* stream);

/* Prefill EXL3 linear for any m: the trellis is decoded into LDS tiles and fed to fp16 MFMA
 * with fp32 accumulation; input and output Hadamards run as separate passes.  xh is an
 * [m, k] fp16 scratch (the rotated input).
 * Replaces the reconstruct + hgemm_recon route of `exl3rocm::linear` (reference ops.py:86-97). */
int exl3_gemm_trellis(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh,
                      void* xh, const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* stream);

/* Prefill EXL3 linear of up to 4 groups sharing x and K but of any widths (the checkpoint tensors
 * of a fused module: q / k / v, gate / up): group i writes the widths[i] columns of y that follow
 * groups 0 .. i-1 (rows ldy apart, ldy >= sum of widths).  xh is an fp16 scratch of groups * m * k
 * elements (each group's rotated input).  No counterpart in the reference: its linear_groups runs
 * one prefill per group (reference vllm_plugin/exl3rocm/ops.py:171-175).  Callers: exl3rocm's
 * linear_groups for M > 32.  All groups' output tiles share one GEMM launch, so a module fills the
 * GPU as one layer would.  workspace / ws_bytes: see exl3_gemm_trellis_workspace_size. */
int exl3_gemm_trellis_grouped(const void* x, int64_t ldx, const void* const* trellis, void* y, int64_t ldy,
                              const void* const* suh, void* xh, const void* const* svh, const int* widths, int groups,
                              int m, int k, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
                              void* stream);

/* Gated MLP output for any m (the prefill form of exl3_gemv_silu_in): the exl3_gemm_trellis_grouped
 * prefill of one group over the input x = fp16(fp16(silu(gate)) * up) (the exl3_silu_mul
 * roundings), formed by the input transform as it loads the rows; gate and up rows ldx apart (a
 * gated module's grouped [m, 2k] output: gate = y, up = y + k, ldx = 2k).  xh: [m, k] fp16
 * scratch (the rotated activation); workspace / ws_bytes: exl3_gemm_trellis_workspace_size(m, k,
 * &n, 1).  Bitwise equal to exl3_silu_mul followed by exl3_gemm_trellis_grouped.  No counterpart in
 * the reference: its down projection reads the SiluAndMul output (reference
 * docs/EFFICIENCY_INVESTIGATION.md:36-66 proposes fusing the activation).  Callers: exl3rocm's
 * silu_mul_linear op for m > 32.  Removes the activation launch and its [m, k] write and read. */
int exl3_gemm_trellis_silu_in(const void* gate, const void* up, int64_t ldx, const void* trellis, void* y, int64_t ldy,
                              const void* suh, void* xh, const void* svh, int m, int k, int n, int K, int mcg, int mul1,
                              void* workspace, size_t ws_bytes, void* stream);

/* Workspace bytes exl3_gemm_trellis_grouped uses to balance the launch's last, partial wave of
 * output tiles (those tiles are split along K; fp32 partials and completion counters).  0 when the
 * shape needs none.  Zero before the first call; every call leaves its counters zero.  With a
 * smaller or NULL workspace the tail is not split: the same results to the tolerance, less
 * balance.  No reference counterpart (the reference prefill has no split). */
size_t exl3_gemm_trellis_workspace_size(int m, int k, const int* widths, int groups);

/* The largest workspace exl3_gemm_trellis_workspace_size returns for any shape (a plan splits at
 * most two thirds of one wave of tiles into two pieces, or fewer tiles into at most one wave of
 * pieces): one workspace of this size serves every prefill call, so a caller that reserves it on a
 * stream at load time never needs another before graph capture there.  No reference counterpart.
 * Callers: exl3rocm's prefill workspace. */
size_t exl3_gemm_trellis_workspace_bound(void);

/* Dispatcher by row count: m <= 32 -> fused GEMV, else the prefill GEMM.  Returns the route
 * tag (1 = GEMV, 2 = prefill GEMM) or a negative error.
 * Replaces `exl3_gemm(A, B, C, suh, A_had, svh, -1, mcg, mul1, 0) -> int` (reference ops.py:82). */
int exl3_gemm(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh, void* A_had,
              const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* workspace, size_t ws_bytes,
              void* stream);

/* exl3_gemv_mr without a workspace argument and without any allocation: the same kernels and the
 * same output, bitwise, with the workspace in a file-scope device array of
 * EXL3_NOALLOC_SCRATCH_BYTES that each GPU keeps until the process ends.  Shapes whose workspace
 * (exl3_gemv_workspace_size(m, k, n, K, 1)) exceeds it return EXL3_EWORKSPACE before any launch:
 * at m <= 32 every k, n <= 32768 with n <= 21760 fits (every Qwen-27B layer), the first that does
 * not is k = 256, n = 21888.  Shapes the GEMV does not take return exl3_gemv_mr's status.  Calls that overlap on one GPU race on the
 * array: serialize them (one stream, or one graph replay at a time).
 * No counterpart in the reference.  For callers that cannot allocate device memory: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc. */
int exl3_gemv_mr_noalloc(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh,
                         const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_MI355X_H */
