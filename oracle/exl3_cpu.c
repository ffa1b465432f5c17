/*
 * exl3_cpu.c -- C restatement of the EXL3 trellis arithmetic.  TEST INFRASTRUCTURE ONLY.
 *
 * The checker and the CPU baseline, never the product: only tests/, the smoke entry
 * point and bench.py's cpu_baseline leg load this library (oracle/libexl3cpu.so).
 * It restates reference/exl3_oracle.py (function citations below) in scalar C with
 * OpenMP over output tiles, and is pinned against oracle/exl3_oracle.py and the golden
 * vectors the reference oracle wrote (tests/test_oracle.py).
 *
 * Numerics follow the oracle's faithful staging exactly: fp16 inputs, fp16 pre-scale
 * product, Hadamard butterflies in float64 (exact for fp16 data), fp16 A_had, float64
 * dot products accumulated in k order, fp16 C, fp16 output Hadamard, fp16 post-scale.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define R_SCALE 0.088388347648   /* reference exl3_oracle.py:47 */

/* ---------------------------------------------------------------- fp16 <-> double */
double exl3cpu_f16_to_f64(uint16_t h)
{
    int s = h >> 15, e = (h >> 10) & 31, f = h & 1023;
    double v;
    if (e == 0) v = ldexp((double) f, -24);
    else if (e == 31) v = f ? NAN : INFINITY;
    else v = ldexp((double) (1024 + f), e - 25);
    return s ? -v : v;
}

/* Round a double to the nearest fp16, ties to even (default FP environment). */
uint16_t exl3cpu_f64_to_f16(double v)
{
    uint16_t sign = signbit(v) ? 0x8000 : 0;
    double a = fabs(v);
    if (isnan(v)) return sign | 0x7E00;
    if (a >= 65520.0) return sign | 0x7C00;
    if (a < 6.103515625e-05) {                 /* below 2^-14: subnormal quantum 2^-24 */
        double q = nearbyint(ldexp(a, 24));
        return sign | (uint16_t) q;            /* q == 1024 lands on the smallest normal */
    }
    int e;
    frexp(a, &e);                              /* a in [2^(e-1), 2^e) */
    int E = e - 1;
    double q = nearbyint(ldexp(a, 10 - E));    /* in [1024, 2048] */
    if (q >= 2048.0) { q = 1024.0; E += 1; }
    if (E > 15) return sign | 0x7C00;
    return sign | (uint16_t) (((E + 15) << 10) | ((int) q - 1024));
}

static double rnd16(double v) { return exl3cpu_f16_to_f64(exl3cpu_f64_to_f16(v)); }

/* ---------------------------------------------------------------- codebooks (oracle :67-123) */
static inline uint32_t hash32(uint32_t w, int cb)
{
    if (cb == 2) return w * 0x83DCD12Du;
    if (cb == 1) return w * 0xCBAC1FEDu;
    return w * 89226354u + 64248484u;
}

uint16_t exl3cpu_codebook(uint16_t state, int cb)
{
    uint32_t x = hash32(state, cb);
    if (cb == 2) {
        uint32_t s = (x & 255) + ((x >> 8) & 255) + ((x >> 16) & 255) + (x >> 24);
        /* (1024 + s) * K_INV + K_BIAS is exact in double: one rounding == fused fp16 fma */
        return exl3cpu_f64_to_f16((1024.0 + s) * exl3cpu_f16_to_f64(0x1EEE) + exl3cpu_f16_to_f64(0xC931));
    }
    x = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
    return exl3cpu_f64_to_f16(exl3cpu_f16_to_f64((uint16_t) x) + exl3cpu_f16_to_f64((uint16_t) (x >> 16)));
}

/* ---------------------------------------------------------------- windows + placement (oracle :129-188) */
static inline void rowcol(int t, int* r, int* c)
{
    int L = t >> 3, i = t & 7;
    *r = 2 * (L & 3) + (i & 1) + 8 * ((i >> 1) & 1);
    *c = 2 * (L >> 3) + ((L >> 2) & 1) + 8 * (i >> 2);
}

static inline uint16_t window(const uint16_t* tile, int bits, int t)
{
    const int nw = 8 * bits;
    int64_t end = (int64_t) (t + 257) * bits;
    int64_t first = end - 16;
    int hi = (int) ((first / 32) % nw), lo = (int) (((end - 1) / 32) % nw);
    int sh = (int) (((end - 1) / 32 + 1) * 32 - end);
    uint64_t whi = (uint64_t) tile[2 * hi] | ((uint64_t) tile[2 * hi + 1] << 16);
    uint64_t wlo = (uint64_t) tile[2 * lo] | ((uint64_t) tile[2 * lo + 1] << 16);
    return (uint16_t) ((((whi << 32) | wlo) >> sh) & 0xFFFF);
}

/* One packed tile -> 16x16 fp16 bit patterns, row-major [row][col]. */
void exl3cpu_decode_tile(const uint16_t* tile, int bits, int cb, uint16_t* out)
{
    for (int t = 0; t < 256; ++t) {
        int r, c;
        rowcol(t, &r, &c);
        out[r * 16 + c] = exl3cpu_codebook(window(tile, bits, t), cb);
    }
}

void exl3cpu_states(const uint16_t* tile, int bits, uint16_t* out)
{
    for (int t = 0; t < 256; ++t) out[t] = window(tile, bits, t);
}

int exl3cpu_decode_states(const uint16_t* states, int64_t count, int cb, uint16_t* out)
{
    if (cb < 0 || cb > 2) return -1;
    for (int64_t i = 0; i < count; ++i) out[i] = exl3cpu_codebook(states[i], cb);
    return 0;
}

/* reconstruct (oracle decode_trellis :206): W[k][n] fp16 bit patterns */
int exl3cpu_reconstruct(const uint16_t* trellis, int k, int n, int bits, int cb, uint16_t* W, int threads)
{
    if (k % 16 || n % 16 || bits < 1 || bits > 8 || cb < 0 || cb > 2) return -1;
    const int kt = k / 16, nt = n / 16, per = 16 * bits;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
    for (int64_t ti = 0; ti < (int64_t) kt * nt; ++ti) {
        uint16_t tile[256];
        int a = (int) (ti / nt), b = (int) (ti % nt);
        exl3cpu_decode_tile(trellis + ti * per, bits, cb, tile);
        for (int r = 0; r < 16; ++r)
            memcpy(W + (int64_t) (a * 16 + r) * n + b * 16, tile + r * 16, 32);
    }
    return 0;
}

/* ---------------------------------------------------------------- Hadamard (oracle :236-304) */
static void wht128(double* v)
{
    for (int h = 1; h < 128; h <<= 1)
        for (int i = 0; i < 128; i += 2 * h)
            for (int j = i; j < i + h; ++j) {
                double a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
}

/* A_had = fp16(Had128(fp16(x * suh))), rows of length k, fp16 bit patterns in and out */
int exl3cpu_had_in(const uint16_t* x, int m, int k, const uint16_t* suh, uint16_t* out)
{
    if (k % 128) return -1;
    for (int64_t r = 0; r < m; ++r)
        for (int b = 0; b < k; b += 128) {
            double v[128];
            for (int i = 0; i < 128; ++i)
                v[i] = rnd16(exl3cpu_f16_to_f64(x[r * k + b + i]) * exl3cpu_f16_to_f64(suh[b + i]));
            wht128(v);
            for (int i = 0; i < 128; ++i) out[r * k + b + i] = exl3cpu_f64_to_f16(v[i] * R_SCALE);
        }
    return 0;
}

/* y = fp16(fp16(Had128(c)) * svh) */
int exl3cpu_had_out(const uint16_t* c, int m, int n, const uint16_t* svh, uint16_t* out)
{
    if (n % 128) return -1;
    for (int64_t r = 0; r < m; ++r)
        for (int b = 0; b < n; b += 128) {
            double v[128];
            for (int i = 0; i < 128; ++i) v[i] = exl3cpu_f16_to_f64(c[r * n + b + i]);
            wht128(v);
            for (int i = 0; i < 128; ++i)
                out[r * n + b + i] = exl3cpu_f64_to_f16(rnd16(v[i] * R_SCALE) * exl3cpu_f16_to_f64(svh[b + i]));
        }
    return 0;
}

/* ---------------------------------------------------------------- faithful linear (oracle gemv_mul1 :307) */
int exl3cpu_linear(const uint16_t* x, int m, int k, int n, const uint16_t* trellis, int bits, int cb,
                   const uint16_t* suh, const uint16_t* svh, uint16_t* y, int threads)
{
    if (m < 1 || k % 128 || n % 128 || bits < 1 || bits > 8 || cb < 0 || cb > 2) return -1;
    const int kt = k / 16, nt = n / 16, per = 16 * bits;
    uint16_t* ah = (uint16_t*) malloc((size_t) m * k * 2);
    double* ahd = (double*) malloc((size_t) m * k * sizeof(double));
    uint16_t* c = (uint16_t*) malloc((size_t) m * n * 2);
    if (!ah || !ahd || !c) { free(ah); free(ahd); free(c); return -2; }
    exl3cpu_had_in(x, m, k, suh, ah);
    for (int64_t i = 0; i < (int64_t) m * k; ++i) ahd[i] = exl3cpu_f16_to_f64(ah[i]);
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 4)
#endif
    for (int b = 0; b < nt; ++b) {
        uint16_t tile[256];
        double wt[256];
        double acc[16 * 32];                      /* up to 32 rows per pass */
        for (int r0 = 0; r0 < m; r0 += 32) {
            int mr = m - r0 < 32 ? m - r0 : 32;
            memset(acc, 0, sizeof(acc));
            for (int a = 0; a < kt; ++a) {
                exl3cpu_decode_tile(trellis + ((int64_t) a * nt + b) * per, bits, cb, tile);
                for (int i = 0; i < 256; ++i) wt[i] = exl3cpu_f16_to_f64(tile[i]);
                for (int r = 0; r < mr; ++r) {
                    const double* av = ahd + (int64_t) (r0 + r) * k + a * 16;
                    double* ac = acc + r * 16;
                    for (int kr = 0; kr < 16; ++kr) {
                        double s = av[kr];
                        const double* wr = wt + kr * 16;
                        for (int cc = 0; cc < 16; ++cc) ac[cc] += s * wr[cc];
                    }
                }
            }
            for (int r = 0; r < mr; ++r)
                for (int cc = 0; cc < 16; ++cc)
                    c[(int64_t) (r0 + r) * n + b * 16 + cc] = exl3cpu_f64_to_f16(acc[r * 16 + cc]);
        }
    }
    exl3cpu_had_out(c, m, n, svh, y);
    free(ah); free(ahd); free(c);
    return 0;
}

int exl3cpu_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
