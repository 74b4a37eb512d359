/*
 * morphocore CPU oracle — TEST INFRASTRUCTURE ONLY.
 *
 * A plain C restatement of the reference CPU extension's algorithm for the csrc hot path
 * (/root/reference/morphocore/functional/csrc/cpp): dilation / erosion forward and backward with
 * index capture, smorph forward and backward, merges MAX, MIN, ADD, AVERAGE, IDENTITY, in float and
 * double. Every function names the reference file:line it follows. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load this library, and only as a checker or as the reported CPU
 * baseline: it is never part of the product path.
 *
 * Parity pins (see tests/test_oracle.py):
 *   forward values and indices: numpy brute force of the reference tests' own construction
 *     (tests/functional/utils.py:6-49, test_padding.py:9-45) and the reference's known-answer tests;
 *   gradients: float64 finite differences (gradcheck) and the closed-form routing on dyadic inputs;
 *   smorph: alpha -> +-inf limits (dilation / erosion), alpha = 0 (plain mean of valid taps), float64
 *     finite differences including alpha;
 *   all of it against the reference's own CPU extension built into oracle/_ref, where present.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off).
 */
#include <float.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum
{
    ORACLE_DILATION = 0,
    ORACLE_EROSION = 1
};

/* Same values as MORPHO_MERGE (morpho_op_enum.hpp:17-25) and merge_enum.py:4-11. */
enum
{
    ORACLE_MAX = 0,
    ORACLE_MIN = 1,
    ORACLE_ADD = 2,
    ORACLE_AVERAGE = 3,
    ORACLE_SMOOTH = 4,
    ORACLE_IDENTITY = 5
};

typedef struct
{
    int64_t b, cin, cout, cw, h, w, kh, kw;
} oracle_geom;

/* Multiply-adds that the reference's compiled AVX2+FMA kernels fuse (GCC contracts a * b + c in
 * C++ by default, and morpho_cpu_dispatch picks the "avx2,fma" build on any AVX2 host) are written
 * here as explicit fma calls, so that the oracle reproduces that binary and not a compiler choice.
 *
 * The reference's vector exponential, restated for one lane (morpho_cpu_simd.hpp:127-169):
 * Cody-Waite reduction x = n ln2 + r with ln2 split in a high and a low part, exp(r) by its Taylor
 * series in Horner form (degree 7 for float, 13 for double, coefficients 1/k! built by repeated
 * division in the element type), 2^n written into the exponent bits. Inputs below the log of the
 * smallest normal return 0; inputs above the overflow threshold are clamped to it. */
static inline float oracle_exp_f32(float x)
{
    const float max_input = 88.0f, min_input = -87.33654f;
    const float log2e = 1.44269504088896340736f;
    const float ln2_hi = 0.693359375f, ln2_lo = -2.12194440e-4f;
    const float round_magic = 12582912.0f; /* 1.5 * 2^23: adding then subtracting rounds to an integer */
    const int underflow = x < min_input;
    float xc = x > max_input ? max_input : x;
    xc = underflow ? min_input : xc;
    const float n = fmaf(xc, log2e, round_magic) - round_magic;
    const float r = fmaf(-n, ln2_lo, fmaf(-n, ln2_hi, xc));
    float inv_fact[8];
    inv_fact[0] = 1.0f;
    for (int k = 1; k <= 7; k++) inv_fact[k] = inv_fact[k - 1] / (float)k;
    float p = inv_fact[7];
    for (int k = 6; k >= 0; k--) p = fmaf(p, r, inv_fact[k]);
    if (underflow) return 0.0f;
    if (isnan(n)) return n;
    const int32_t bits = ((int32_t)n + 127) << 23;
    float scale;
    memcpy(&scale, &bits, sizeof(scale));
    return p * scale;
}

static inline double oracle_exp_f64(double x)
{
    const double max_input = 709.0, min_input = -708.39641;
    const double log2e = 1.44269504088896340736;
    const double ln2_hi = 6.93145751953125e-1, ln2_lo = 1.42860682030941723212e-6;
    const double round_magic = 6755399441055744.0; /* 1.5 * 2^52 */
    const int underflow = x < min_input;
    double xc = x > max_input ? max_input : x;
    xc = underflow ? min_input : xc;
    const double n = fma(xc, log2e, round_magic) - round_magic;
    const double r = fma(-n, ln2_lo, fma(-n, ln2_hi, xc));
    double inv_fact[14];
    inv_fact[0] = 1.0;
    for (int k = 1; k <= 13; k++) inv_fact[k] = inv_fact[k - 1] / (double)k;
    double p = inv_fact[13];
    for (int k = 12; k >= 0; k--) p = fma(p, r, inv_fact[k]);
    if (underflow) return 0.0;
    if (isnan(n)) return n;
    const int64_t bits = ((int64_t)n + 1023) << 52;
    double scale;
    memcpy(&scale, &bits, sizeof(scale));
    return p * scale;
}

/* Exported for the oracle's own tests of the exponential. */
float oracle_expf(float x) { return oracle_exp_f32(x); }
double oracle_exp(double x) { return oracle_exp_f64(x); }

/* The exponential over an array (y[j] = exp(x[j])), for bitwise comparisons of many arguments. */
/* Test helper, no counterpart in the reference: while set, the smorph backwards accumulate the magnitude
 * of every grad_weight, grad_alpha and grad_beta term instead of the term (each routed tap's |c|, each
 * pixel's |pg (v - ref)(v - out)| and |q (c - ref)(c - out) g|, in ACC), giving the sum of the terms'
 * magnitudes: the scale against which the float32 error of those sums, whose terms can cancel far below
 * their size, is measured. */
static int oracle_abs_terms = 0;
void oracle_set_abs_terms(int on) { oracle_abs_terms = on; }
#define TERM(v) (oracle_abs_terms ? fabsl((long double)(v)) : (long double)(v))

void oracle_expf_array(const float* x, float* y, int64_t n)
{
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < n; j++) y[j] = oracle_exp_f32(x[j]);
}

void oracle_exp_array(const double* x, double* y, int64_t n)
{
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < n; j++) y[j] = oracle_exp_f64(x[j]);
}

#define T float
#define ACC double
#define SFX f32
#define T_LOWEST (-FLT_MAX)
#define T_MAX FLT_MAX
#define T_INF ((float)INFINITY)
#define EXP_T oracle_exp_f32
#define FMA_T fmaf
#include "morpho_oracle_impl.h"
#undef T
#undef ACC
#undef SFX
#undef T_LOWEST
#undef T_MAX
#undef T_INF
#undef EXP_T
#undef FMA_T

#define T double
#define ACC long double
#define SFX f64
#define T_LOWEST (-DBL_MAX)
#define T_MAX DBL_MAX
#define T_INF ((double)INFINITY)
#define EXP_T oracle_exp_f64
#define FMA_T fma
#include "morpho_oracle_impl.h"
#undef T
#undef ACC
#undef SFX
#undef T_LOWEST
#undef T_MAX
#undef T_INF
#undef EXP_T
#undef FMA_T
