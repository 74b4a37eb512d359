// Definitions shared by the smorph kernels (smorph.hip: any structuring-element size; smorph_static.hip:
// the common square sizes in float32).
#pragma once

#include "launch.hpp"

namespace mca
{

// The exponential of the reference's CPU smorph (morpho_cpu_simd.hpp:127-169), one lane at a time:
// Cody-Waite reduction x = n ln2 + r with ln2 split in a high and a low part, exp(r) by its Taylor
// series in Horner form with fused multiply-adds (degree 7 for float, 13 for double, coefficients
// 1/k! by repeated division in the element type), 2^n assembled in the exponent bits; inputs below
// the log of the smallest normal give 0 (exp_ref below).
// The kernels need these exact roundings: the smorph gradients scale the rounding error of each
// pair's output by alpha, so an exponential that differs by an ulp (even a correctly rounded one)
// moves float32 gradients by ~1e-6 relative at |alpha| = 20.
template <typename T>
struct ExpConsts;

template <>
struct ExpConsts<float>
{
    using Bits = int32_t;
    static constexpr int degree = 7;
    static constexpr float max_input = 88.0f, min_input = -87.33654f;
    static constexpr float log2e = 1.44269504088896340736f;
    static constexpr float ln2_hi = 0.693359375f, ln2_lo = -2.12194440e-4f;
    static constexpr float magic = 12582912.0f;  // 1.5 * 2^23: adding then subtracting rounds to an integer
    static constexpr int mant = 23, bias = 127;
};

template <>
struct ExpConsts<double>
{
    using Bits = int64_t;
    static constexpr int degree = 13;
    static constexpr double max_input = 709.0, min_input = -708.39641;
    static constexpr double log2e = 1.44269504088896340736;
    static constexpr double ln2_hi = 6.93145751953125e-1, ln2_lo = 1.42860682030941723212e-6;
    static constexpr double magic = 6755399441055744.0;  // 1.5 * 2^52
    static constexpr int mant = 52, bias = 1023;
};

template <typename T, int K>
struct InvFact
{
    static constexpr T value = InvFact<T, K - 1>::value / T(K);
};

template <typename T>
struct InvFact<T, 0>
{
    static constexpr T value = T(1);
};

template <typename T, int K>
__device__ __forceinline__ T horner(T r)
{
    if constexpr (K == ExpConsts<T>::degree)
        return InvFact<T, K>::value;
    else
        return fma(horner<T, K + 1>(r), r, InvFact<T, K>::value);
}

// The target the reference's MAX / MIN backward compares the pair outputs with: the extremum over the
// channels starting from channel 0's pair output (smorph_cpu_kernels.hxx:491-503), which is the
// forward's output (merged from lowest() / max(), where NaN never wins) unless channel 0's output is
// NaN: then NaN, and no pair is a winner.
template <typename T>
__device__ __forceinline__ T smorph_merge_target(T forward_out, T channel0_out)
{
    return channel0_out != channel0_out ? channel0_out : forward_out;
}

// Tolerance within which a channel counts as a MAX / MIN winner (reference: smorph.cu:7-9,
// smorph_cpu_kernels.hxx:622-627). `out` is the pair output rounded to T, as the reference stores it:
// the subtraction is never fused with a caller's W * (1 / S) (an unrounded product moves d by up to
// half a unit of the output's last place, which decides a pair lying that close to the tolerance
// differently from the reference, and from the routing's own rounded test).
template <typename T>
__device__ __forceinline__ bool is_winner(T out, T target)
{
#pragma clang fp contract(off)
    const T d = out - target;
    const T tol = T(1e-6);
    return d < tol && d > -tol;
}

template <typename T>
struct SmorphFwdParams
{
    const T* __restrict__ x;
    const T* __restrict__ w;
    const T* __restrict__ alpha;
    T* __restrict__ out;           // forward output, or the winner counts in STATS mode
    const T* __restrict__ target;  // STATS mode: the forward output
    T* __restrict__ tout;          // STATS mode: the backward's merge target (see smorph_merge_target)
    // Saved pair statistics (float32 static kernels; null: none saved): ref, then 1 / S, then W / S of
    // every (batch element, output channel, pair, pixel), `nstat` values each.
    float* __restrict__ pstats;
    int64_t nstat;
    // SMOOTH merge: every pair's output c, [B, Cout, Cin, H, W], merged afterwards by
    // smorph_soft_merge_kernel.
    T* __restrict__ pout;
    Geom g;
    Tiling t;
    int average;
};

// Half of exp(r)'s Taylor polynomial: Horner with every coefficient halved (exact), so each step is
// exactly half of horner<T, K>'s (scaling by a power of two commutes with rounding).
template <typename T, int K>
__device__ __forceinline__ T horner_half(T r)
{
    if constexpr (K == ExpConsts<T>::degree)
        return InvFact<T, K>::value * T(0.5);
    else
        return fma(horner_half<T, K + 1>(r), r, InvFact<T, K>::value * T(0.5));
}

// The same exponential for the arguments the smorph kernels pass, alpha (v - ref) with ref the
// extremum of the window: never positive, or NaN. Bit for bit equal to exp_t on (-inf, max_input]
// (checked exhaustively for float32 on [-200, 0], NaN and -inf); a NaN argument gives NaN, as in the
// reference (whose range checks let NaN through), and the upper clamp is dropped since no argument
// reaches it. `lo` is the lower clamp, min_input (a caller may hold it in a register, which makes the
// comparison a register-only one). Arranged for fewer instructions than exp_t:
//  * below `lo` the result is selected to 0 at the end, so the argument needs no clamp (what the
//    reduction computes there is discarded);
//  * the rounding constant carries bias + 1 (even, and in the same binade, so every rounding is
//    unchanged): the low bits of nm hold n + bias + 1, and shifting them into the exponent field is
//    2^(n + 1) with no add; the halved polynomial compensates, and (p / 2) 2^(n + 1) is the same
//    exact product as p 2^n, rounded once. n + bias + 1 stays in [2, bias + 1] for n in
//    [log2(min normal), 0].
// exp_ref of an argument scaled by alpha = 0, which can only be +-0, -inf or NaN ((v - ref) * 0, less
// a masked tap's +inf): exactly what exp_ref returns for those (1, 0 and NaN), in three instructions.
template <typename T>
__device__ __forceinline__ T exp_ref_zero_alpha(T x, T lo)
{
    return x < lo ? T(0) : x + T(1);
}

template <typename T>
__device__ __forceinline__ T exp_ref(T x, T lo = ExpConsts<T>::min_input)
{
    using C = ExpConsts<T>;
    using Bits = typename C::Bits;
    constexpr T magic = C::magic + T(C::bias + 1);
    const bool under = x < lo;
    const T nm = fma(x, C::log2e, magic);
    const T n = nm - magic;
    const T r = fma(-n, C::ln2_lo, fma(-n, C::ln2_hi, x));
    const T ph = horner_half<T, 0>(r);
    const T scale = __builtin_bit_cast(T, (Bits)((uint64_t)__builtin_bit_cast(Bits, nm) << C::mant));
    const T e = ph * scale;
    return under ? T(0) : e;
}

// exp(x) for the routing of gradients only, from the hardware base-2 exponential (v_exp_f32, one
// transcendental instruction) of x log2(e): relative error about 1.2e-7 (the instruction's) plus
// |x| 7.5e-8 (the rounding of the product and of log2(e)), i.e. within 5e-7 wherever e > 1e-3, and a
// far smaller absolute error below. The routing scales each e by 1 / S (S >= 1 holds the extremum's
// e = 1), so gradients move by a few 1e-7 of their size at most: inside the 1e-6 contract. Never used
// where S, W or the output are formed: those need the reference's exponential bit for bit (exp_ref),
// since the gradients amplify an output's rounding by alpha. -inf gives 0 and NaN gives NaN, as
// exp_ref; 2^x below the normal range may give a subnormal where exp_ref gives 0.
__device__ __forceinline__ float exp_route(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896340736f); }

// exp_ref for an argument known to be at or above its lower threshold (or NaN): the same bits
// without the final select.
template <typename T>
__device__ __forceinline__ T exp_ref_above(T x)
{
    using C = ExpConsts<T>;
    using Bits = typename C::Bits;
    constexpr T magic = C::magic + T(C::bias + 1);
    const T nm = fma(x, C::log2e, magic);
    const T n = nm - magic;
    const T r = fma(-n, C::ln2_lo, fma(-n, C::ln2_hi, x));
    const T ph = horner_half<T, 0>(r);
    const T scale = __builtin_bit_cast(T, (Bits)((uint64_t)__builtin_bit_cast(Bits, nm) << C::mant));
    return ph * scale;
}

// Whether a wave-uniform alpha is zero (+0 or -0), as a scalar condition (a branch, not a mask).
__device__ __forceinline__ bool alpha_is_zero(float a)
{
    return (__builtin_amdgcn_readfirstlane(__builtin_bit_cast(unsigned, a)) & 0x7fffffffu) == 0u;
}

template <typename T>
struct SmorphBwdParams
{
    const T* __restrict__ x;
    const T* __restrict__ w;
    const T* __restrict__ alpha;
    const T* __restrict__ out;     // forward output (MAX / MIN)
    const T* __restrict__ counts;  // winner counts (MAX / MIN)
    const T* __restrict__ gout;
    T* __restrict__ gin;
    T* __restrict__ part_w;
    T* __restrict__ part_a;
    const float* __restrict__ pstats;  // the forward's saved pair statistics, or null (recomputed)
    int64_t nstat;
    // Generic kernel for elements whose tile and grad_input copy exceed the LDS: grad_input summed in
    // global memory, [B, Cin, H, W] double (grad_input itself for double tensors), else null.
    Acc* __restrict__ gacc;
    // SMOOTH merge (smorph_scm): beta per output channel, the forward's soft-merge statistics (ref,
    // then 1 / sum, [B, Cout, H, W] each; `out` holds the merged output), and the grad_beta partials
    // [slot][Cin][Cout].
    const T* __restrict__ beta;
    const T* __restrict__ sstats;
    T* __restrict__ part_b;
    Geom g;
    Tiling t;
    int nstrips;
    int tps;
    int ncopy;
    int npairs;
    T scale;
};

// Structuring-element sizes with static-size smorph kernels (smorph_static.hip).
template <typename T>
inline bool smorph_static_supported(const Geom& g)
{
    if constexpr (sizeof(T) != 4)
        return false;
    else
        return g.KH == g.KW && (g.KH == 3 || g.KH == 5 || g.KH == 7 || g.KH == 11) && g.plane() <= 0x7fffffff;
}

// The static backward up to 5x5 sums each workgroup's grad_weight / grad_alpha (and, for the SMOOTH
// merge, grad_beta) partials over its tiles in LDS (at most this many values: output channels x
// (taps + 1 or 2)) and stores them once, every entry of its slot; otherwise it adds each tile's sums
// to the zero-filled slot with atomics. (At 7x7 the 12.8 KiB they need would hold the kernel to four
// workgroups per CU; it runs five. The two-row kernel at 5x5 keeps seven per CU with 64 x 26 values,
// not with 64 x 27.)
__host__ __device__ constexpr int smorph_lds_partials(bool smooth) { return smooth ? 64 * 27 : 64 * 26; }

__host__ __device__ inline bool smorph_bwd_lds_partials(const Geom& g, bool identity, bool smooth = false)
{
    const int K = g.KH * g.KW;
    return K <= 25 && (identity ? 1 : g.Cout) * (K + (smooth ? 2 : 1)) <= smorph_lds_partials(smooth);
}

// Pair statistics the float32 static forward can save for the backward: ref (the window's extremum),
// 1 / S and W / S of every channel pair at every output pixel, index
// ((b * Cout + o) * pairs_per_output + i') * H * W + pixel (i' = i, or 0 for IDENTITY). 0 when the
// configuration has no static kernels.
template <typename T>
inline int64_t smorph_stats_count(int merge, const Geom& g)
{
    if (!smorph_static_supported<T>(g)) return 0;
    return (int64_t)g.B * g.Cout * (merge == MERGE_IDENTITY ? 1 : g.Cin) * g.plane();
}

// Launchers of the static-size kernels (smorph_static.hip), float32; a non-null `pstats` selects the
// forward that saves the pair statistics and the backward that reads them.
hipError_t launch_smorph_fwd_static(int mk, bool stats, const SmorphFwdParams<float>& p, hipStream_t stream);
hipError_t launch_smorph_bwd_static(int mk, const SmorphBwdParams<float>& p, hipStream_t stream);
// MAX / MIN merge target and winner counts of every output pixel from the saved W / S values (`outp`).
hipError_t launch_smorph_counts_saved(const float* outp, const float* out, float* counts, float* target, const Geom& g, hipStream_t stream);

}  // namespace mca
