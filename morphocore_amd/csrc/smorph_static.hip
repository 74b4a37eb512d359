// Smorph forward and backward for the common square structuring elements (3, 5, 7, 11) in float32
// (reference semantics: smorph_cpu_kernels.hxx:14-229, 387-638).
//
// Same arithmetic as the any-size kernels of smorph.hip, organised for gfx950's VALU:
//  * every tap loop is unrolled, and the pair's structuring element and alpha are read from LDS
//    into vector registers: a VALU operation that reads a scalar register issues at about half the
//    rate of one whose operands are vector registers or constants (measured on MI355X);
//  * one output pixel per lane, one output row per wave: the validity of a tap row is uniform over
//    the wave (a scalar branch), only the KW tap columns carry per-lane masks, and tiles whose
//    windows lie inside the image take a path without any check. Out-of-image taps are excluded by
//    position, as in the reference (SmorphBlockMask, smorph_valid_rows); an in-image NaN propagates
//    as in the reference;
//  * the forward can save each pair's ref, 1 / S and W / S, and the backward from them (two output
//    rows per wave) evaluates each exponential once; the backward that recomputes them keeps every
//    tap's e in registers (up to 7x7) between the pass that forms S and W and the pass that routes
//    the gradient (11x11 keeps its first two rows and re-evaluates the rest: 121 registers would
//    cost more waves than the exponentials cost VALU);
//  * every lane of a wave routes the same tap at once: a row of KW taps is summed per tile column
//    across the wave (a DPP shift per tap) before one LDS atomic per row, and the grad_weight LDS
//    atomics hit lane-striped copies (no bank conflicts). LDS atomics cost per instruction, not per
//    active lane (measured), so partial sums replace instructions, never lanes.
#include "smorph_common.hpp"

namespace mca
{

// Copies of each grad_weight / grad_alpha bin of the backward, one per lane of a half wave.
// 11x11 takes 16 (two lanes of a half wave share each copy, 2.4x the cost of an LDS add): its 122 bins
// then fit five workgroups per CU, measured 16% faster than three workgroups with 32 copies.
constexpr int smorph_bin_copies(int K) { return K > 49 ? 16 : 32; }

namespace
{

__device__ __forceinline__ float smorph_init(bool dilation_like)
{
    return dilation_like ? -std::numeric_limits<float>::infinity() : std::numeric_limits<float>::infinity();
}

// Validity of this wave's tap rows (bit kh: the input row lies in the image, uniform over the wave)
// and of this lane's tap columns, as a penalty: 0 in the image, +inf outside. Masking by arithmetic
// (v - pen never wins a max, an exponential's argument minus pen gives e = 0) keeps the masked taps
// branch free: a select between a loaded value and a constant is turned into a branch around the
// load by the compiler.
template <int KH, int KW>
struct TapMask
{
    unsigned rows;
    float pen[KW];
    float keep[KW];  // 1 in the image, 0 outside

    __device__ __forceinline__ void init(const Geom& g, int h, int wc)
    {
        unsigned r = 0;
#pragma unroll
        for (int kh = 0; kh < KH; ++kh)
        {
            const int y = h + KH / 2 - kh;
            r |= (y >= 0 && y < g.H) ? 1u << kh : 0u;
        }
        rows = __builtin_amdgcn_readfirstlane(r);
#pragma unroll
        for (int kw = 0; kw < KW; ++kw)
        {
            const int c = wc + KW / 2 - kw;
            pen[kw] = c >= 0 && c < g.W ? 0.0f : std::numeric_limits<float>::infinity();
            keep[kw] = c >= 0 && c < g.W ? 1.0f : 0.0f;
        }
    }
    __device__ __forceinline__ bool row(int kh) const { return (rows >> kh) & 1u; }
};

// Pass 1 of a pair: the extremum of the valid taps (NaN never wins, as with the reference's strict
// scan). xb: this lane's tap-0 input in the staged tile; tap (kh, kw) reads xb[-(kh * COLS + kw)].
template <int KH, int KW, bool MASKED>
__device__ __forceinline__ float smorph_ref(const float* xb, const float* wl, bool dil, const TapMask<KH, KW>& tm)
{
    constexpr int COLS = TILE_W + KW - 1;
    float ref = smorph_init(dil);
    if (dil)
    {
#pragma unroll
        for (int kh = 0; kh < KH; ++kh)
        {
            if (MASKED && !tm.row(kh)) continue;
#pragma unroll
            for (int kw = 0; kw < KW; ++kw)
            {
                float v = xb[-(kh * COLS + kw)] + wl[kh * KW + kw];
                if constexpr (MASKED) v = v - tm.pen[kw];  // -inf (or NaN) outside: never wins
                ref = fmaxf(ref, v);
            }
        }
    }
    else
    {
#pragma unroll
        for (int kh = 0; kh < KH; ++kh)
        {
            if (MASKED && !tm.row(kh)) continue;
#pragma unroll
            for (int kw = 0; kw < KW; ++kw)
            {
                float v = xb[-(kh * COLS + kw)] + wl[kh * KW + kw];
                if constexpr (MASKED) v = v + tm.pen[kw];
                ref = fminf(ref, v);
            }
        }
    }
    return ref;
}

// Pass 1 of a pair on an interior tile: the extremum `ref` (as smorph_ref) and the opposite one,
// `far`, so that (far - ref) * a bounds every tap's exponential argument from below (the taps round
// (v - ref) * a the same way, and rounding is monotone).
// MASKED: ref over the in-image taps only (as smorph_ref), far over every tap of the in-image rows,
// the out-of-image columns included (their staged x is 0): it bounds the arguments of all the taps
// the sums evaluate.
template <int KH, int KW, bool MASKED>
__device__ __forceinline__ float smorph_ref_far(const float* xb, const float* wl, bool dil, const TapMask<KH, KW>& tm, float& far)
{
    constexpr int COLS = TILE_W + KW - 1;
    float ref = smorph_init(dil), opp = smorph_init(!dil);
    if (dil)
    {
#pragma unroll
        for (int kh = 0; kh < KH; ++kh)
        {
            if (MASKED && !tm.row(kh)) continue;
#pragma unroll
            for (int kw = 0; kw < KW; ++kw)
            {
                const float v = xb[-(kh * COLS + kw)] + wl[kh * KW + kw];
                ref = fmaxf(ref, MASKED ? v - tm.pen[kw] : v);
                opp = fminf(opp, v);
            }
        }
    }
    else
    {
#pragma unroll
        for (int kh = 0; kh < KH; ++kh)
        {
            if (MASKED && !tm.row(kh)) continue;
#pragma unroll
            for (int kw = 0; kw < KW; ++kw)
            {
                const float v = xb[-(kh * COLS + kw)] + wl[kh * KW + kw];
                ref = fminf(ref, MASKED ? v + tm.pen[kw] : v);
                opp = fmaxf(opp, v);
            }
        }
    }
    far = opp;
    return ref;
}

}  // namespace

// ------------------------------------------------------------------------------------------------
// Forward: one workgroup per (batch element, output channel, 64 x 4 tile), walking the input
// channels with the next channel's tile prefetched into registers.
// ------------------------------------------------------------------------------------------------

// Pass 2 of a pair: S and W in tap order (kh, then kw), W fused as in the reference's AVX2 build.
// ZA: the pair's alpha is zero (every e is 1 on an in-image tap of finite v).
// SAFE: no tap's argument lies below the exponential's lower threshold and every v is finite (checked
// by the caller for the whole wave): exp_ref's final select never fires and is left out, and with
// ZA every e is exactly 1 (S counts the taps, W sums the v).
template <int KH, int KW, bool MASKED, bool ZA, bool SAFE = false>
__device__ __forceinline__ void smorph_sums(const float* xb, const float* wl, float a, float ref, const TapMask<KH, KW>& tm, float& S, float& Wsum)
{
#pragma clang fp contract(off)  // fused only where the reference fuses (written as fmaf)
    constexpr int COLS = TILE_W + KW - 1;
    float lo = ExpConsts<float>::min_input;
    asm volatile("" : "+v"(lo));  // the exponential's clamp in a register: register-only comparisons
    float s = 0.0f, wsum = 0.0f;
#pragma unroll
    for (int kh = 0; kh < KH; ++kh)
    {
        if (MASKED && !tm.row(kh)) continue;
#pragma unroll
        for (int kw = 0; kw < KW; ++kw)
        {
            const float v = xb[-(kh * COLS + kw)] + wl[kh * KW + kw];
            // An out-of-image tap adds e = 0 (its staged x is 0, so v and the argument are finite, and
            // the argument less +inf is -inf): S + 0 and fma(0, v, W) leave both sums exactly as
            // skipping it does.
            if constexpr (SAFE && ZA)
            {
                // e = 1 in the image, 0 outside: S + e and fma(e, v, W) with one rounding each.
                s = s + (MASKED ? tm.keep[kw] : 1.0f);
                wsum = MASKED ? fmaf(tm.keep[kw], v, wsum) : wsum + v;
                continue;
            }
            if constexpr (SAFE)
            {
                // Every argument lies at or above the threshold and is finite; an out-of-image tap's e
                // is multiplied by 0 (exactly 0: its v is finite).
                const float ef = exp_ref_above((v - ref) * a);
                const float e = MASKED ? ef * tm.keep[kw] : ef;
                s = s + e;
                wsum = fmaf(e, v, wsum);
                continue;
            }
            const float arg = MASKED ? (v - ref) * a - tm.pen[kw] : (v - ref) * a;
            const float e = ZA ? exp_ref_zero_alpha(arg, lo) : exp_ref(arg, lo);
            s = s + e;  // unfused, as in the reference (e is rounded before the sum)
            wsum = fmaf(e, v, wsum);
        }
    }
    S = s;
    Wsum = wsum;
}

// SAVE: also store each pair's ref, 1 / S and W / S at every in-image pixel (p.pstats), which the
// backward then reads instead of recomputing them.
// Waves per SIMD requested: seven up to 7x7, five at 11x11 (without a request the compiler takes more
// registers for fewer waves, ~2% slower; eight spill at 7x7 and measured 0.6% slower than seven).
template <int MK, int KH, int KW, bool STATS, bool SAVE>
__global__ __launch_bounds__(BLOCK) __attribute__((amdgpu_waves_per_eu(KH * KW > 49 ? 5 : 7, 8))) void smorph_fwd_static(
    const SmorphFwdParams<float> p)
{
    constexpr int K = KH * KW, PH = KH / 2, PW = KW / 2;
    constexpr int TH = NWAVES, ROWS = TH + KH - 1, COLS = TILE_W + KW - 1, ELEMS = ROWS * COLS;
    constexpr int NS = (ELEMS + BLOCK - 1) / BLOCK;
    __shared__ float tile[2][ELEMS];
    // The pair's structuring element, then its alpha; rows padded to 16 bytes so the taps load as
    // 128-bit broadcast reads.
    __shared__ __align__(16) float wl[2][(K + 4) & ~3];
    const Geom g = p.g;
    const Tiling t = p.t;
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    int work = xcd_work_index(blockIdx.x, gridDim.x);
    const int o = work % g.Cout;
    work /= g.Cout;
    const int tx = work % t.ntx;
    work /= t.ntx;
    const int ty = work % t.nty;
    const int b = work / t.nty;
    const int h0 = ty * TH, w0 = tx * TILE_W;
    const int y0 = h0 + PH - (KH - 1), x0 = w0 + PW - (KW - 1);
    const int64_t plane = g.plane();
    const int h = h0 + wave, wc = w0 + lane;
    const bool in = h < g.H && wc < g.W;
    const bool interior = y0 >= 0 && y0 + ROWS <= g.H && x0 >= 0 && x0 + COLS <= g.W;
    TapMask<KH, KW> tm;
    tm.init(g, h, wc);

    // Staging plan, the same for every input channel: the clamped in-image offset of each element
    // this thread stages, and whether it lies in the image (else it stages 0, never read unmasked).
    int off[NS];
    bool ok[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j)
    {
        const int idx = min((int)threadIdx.x + j * BLOCK, ELEMS - 1);
        const int ly = idx / COLS, lx = idx - ly * COLS;
        const int y = y0 + ly, x = x0 + lx;
        ok[j] = y >= 0 && y < g.H && x >= 0 && x < g.W;
        off[j] = clampi(y, 0, g.H - 1) * g.W + clampi(x, 0, g.W - 1);
    }
    const int i_begin = MK == MK_IDENT ? o : 0;
    const int i_end = MK == MK_IDENT ? o + 1 : g.Cin;
    const int wt = min((int)threadIdx.x, K);
    float pre[NS], wpre;
    auto load = [&](int i) {
        i = min(i, i_end - 1);
        const float* __restrict__ xp = p.x + ((int64_t)b * g.Cin + i) * plane;
#pragma unroll
        for (int j = 0; j < NS; ++j) pre[j] = xp[off[j]];
        const int pair = MK == MK_IDENT ? o : o * g.Cin + i;
        wpre = wt < K ? p.w[((int64_t)o * g.Cw + (MK == MK_IDENT ? 0 : i)) * K + wt] : p.alpha[pair];
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int j = 0; j < NS; ++j)
        {
            const int idx = threadIdx.x + j * BLOCK;
            if (j < NS - 1 || idx < ELEMS) tile[buf][idx] = ok[j] ? pre[j] : 0.0f;
        }
        if (threadIdx.x <= K) wl[buf][threadIdx.x] = wpre;
    };

    float m = STATS ? 0.0f : (MK == MK_MAX ? lowest_of<float>() : (MK == MK_MIN ? max_of<float>() : 0.0f));
    float tgt = 0.0f;
    if constexpr (STATS)
    {
        if (in) tgt = p.target[((int64_t)b * g.Cout + o) * plane + (int64_t)h * g.W + wc];
    }

    load(i_begin);
    store(0);
    __syncthreads();
    for (int i = i_begin; i < i_end; ++i)
    {
        const int buf = (i - i_begin) & 1;
        load(i + 1);  // in flight while this channel computes (the last one re-reads itself)
        const float* xb = &tile[buf][(wave + KH - 1) * COLS + lane + KW - 1];
        const float* w = wl[buf];
        const float a = w[K];
        const bool dil = a >= 0.0f;
        const bool za = alpha_is_zero(a);
        float ref, S, Wsum;
        // Every lane's smallest argument at or above the exponential's threshold and every v finite
        // (ref and far finite): the wave takes the select-free sums, bit for bit the same.
        auto safe_wave = [&](float far) {
            const float bound = (far - ref) * a;
            const bool ok = bound >= ExpConsts<float>::min_input && fabsf(far) <= 3.40282347e38f && fabsf(ref) <= 3.40282347e38f;
            return __builtin_amdgcn_uicmp((unsigned)!ok, 0u, 33) == 0;  // no lane fails
        };
        if (interior)
        {
            float far;
            ref = smorph_ref_far<KH, KW, false>(xb, w, dil, tm, far);
            const bool safe = safe_wave(far);
            if (za)
            {
                if (safe)
                    smorph_sums<KH, KW, false, true, true>(xb, w, a, ref, tm, S, Wsum);
                else
                    smorph_sums<KH, KW, false, true>(xb, w, a, ref, tm, S, Wsum);
            }
            else
            {
                if (safe)
                    smorph_sums<KH, KW, false, false, true>(xb, w, a, ref, tm, S, Wsum);
                else
                    smorph_sums<KH, KW, false, false>(xb, w, a, ref, tm, S, Wsum);
            }
        }
        else if constexpr (KW > 7)
        {
            // 11x11: the border tiles keep the select (the keep factors of the select-free masked sums
            // spill registers there: 60 bytes per lane, measured 1.5% slower on configs[4]).
            ref = smorph_ref<KH, KW, true>(xb, w, dil, tm);
            if (za)
                smorph_sums<KH, KW, true, true>(xb, w, a, ref, tm, S, Wsum);
            else
                smorph_sums<KH, KW, true, false>(xb, w, a, ref, tm, S, Wsum);
        }
        else
        {
            float far;
            ref = smorph_ref_far<KH, KW, true>(xb, w, dil, tm, far);
            const bool safe = safe_wave(far);
            if (za)
            {
                if (safe)
                    smorph_sums<KH, KW, true, true, true>(xb, w, a, ref, tm, S, Wsum);
                else
                    smorph_sums<KH, KW, true, true>(xb, w, a, ref, tm, S, Wsum);
            }
            else
            {
                if (safe)
                    smorph_sums<KH, KW, true, false, true>(xb, w, a, ref, tm, S, Wsum);
                else
                    smorph_sums<KH, KW, true, false>(xb, w, a, ref, tm, S, Wsum);
            }
        }
        const float inv = 1.0f / S;
        if constexpr (STATS)
        {
            if (i == i_begin) tgt = smorph_merge_target(tgt, Wsum * inv);
        }
        if constexpr (SAVE)
        {
            // Streamed out (read back by the backward, long after this kernel): non-temporal stores.
            if (in)
            {
                const int pi = MK == MK_IDENT ? 0 : i;
                float* q = p.pstats + ((((int64_t)b * g.Cout + o) * (MK == MK_IDENT ? 1 : g.Cin) + pi) * plane + (int64_t)h * g.W + wc);
                __builtin_nontemporal_store(ref, q);
                __builtin_nontemporal_store(inv, q + p.nstat);
                __builtin_nontemporal_store(Wsum * inv, q + 2 * p.nstat);
            }
        }
        if constexpr (STATS)
        {
            if (is_winner(Wsum * inv, tgt)) m = m + 1.0f;
        }
        else if constexpr (MK == MK_MAX)
        {
            const float c = Wsum * inv;
            m = m < c ? c : m;
        }
        else if constexpr (MK == MK_MIN)
        {
            const float c = Wsum * inv;
            m = c < m ? c : m;
        }
        else if constexpr (MK == MK_SUM)
        {
            m = fmaf(Wsum, inv, m);
        }
        else if constexpr (MK == MK_SMOOTH)
        {
            // Every pair's output, merged afterwards by the soft merge (smorph.hip); with SAVE the
            // saved W / S values above are those outputs (the same index), read from there.
            if (!SAVE && in) p.pout[(((int64_t)b * g.Cout + o) * g.Cin + i) * plane + (int64_t)h * g.W + wc] = Wsum * inv;
        }
        else
        {
            m = Wsum * inv;
        }
        if (i + 1 < i_end) store(buf ^ 1);
        __syncthreads();
    }

    if (!in || MK == MK_SMOOTH) return;
    float v = m;
    if constexpr (MK == MK_SUM && !STATS)
    {
        if (p.average) v = v / (float)g.Cin;
    }
    p.out[((int64_t)b * g.Cout + o) * plane + (int64_t)h * g.W + wc] = v;
    if constexpr (STATS) p.tout[((int64_t)b * g.Cout + o) * plane + (int64_t)h * g.W + wc] = tgt;
}

// ------------------------------------------------------------------------------------------------
// Backward: one workgroup per (batch element, input channel, strip of 64 x 4 tiles), one output row
// per wave; for each tile it walks every output channel o.
// ------------------------------------------------------------------------------------------------

// The value of the next lower lane (0 in lane 0): DPP wave_shr:1 with bound_ctrl.
__device__ __forceinline__ float wave_shift_up(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x138, 0xf, 0xf, true));
}

// The forward statistics of one pair at this lane's pixel: ref (the window's extremum), 1 / S and
// W / S (taken from the forward's saved values, or recomputed).
struct PairStats
{
    float ref, inv, outp;
};

// One pair (o, i) at this lane's pixel, recomputing: the forward's ref, S and W (every tap's e kept
// up to 7x7), then the routing of c_k = p_k (1 + alpha (v_k - out)) g' to grad_input
// (the LDS tile), to the grad_weight bin of tap k and to grad_alpha (returned: the sum of
// p_k (v_k - ref)(v_k - out) over the taps). gv is g * scale (0 outside the image); for MAX / MIN it
// is divided by the pixel's winner count, and a pair not within 1e-6 of the merge target outv routes
// with g' = 0. For SMOOTH, outv is the merged output, sm the soft merge's beta, ref and 1 / sum at the
// pixel: g' = g q (1 + beta (c - outv)) with q = exp(beta (c - ref)) / sum the pair's share, and
// grad_beta's term q (c - ref)(c - outv) g goes to bterm (smorph_cpu_kernels.hxx:231-266).
struct SmoothPixel
{
    float beta, ref, inv;
};

template <int MK, int KH, int KW, bool MASKED>
__device__ __forceinline__ float smorph_bwd_pair(const float* xb, const float* wl, float a, float gv, float cnt, float outv, bool in,
                                                 const TapMask<KH, KW>& tm, Acc* gxb, Acc* bl, int lane, const SmoothPixel& sm,
                                                 float& bterm)
{
#pragma clang fp contract(off)  // fused only where the reference fuses (written as fmaf)
    constexpr int K = KH * KW, COLS = TILE_W + KW - 1;
    // A lane outside the image may meet a non-finite e (with saved statistics it holds another
    // pixel's ref; recomputing, a window with no tap in the image has an infinite ref): its c is
    // cleared.
    constexpr bool GATE = MASKED;
    float lo = ExpConsts<float>::min_input;
    asm volatile("" : "+v"(lo));  // the exponential's clamp in a register: register-only comparisons
    // Taps whose e stays in registers between the passes: all up to 7x7; for 11x11 the first two
    // rows (three waves per SIMD still; a third row takes 256 registers), except IDENTITY (no room).
    constexpr int KE = K <= 49 ? K : (MK == MK_IDENT ? 0 : 2 * KW);
    float e[KE > 0 ? KE : 1];
    PairStats st;
    {
        const bool dil = a >= 0.0f;
        const float ref = smorph_ref<KH, KW, MASKED>(xb, wl, dil, tm);
        // v is re-read from LDS in each pass: keep the compiler from holding the first pass's loads
        // in registers across the passes.
        asm volatile("" ::: "memory");
        float s = 0.0f, wsum = 0.0f;
#pragma unroll
        for (int kh = 0; kh < KH; ++kh)
        {
            if (MASKED && !tm.row(kh)) continue;
#pragma unroll
            for (int kw = 0; kw < KW; ++kw)
            {
                const int k = kh * KW + kw;
                const float vk = xb[-(kh * COLS + kw)] + wl[k];
                // Out-of-image taps: e = 0 leaves S and W as skipping them does, and routes c = 0.
                const float ek = exp_ref(MASKED ? (vk - ref) * a - tm.pen[kw] : (vk - ref) * a, lo);
                s = s + ek;  // unfused, as in the reference
                wsum = fmaf(ek, vk, wsum);
                if (k < KE) e[k] = ek;  // a constant condition once unrolled
            }
        }
        asm volatile("" ::: "memory");
        st.ref = ref;
        st.inv = 1.0f / s;
        st.outp = wsum * st.inv;
    }
    const float ref = st.ref;
    if constexpr (MK == MK_MAX || MK == MK_MIN)
    {
        // As the reference (smorph_cpu_kernels.hxx:507-545): a pair that is not a winner routes with
        // g' = 0, so its c are 0, or NaN where its own values are not finite.
        gv = gv / (cnt > 0.0f ? cnt : 1.0f);
        gv = is_winner(st.outp, outv) ? gv : 0.0f;
    }
    if constexpr (MK == MK_SMOOTH)
    {
        // Every in-image pixel adds its term, also with a zero gradient (a NaN pair reaches grad_beta).
        const float c = st.outp;
        const float q = exp_ref((c - sm.ref) * sm.beta, lo) * sm.inv;
        bterm = in ? q * (c - sm.ref) * (c - outv) * gv : 0.0f;
        gv = gv * fmaf(sm.beta * q, c - outv, q);
    }
    // A lane outside the image (where S may be 0 and out NaN) gets g' = 0 and a finite centre, and
    // its c are cleared.
    const float scaled = in ? gv * st.inv : 0.0f;
    const float outc = in ? st.outp : 0.0f;
    float asum = 0.0f;
#pragma unroll
    for (int kh = 0; kh < KH; ++kh)
    {
        if (MASKED && !tm.row(kh)) continue;
        // grad_input of the row's taps, summed per tile column across the wave before the LDS add:
        // lane l's tap kw lands in column l + KW - 1 - kw, so a Horner scheme over kw with a one-lane
        // shift (DPP wave_shr) leaves column l's total in lane l. What leaves lane 63 at step kw is
        // the (complete) total of the right halo column 63 + KW - kw; lane KW - 1 - kw keeps it.
        float racc = 0.0f, halo = 0.0f;
        __builtin_amdgcn_sched_barrier(0);
        // x and w of the next tap read from LDS one tap ahead of their use, so that the reads'
        // latency overlaps this tap's arithmetic (each tap is one long dependent chain).
        float xn = xb[-(kh * COLS)], wn = wl[kh * KW];
#pragma unroll
        for (int kw = 0; kw < KW; ++kw)
        {
            const int k = kh * KW + kw;
            const float vk = xn + wn;
            if (kw + 1 < KW)
            {
                xn = xb[-(kh * COLS + kw + 1)];
                wn = wl[k + 1];
            }
            float ekr;
            if (k >= KE)
            {
                ekr = exp_route(MASKED ? (vk - ref) * a - tm.pen[kw] : (vk - ref) * a);
            }
            else
            {
                ekr = e[k < KE ? k : 0];
            }
            const float pg = ekr * scaled;
            const float centered = vk - outc;
            // c = pg (1 + a centered) and the alpha term pg (v - ref) centered share pg centered.
            const float q = pg * centered;
            float c = fmaf(a, q, pg);
            if constexpr (GATE) c = in ? c : 0.0f;
            if (kw == 0)
            {
                racc = c;
            }
            else
            {
                const int fell = __builtin_amdgcn_readlane(__float_as_int(racc), WAVE - 1);
                asm("v_writelane_b32 %0, %1, %2" : "+v"(halo) : "s"(fell), "i"(KW - 1 - kw));
                racc = wave_shift_up(racc) + c;
            }
            lds_add(&bl[k * smorph_bin_copies(K)], (Acc)c);
            asum = fmaf(q, vk - ref, asum);
            // Keeps the compiler from deferring the alpha terms to the end of the pair, which would
            // hold every tap's factors in registers.
            asm volatile("" : "+v"(asum));
        }
        Acc* grow = gxb - (kh * COLS + KW - 1);  // this row's tile column `lane`
        lds_add(grow, (Acc)racc);
        if (lane < KW - 1) lds_add(grow + WAVE, (Acc)halo);
    }
    return in ? asum : 0.0f;
}

// The backward recomputing each pair's statistics (the saved-statistics backward is
// smorph_bwd_saved2 below). Waves per SIMD requested (measured on MI355X): up to 7x7 six (80
// registers, a few spilled; 7% faster than four, five fit without spills), 11x11 five (95 registers,
// 2 spilled; 16% faster than three, with 16 bin copies so that five workgroups' LDS fits a CU).
template <int MK, int KH, int KW>
__global__ __launch_bounds__(BLOCK) __attribute__((amdgpu_waves_per_eu(KH * KW > 49 ? 5 : 6, 8))) void smorph_bwd_static(
    const SmorphBwdParams<float> p)
{
    constexpr int K = KH * KW, PH = KH / 2, PW = KW / 2;
    constexpr int TH = NWAVES, ROWS = TH + KH - 1, COLS = TILE_W + KW - 1;
    constexpr int NC = smorph_bin_copies(K);
    // Bins after the K taps: grad_alpha, then grad_beta for SMOOTH.
    constexpr int NB = MK == MK_SMOOTH ? 2 : 1;
    __shared__ float tile[ROWS * COLS];
    __shared__ Acc gtile[ROWS * COLS];
    __shared__ __align__(32) Acc bins[(K + NB) * NC];  // grad_weight bins of the K taps, then the NB others; NC copies each
    // Structuring element, alpha and (SMOOTH) beta of the current / next pair, rows padded to 16 bytes
    // (128-bit reads; K is odd, so K + 2 entries fit).
    __shared__ __align__(16) float wl[2][(K + 4) & ~3];
    const Geom g = p.g;
    const Tiling t = p.t;
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    int work = xcd_work_index(blockIdx.x, gridDim.x);
    // Input channel fastest: the workgroups of one XCD share their strip's output gradients in L2.
    const int i = work % g.Cin;
    work /= g.Cin;
    const int strip = work % p.nstrips;
    const int b = work / p.nstrips;
    const int64_t plane = g.plane();
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * K;
    const int slot = b * p.nstrips + strip;
    float* __restrict__ part_w = p.part_w + (int64_t)slot * wnumel;
    float* __restrict__ part_a = p.part_a + (int64_t)slot * p.npairs;
    const int wi = MK == MK_IDENT ? 0 : i;
    const int o_begin = MK == MK_IDENT ? i : 0;
    const int o_end = MK == MK_IDENT ? i + 1 : g.Cout;
    const float* __restrict__ xp = p.x + ((int64_t)b * g.Cin + i) * plane;
    float* __restrict__ gplane = p.gin + ((int64_t)b * g.Cin + i) * plane;
    auto pair_index = [&](int o) { return MK == MK_IDENT ? o : o * g.Cin + i; };
    auto stage_weights = [&](int o, int buf) {
        if (threadIdx.x < K)
            wl[buf][threadIdx.x] = p.w[((int64_t)o * g.Cw + wi) * K + threadIdx.x];
        else if (threadIdx.x == K)
            wl[buf][K] = p.alpha[pair_index(o)];
        else if (MK == MK_SMOOTH && threadIdx.x == K + 1)
            wl[buf][K + 1] = p.beta[o];
    };

    // This workgroup's grad_weight / grad_alpha / grad_beta partials summed over its tiles (pair
    // o - o_begin, tap k, K for alpha, K + 1 for beta), stored once at the end, when they fit.
    constexpr int NPART = K <= 25 ? smorph_lds_partials(MK == MK_SMOOTH) : 1;
    __shared__ float partials[NPART];
    const bool lds_partials = smorph_bwd_lds_partials(g, MK == MK_IDENT, MK == MK_SMOOTH);
    for (int j = threadIdx.x; j < NPART; j += BLOCK) partials[j] = 0.0f;
    for (int j = threadIdx.x; j < (K + NB) * NC; j += BLOCK) bins[j] = Acc(0);
    // grad_beta partials: row (slot, i) of Cout values.
    float* __restrict__ part_b = MK == MK_SMOOTH ? p.part_b + ((int64_t)slot * g.Cin + i) * g.Cout : nullptr;
    const int tile_begin = strip * p.tps;
    const int tile_end = min(tile_begin + p.tps, t.ntiles());
    const float* xb = tile + (wave + KH - 1) * COLS + lane + KW - 1;
    Acc* gxb = gtile + (wave + KH - 1) * COLS + lane + KW - 1;
    Acc* bl = bins + (lane & (NC - 1));
    for (int tid = tile_begin; tid < tile_end; ++tid)
    {
        const int ty = tid / t.ntx, tx = tid - ty * t.ntx;
        const int h0 = ty * TH, w0 = tx * TILE_W;
        const int y0 = h0 + PH - (KH - 1), x0 = w0 + PW - (KW - 1);
        const int h = h0 + wave, wc = w0 + lane;
        const bool in = h < g.H && wc < g.W;
        const bool interior = y0 >= 0 && y0 + ROWS <= g.H && x0 >= 0 && x0 + COLS <= g.W;
        TapMask<KH, KW> tm;
        tm.init(g, h, wc);
        __syncthreads();
        for (int idx = threadIdx.x; idx < ROWS * COLS; idx += BLOCK)
        {
            const int ly = idx / COLS, lx = idx - ly * COLS;
            const int y = y0 + ly, x = x0 + lx;
            tile[idx] = (y >= 0 && y < g.H && x >= 0 && x < g.W) ? xp[(int64_t)y * g.W + x] : 0.0f;
            gtile[idx] = Acc(0);
        }
        stage_weights(o_begin, 0);
        // The output gradient (and, for MAX / MIN, the merged output and winner count; for SMOOTH, the
        // merged output and the soft merge's ref and 1 / sum) of this lane's pixel, one output channel
        // ahead.
        const int64_t pix = (int64_t)min(h, g.H - 1) * g.W + min(wc, g.W - 1);
        float gv_n = 0.0f, cnt_n = 0.0f, out_n = 0.0f, sref_n = 0.0f, sinv_n = 0.0f;
        auto load_g = [&](int o) {
            o = min(o, o_end - 1);
            const int64_t oi = ((int64_t)b * g.Cout + o) * plane + pix;
            gv_n = p.gout[oi];
            if constexpr (MK == MK_MAX || MK == MK_MIN)
            {
                cnt_n = p.counts[oi];
                out_n = p.out[oi];
            }
            if constexpr (MK == MK_SMOOTH)
            {
                out_n = p.out[oi];
                sref_n = p.sstats[oi];
                sinv_n = p.sstats[(int64_t)g.B * g.Cout * plane + oi];
            }
        };
        load_g(o_begin);
        __syncthreads();
        for (int o = o_begin; o < o_end; ++o)
        {
            const int buf = (o - o_begin) & 1;
            const float gv = in ? gv_n * p.scale : 0.0f, cnt = cnt_n, outv = out_n;
            SmoothPixel sm{0.0f, sref_n, sinv_n};
            load_g(o + 1);
            const float* w = wl[buf];
            const float a = w[K];
            if constexpr (MK == MK_SMOOTH) sm.beta = w[K + 1];
            float asum, bterm = 0.0f;
            if (interior)
                asum = smorph_bwd_pair<MK, KH, KW, false>(xb, w, a, gv, cnt, outv, in, tm, gxb, bl, lane, sm, bterm);
            else
                asum = smorph_bwd_pair<MK, KH, KW, true>(xb, w, a, gv, cnt, outv, in, tm, gxb, bl, lane, sm, bterm);
            lds_add(&bl[K * NC], (Acc)asum);
            if constexpr (MK == MK_SMOOTH) lds_add(&bl[(K + 1) * NC], (Acc)bterm);
            if (o + 1 < o_end) stage_weights(o + 1, buf ^ 1);
            __syncthreads();
            // Sum the NC copies of each bin: 8 threads per bin each add NC / 8 adjacent copies (16-byte
            // LDS reads) and clear them, a butterfly over the 8 finishes; the sums go to this
            // workgroup's slot. (K + NB) * 8 is a multiple of 8, so every group of 8 lanes is whole.
            constexpr int PER = NC / 8;  // copies per thread
            for (int j = threadIdx.x; j < (K + NB) * 8; j += BLOCK)
            {
                Acc v;
                if constexpr (PER == 4)
                {
                    double4* q = reinterpret_cast<double4*>(&bins[j * 4]);
                    const double4 c4 = *q;
                    *q = make_double4(0.0, 0.0, 0.0, 0.0);
                    v = (c4.x + c4.y) + (c4.z + c4.w);
                }
                else
                {
                    double2* q = reinterpret_cast<double2*>(&bins[j * 2]);
                    const double2 c2 = *q;
                    *q = make_double2(0.0, 0.0);
                    v = c2.x + c2.y;
                }
#pragma unroll
                for (int d = 4; d >= 1; d /= 2) v += __shfl_xor(v, d, 8);
                if ((j & 7) == 0)
                {
                    const int k = j >> 3;
                    if (lds_partials)
                        partials[(o - o_begin) * (K + NB) + k] += (float)v;  // one owner per entry
                    else if (k < K)
                        global_add(&part_w[((int64_t)o * g.Cw + wi) * K + k], (float)v);
                    else if (k == K)
                        global_add(&part_a[pair_index(o)], (float)v);
                    else
                        global_add(&part_b[o], (float)v);
                }
            }
            __syncthreads();
        }
        // grad_input of the tile and its halo: every cell may be shared with neighbouring tiles (the
        // tile is no taller than the element), so all go by atomics onto the zero-filled gradient.
        for (int idx = threadIdx.x; idx < ROWS * COLS; idx += BLOCK)
        {
            const int ly = idx / COLS, lx = idx - ly * COLS;
            const int y = y0 + ly, x = x0 + lx;
            if (y < 0 || y >= g.H || x < 0 || x >= g.W) continue;
            const float v = (float)gtile[idx];
            if (v != 0.0f) global_add(&gplane[(int64_t)y * g.W + x], v);
        }
    }
    if (lds_partials)
    {
        // Every entry of this workgroup's share of the slot (zeros for a strip without tiles): the
        // host skips the slot's zero fill.
        __syncthreads();
        const int n = (o_end - o_begin) * (K + NB);
        for (int j = threadIdx.x; j < n; j += BLOCK)
        {
            const int ol = j / (K + NB), k = j - ol * (K + NB), o = o_begin + ol;
            if (k < K)
                part_w[((int64_t)o * g.Cw + wi) * K + k] = partials[j];
            else if (k == K)
                part_a[pair_index(o)] = partials[j];
            else
                part_b[o] = partials[j];
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Backward from saved statistics, two output rows per wave: pixels A (row h) and B (row h + 1) of a
// lane's column. Tile row j = 0 .. KH of the wave's staged input holds tap row KH - 1 - j of A and tap
// row KH - j of B, so
//  * both pixels' taps of a tile row share its x reads, and their c values are added before the
//    row's DPP Horner sum and its LDS add (KH + 1 row sums for the two pixels instead of 2 KH);
//  * a tap's bin receives A's value (kept for one tile row) plus B's in one f64 LDS add.
// ------------------------------------------------------------------------------------------------

// Bins of the two-row backward at 7x7 and 11x11, packed: four bin values of a lane summed over
// groups of four lanes into one register (v_permlane32_swap then v_permlane16_swap, gfx950), so that
// one LDS add with 64 distinct addresses takes all four. The 16-lane row r of the result holds value
// smorph_pack_value(r) (0, 2, 1, 3 for rows 0-3) of the four, summed over lanes (l, l + 16, l + 32,
// l + 48) of the inputs. Every lane of the wave takes part. Measured on MI355X: 2% faster at 7x7
// (a quarter of the LDS adds for 0.4 VALU instructions per tap), 3% at 11x11 (whose unpacked 16-copy
// bins share each address between two lanes of a half wave, 2.4x the cost of an add).
__device__ __forceinline__ float smorph_pack4(float c0, float c1, float c2, float c3)
{
    const auto h01 = __builtin_amdgcn_permlane32_swap(__float_as_uint(c0), __float_as_uint(c1), false, false);
    const auto h23 = __builtin_amdgcn_permlane32_swap(__float_as_uint(c2), __float_as_uint(c3), false, false);
    const float s01 = __uint_as_float(h01[0]) + __uint_as_float(h01[1]);  // lanes 0-31: c0, 32-63: c1
    const float s23 = __uint_as_float(h23[0]) + __uint_as_float(h23[1]);  // lanes 0-31: c2, 32-63: c3
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(s01), __float_as_uint(s23), false, false);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

__host__ __device__ constexpr int smorph_pack_value(int row) { return ((row & 1) << 1) | (row >> 1); }

// Packed bins: the K tap values in the order the two-row backward emits them (tile row j = 1 .. KH,
// then kw: tap (KH - j) KW + kw) in groups of four, group q of 64 doubles, 16-lane row r holding
// emission 4 q + smorph_pack_value(r), 16 copies; then the last emission (K % 4 == 1), alpha and for
// SMOOTH (NB = 2) beta, unpacked, 16 copies each (a tail of 32 or 48 doubles keeps the 11x11
// kernel's LDS within five workgroups per CU).
template <int K, int NB = 1>
struct PackedBins
{
    static constexpr bool on = K > 25;
    static constexpr int groups = K / 4;
    static constexpr int size = groups * WAVE + (1 + NB) * 16;
};

// Rows of right-halo values (KW - 1 each) that one register holds, and the registers for NR rows.
template <int NR, int KW>
struct HaloRows
{
    static constexpr int rows = WAVE / (KW - 1);
    static constexpr int regs = (NR + rows - 1) / rows;
};

// One pixel's routing state for a pair: its saved ref, g' / S and the centre W / S (both 0 outside
// the image).
struct RoutePixel
{
    float ref, scaled, outc;
    bool in;
};

// MASKED: the tile reaches past the image, so some taps read outside it (tile rows skipped by the
// uniform `rows` bits, tap columns masked by `pen`). GATE: some of the wave's pixels lie outside the
// image (another pixel's ref, so their e may be infinite): their c is cleared. Border tiles of an image
// whose sides are multiples of the tile's (64 x 8) have no such pixel and skip that select per tap.
template <int MK, int KH, int KW, bool MASKED, bool ZA, bool GATE = MASKED>
__device__ __forceinline__ float smorph_bwd_pair2(const float* xw, const float* wl, float a, const RoutePixel& A, const RoutePixel& B,
                                                  unsigned rows, const float (&pen)[KW], Acc* gw, Acc* bl, Acc* btail,
                                                  const int (&hcell)[HaloRows<KH + 1, KW>::regs], Acc* gtile)
{
#pragma clang fp contract(off)  // fused only where the reference fuses (written as fmaf)
    constexpr int K = KH * KW, COLS = TILE_W + KW - 1, NC = smorph_bin_copies(K);
    float lo = ExpConsts<float>::min_input;
    asm volatile("" : "+v"(lo));  // the exponential's clamp in a register: register-only comparisons
    float asumA = 0.0f, asumB = 0.0f;
    float abuf[KW];  // A's c of the previous tile row's taps, added to B's in the same taps' bins
    constexpr bool PACK = PackedBins<K>::on;
    float pk[4];  // PACK: the current group of four bin values
    // The right-halo columns of all KH + 1 tile rows, HaloRows<>::rows rows per register: tile row j's
    // value for halo column c in lane (j % rows) (KW - 1) + c of register j / rows; one LDS add each
    // at the end of the pair.
    constexpr int HRW = HaloRows<KH + 1, KW>::rows, HREGS = HaloRows<KH + 1, KW>::regs;
    // 11x11 (not SMOOTH): lane 63 adds each value it shifts out to its halo cell itself, one f64 LDS
    // add under an exec mask per step, instead of a readlane and a writelane into the halo registers:
    // measured on MI355X 1.7% faster at 11x11, but 1.2% slower at 7x7 and 2.6% slower for SMOOTH.
    constexpr bool LANE_HALO = KW == 11 && MK != MK_SMOOTH;
    const int lane = threadIdx.x & (WAVE - 1);
    float halo[HREGS];
#pragma unroll
    for (int r = 0; r < HREGS; ++r) halo[r] = 0.0f;
    // alpha log2(e) once per pair, in a vector register: each tap's exponential is 2^((v - ref) a2).
    float a2 = a * 1.44269504088896340736f;
    asm volatile("" : "+v"(a2));
    // 11x11: each tap's two element values are read from LDS two taps ahead of their use, so that the
    // read's latency overlaps the previous taps' arithmetic (the asm statement below ends each tap's
    // scheduling region, which otherwise leaves every read just before its use, then a wait):
    // measured on MI355X 5% faster at 11x11 one tap ahead, 1.2% more two taps ahead; one tap ahead
    // was 0.5% slower at 7x7 (more spills there), and pinning the reads at the start of the tap with a
    // scheduling barrier 3.8% slower at 11x11.
    constexpr bool WAHEAD = KW > 7;
    auto route_tap = [&](const RoutePixel& P, float x, float wk, int kw, float& asum) {
        const float vk = x + wk;
        float ek;
        if constexpr (ZA)
            ek = exp_ref_zero_alpha(MASKED ? (vk - P.ref) * a - pen[kw] : (vk - P.ref) * a, lo);
        else
            ek = __builtin_amdgcn_exp2f(MASKED ? (vk - P.ref) * a2 - pen[kw] : (vk - P.ref) * a2);  // exp_route, log2(e) folded
        const float pg = ek * P.scaled;
        const float centered = vk - P.outc;
        // c = pg (1 + a centered) and the alpha term pg (v - ref) centered share pg centered.
        const float q = pg * centered;
        float c = fmaf(a, q, pg);
        if constexpr (GATE) c = P.in ? c : 0.0f;
        asum = fmaf(q, vk - P.ref, asum);
        // Keeps the compiler from deferring the alpha terms, which would hold every tap's factors
        // in registers.
        asm volatile("" : "+v"(asum));
        return c;
    };
#pragma unroll
    for (int j = 0; j <= KH; ++j)
    {
        const bool rv = !MASKED || ((rows >> j) & 1u);  // the tile row lies in the image (uniform)
        const int khA = j < KH ? KH - 1 - j : 0, khB = j > 0 ? KH - j : 0;
        float xr[KW];
#pragma unroll
        for (int kw = 0; kw < KW; ++kw) xr[kw] = xw[j * COLS - kw];
        float racc = 0.0f;
        float wAn = 0.0f, wBn = 0.0f, wAm = 0.0f, wBm = 0.0f;  // WAHEAD: the element values of the next two taps
        if (WAHEAD && rv)
        {
            if (j < KH)
            {
                wAn = wl[khA * KW];
                wAm = wl[khA * KW + 1];
            }
            if (j > 0)
            {
                wBn = wl[khB * KW];
                wBm = wl[khB * KW + 1];
            }
        }
#pragma unroll
        for (int kw = 0; kw < KW; ++kw)
        {
            float cA = 0.0f, cB = 0.0f;
            if (rv)
            {
                if constexpr (WAHEAD)
                {
                    const float wA = wAn, wB = wBn;
                    wAn = wAm;
                    wBn = wBm;
                    if (kw + 2 < KW)
                    {
                        if (j < KH) wAm = wl[khA * KW + kw + 2];
                        if (j > 0) wBm = wl[khB * KW + kw + 2];
                    }
                    if (j < KH) cA = route_tap(A, xr[kw], wA, kw, asumA);
                    if (j > 0) cB = route_tap(B, xr[kw], wB, kw, asumB);
                }
                else
                {
                    if (j < KH) cA = route_tap(A, xr[kw], wl[khA * KW + kw], kw, asumA);
                    if (j > 0) cB = route_tap(B, xr[kw], wl[khB * KW + kw], kw, asumB);
                }
                const float cs = j == 0 ? cA : (j == KH ? cB : cA + cB);
                // Row sums per tile column across the wave (DPP wave_shr Horner over kw); what leaves
                // lane 63 at step kw is the right halo column 63 + KW - kw: lane KW - 1 - kw keeps it.
                if (kw == 0)
                {
                    racc = cs;
                }
                else
                {
                    if constexpr (LANE_HALO)
                    {
                        if (lane == WAVE - 1) lds_add(gw + j * COLS + KW - kw, (Acc)racc);  // column 63 + KW - kw
                    }
                    else
                    {
                        const int fell = __builtin_amdgcn_readlane(__float_as_int(racc), WAVE - 1);
                        asm("v_writelane_b32 %0, %1, %2" : "+v"(halo[j / HRW]) : "s"(fell), "i"((j % HRW) * (KW - 1) + KW - 1 - kw));
                    }
                    racc = wave_shift_up(racc) + cs;
                }
            }
            if (j > 0)
            {
                if constexpr (PACK)
                {
                    const int e = (j - 1) * KW + kw;  // emission index (a constant once unrolled)
                    pk[e & 3] = cB + abuf[kw];
                    if ((e & 3) == 3) lds_add(&bl[(e >> 2) * WAVE], (Acc)smorph_pack4(pk[0], pk[1], pk[2], pk[3]));
                }
                else
                {
                    lds_add(&bl[(khB * KW + kw) * NC], (Acc)(cB + abuf[kw]));
                }
            }
            if (j < KH) abuf[kw] = cA;
        }
        if (rv)
        {
            lds_add(gw + j * COLS, (Acc)racc);  // tile row 2 wave + j, column `lane`
        }
    }
    if constexpr (!LANE_HALO)
    {
#pragma unroll
        for (int r = 0; r < HREGS; ++r)
            if (hcell[r] >= 0) lds_add(&gtile[hcell[r]], (Acc)halo[r]);
    }
    const float asum = (A.in ? asumA : 0.0f) + (B.in ? asumB : 0.0f);
    if constexpr (PACK)
    {
        // The tail: the last emission (K % 4 == 1 for odd square elements), then alpha.
        static_assert(K % 4 == 1, "odd square elements");
        lds_add(&btail[0], (Acc)pk[0]);
        lds_add(&btail[16], (Acc)asum);
    }
    return asum;
}

// Waves per SIMD requested: seven up to 5x5, six at 7x7, five at 11x11; SMOOTH (two more pixel
// values and the soft merge's share per pair) five from 5x5 on: 87 registers without spills at 5x5,
// where seven were out of reach (91 registers), and at 7x7 3 registers spilled instead of 18 at six
// (measured on MI355X: 1% faster at 7x7, the same at 5x5).
template <int MK, int KH, int KW>
__global__ __launch_bounds__(BLOCK) __attribute__((amdgpu_waves_per_eu(
    KH * KW > 49 ? 5 : ((MK == MK_SMOOTH && KH * KW >= 25) ? 5 : (KH * KW > 25 ? 6 : 7)), 8))) void
smorph_bwd_saved2(const SmorphBwdParams<float> p)
{
    constexpr int K = KH * KW, PH = KH / 2, PW = KW / 2;
    constexpr int RH = 2, TH = NWAVES * RH, ROWS = TH + KH - 1, COLS = TILE_W + KW - 1;
    constexpr int NC = smorph_bin_copies(K);
    // Values after the K taps: grad_alpha, then grad_beta for SMOOTH.
    constexpr int NB = MK == MK_SMOOTH ? 2 : 1;
    constexpr bool PACK = PackedBins<K>::on;
    constexpr int NBINS = PACK ? PackedBins<K, NB>::size : (K + NB) * NC;
    __shared__ float tile[ROWS * COLS];
    __shared__ Acc gtile[ROWS * COLS];
    // grad_weight bins of the K taps, then the NB others: NC copies each, or PACK's groups of four.
    __shared__ __align__(32) Acc bins[NBINS];
    // Structuring element, alpha and (SMOOTH) beta of the current / next pair.
    __shared__ __align__(16) float wl[2][(K + 4) & ~3];
    const Geom g = p.g;
    const Tiling t = p.t;
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    int work = xcd_work_index(blockIdx.x, gridDim.x);
    const int i = work % g.Cin;  // input channel fastest: an XCD's workgroups share the strip's g in L2
    work /= g.Cin;
    const int strip = work % p.nstrips;
    const int b = work / p.nstrips;
    const int64_t plane = g.plane();
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * K;
    const int slot = b * p.nstrips + strip;
    float* __restrict__ part_w = p.part_w + (int64_t)slot * wnumel;
    float* __restrict__ part_a = p.part_a + (int64_t)slot * p.npairs;
    const int wi = MK == MK_IDENT ? 0 : i;
    const int o_begin = MK == MK_IDENT ? i : 0;
    const int o_end = MK == MK_IDENT ? i + 1 : g.Cout;
    const int cpair = MK == MK_IDENT ? 1 : g.Cin;
    const float* __restrict__ xp = p.x + ((int64_t)b * g.Cin + i) * plane;
    float* __restrict__ gplane = p.gin + ((int64_t)b * g.Cin + i) * plane;
    auto pair_index = [&](int o) { return MK == MK_IDENT ? o : o * g.Cin + i; };
    auto stage_weights = [&](int o, int buf) {
        if (threadIdx.x < K)
            wl[buf][threadIdx.x] = p.w[((int64_t)o * g.Cw + wi) * K + threadIdx.x];
        else if (threadIdx.x == K)
            wl[buf][K] = p.alpha[pair_index(o)];
        else if (MK == MK_SMOOTH && threadIdx.x == K + 1)
            wl[buf][K + 1] = p.beta[o];
    };
    constexpr int NPART = K <= 25 ? smorph_lds_partials(MK == MK_SMOOTH) : 1;
    __shared__ float partials[NPART];
    const bool lds_partials = smorph_bwd_lds_partials(g, MK == MK_IDENT, MK == MK_SMOOTH);
    for (int j = threadIdx.x; j < NPART; j += BLOCK) partials[j] = 0.0f;
    for (int j = threadIdx.x; j < NBINS; j += BLOCK) bins[j] = Acc(0);
    // grad_beta partials: row (slot, i) of Cout values.
    float* __restrict__ part_b = MK == MK_SMOOTH ? p.part_b + ((int64_t)slot * g.Cin + i) * g.Cout : nullptr;
    const int tile_begin = strip * p.tps;
    const int tile_end = min(tile_begin + p.tps, t.ntiles());
    const float* xw = tile + RH * wave * COLS + lane + KW - 1;  // tile row 2 wave, this lane's tap-0 column
    Acc* gw = gtile + RH * wave * COLS + lane;
    Acc* bl = bins + (PACK ? lane : (lane & (NC - 1)));
    Acc* btail = bins + (PACK ? PackedBins<K>::groups * WAVE : 0) + (lane & 15);
    // The gtile cell of this lane's value in each halo register (tile row RH wave + j, halo column c,
    // right of the wave's 64 columns), or -1 for lanes past the last tile row.
    constexpr int HRW = HaloRows<KH + 1, KW>::rows, HREGS = HaloRows<KH + 1, KW>::regs;
    int hcell[HREGS];
#pragma unroll
    for (int r = 0; r < HREGS; ++r)
    {
        const int j = r * HRW + lane / (KW - 1), c = lane % (KW - 1);
        hcell[r] = lane < HRW * (KW - 1) && j <= KH ? (RH * wave + j) * COLS + WAVE + c : -1;
    }
    for (int tid = tile_begin; tid < tile_end; ++tid)
    {
        const int ty = tid / t.ntx, tx = tid - ty * t.ntx;
        const int h0 = ty * TH, w0 = tx * TILE_W;
        const int y0 = h0 + PH - (KH - 1), x0 = w0 + PW - (KW - 1);
        const int hA = h0 + RH * wave, wc = w0 + lane;
        const bool inA = hA < g.H && wc < g.W, inB = hA + 1 < g.H && wc < g.W;
        const bool interior = y0 >= 0 && y0 + ROWS <= g.H && x0 >= 0 && x0 + COLS <= g.W;
        // Some pixel of this wave's two rows lies outside the image (uniform over the wave).
        const bool gate = __builtin_amdgcn_uicmp((unsigned)!(inA && inB), 0u, 33) != 0;
        unsigned rows = 0;
#pragma unroll
        for (int j = 0; j <= KH; ++j)
        {
            const int y = y0 + RH * wave + j;
            rows |= (y >= 0 && y < g.H) ? 1u << j : 0u;
        }
        rows = __builtin_amdgcn_readfirstlane(rows);
        float pen[KW];
#pragma unroll
        for (int kw = 0; kw < KW; ++kw)
        {
            const int c = wc + PW - kw;
            pen[kw] = c >= 0 && c < g.W ? 0.0f : std::numeric_limits<float>::infinity();
        }
        __syncthreads();
        for (int idx = threadIdx.x; idx < ROWS * COLS; idx += BLOCK)
        {
            const int ly = idx / COLS, lx = idx - ly * COLS;
            const int y = y0 + ly, x = x0 + lx;
            tile[idx] = (y >= 0 && y < g.H && x >= 0 && x < g.W) ? xp[(int64_t)y * g.W + x] : 0.0f;
            gtile[idx] = Acc(0);
        }
        stage_weights(o_begin, 0);
        // Output gradient, saved statistics (and for MAX / MIN the merged output and winner count;
        // for SMOOTH the merged output and the soft merge's ref and 1 / sum) of both pixels, one
        // output channel ahead.
        const int64_t pixA = (int64_t)min(hA, g.H - 1) * g.W + min(wc, g.W - 1);
        const int64_t pixB = (int64_t)min(hA + 1, g.H - 1) * g.W + min(wc, g.W - 1);
        float gA_n = 0.0f, gB_n = 0.0f, cA_n = 0.0f, cB_n = 0.0f, oA_n = 0.0f, oB_n = 0.0f;
        SmoothPixel mA_n{0.0f, 0.0f, 0.0f}, mB_n{0.0f, 0.0f, 0.0f};
        PairStats sA_n{0.0f, 0.0f, 0.0f}, sB_n{0.0f, 0.0f, 0.0f};
        auto load_g = [&](int o) {
            o = min(o, o_end - 1);
            const int64_t ob = ((int64_t)b * g.Cout + o) * plane;
            gA_n = p.gout[ob + pixA];
            gB_n = p.gout[ob + pixB];
            if constexpr (MK == MK_MAX || MK == MK_MIN)
            {
                cA_n = p.counts[ob + pixA];
                cB_n = p.counts[ob + pixB];
            }
            if constexpr (MK == MK_MAX || MK == MK_MIN || MK == MK_SMOOTH)
            {
                oA_n = p.out[ob + pixA];
                oB_n = p.out[ob + pixB];
            }
            if constexpr (MK == MK_SMOOTH)
            {
                const int64_t nout = (int64_t)g.B * g.Cout * plane;
                mA_n.ref = p.sstats[ob + pixA];
                mA_n.inv = p.sstats[nout + ob + pixA];
                mB_n.ref = p.sstats[ob + pixB];
                mB_n.inv = p.sstats[nout + ob + pixB];
            }
            const float* q = p.pstats + (((int64_t)b * g.Cout + o) * cpair + (MK == MK_IDENT ? 0 : i)) * plane;
            sA_n.ref = __builtin_nontemporal_load(q + pixA);
            sA_n.inv = __builtin_nontemporal_load(q + p.nstat + pixA);
            sA_n.outp = __builtin_nontemporal_load(q + 2 * p.nstat + pixA);
            sB_n.ref = __builtin_nontemporal_load(q + pixB);
            sB_n.inv = __builtin_nontemporal_load(q + p.nstat + pixB);
            sB_n.outp = __builtin_nontemporal_load(q + 2 * p.nstat + pixB);
        };
        // bterm (SMOOTH): the pixel's grad_beta term.
        auto route_pixel = [&](bool in, float gv, float cnt, float outv, const PairStats& st, const SmoothPixel& sm, float& bterm) {
#pragma clang fp contract(off)  // fused only where the reference fuses (written as fmaf)
            RoutePixel r;
            gv = in ? gv * p.scale : 0.0f;
            if constexpr (MK == MK_MAX || MK == MK_MIN)
            {
                // A pair that is not a winner routes with g' = 0 (its c are 0, or NaN where its own
                // values are not finite), as the reference.
                gv = gv / (cnt > 0.0f ? cnt : 1.0f);
                gv = is_winner(st.outp, outv) ? gv : 0.0f;
            }
            if constexpr (MK == MK_SMOOTH)
            {
                // g' = g q (1 + beta (c - out)) with q = exp(beta (c - ref)) / sum the pair's share of
                // the soft merge, and grad_beta's term q (c - ref)(c - out) g, also with a zero gradient
                // (a NaN pair reaches grad_beta), as the recomputing kernel (smorph_bwd_pair).
                const float c = st.outp;
                const float q = exp_ref((c - sm.ref) * sm.beta) * sm.inv;
                bterm = in ? q * (c - sm.ref) * (c - outv) * gv : 0.0f;
                gv = gv * fmaf(sm.beta * q, c - outv, q);
            }
            r.ref = st.ref;
            r.scaled = in ? gv * st.inv : 0.0f;
            r.outc = in ? st.outp : 0.0f;
            r.in = in;
            return r;
        };
        load_g(o_begin);
        __syncthreads();
        for (int o = o_begin; o < o_end; ++o)
        {
            const int buf = (o - o_begin) & 1;
            const float* w = wl[buf];
            float btA = 0.0f, btB = 0.0f;
            if constexpr (MK == MK_SMOOTH) mA_n.beta = mB_n.beta = w[K + 1];
            const RoutePixel A = route_pixel(inA, gA_n, cA_n, oA_n, sA_n, mA_n, btA);
            const RoutePixel B = route_pixel(inB, gB_n, cB_n, oB_n, sB_n, mB_n, btB);
            load_g(o + 1);
            const float a = w[K];
            float asum;
            const bool za = alpha_is_zero(a);
            if (interior)
                asum = za ? smorph_bwd_pair2<MK, KH, KW, false, true>(xw, w, a, A, B, rows, pen, gw, bl, btail, hcell, gtile)
                          : smorph_bwd_pair2<MK, KH, KW, false, false>(xw, w, a, A, B, rows, pen, gw, bl, btail, hcell, gtile);
            else if (!gate)
                asum = za ? smorph_bwd_pair2<MK, KH, KW, true, true, false>(xw, w, a, A, B, rows, pen, gw, bl, btail, hcell, gtile)
                          : smorph_bwd_pair2<MK, KH, KW, true, false, false>(xw, w, a, A, B, rows, pen, gw, bl, btail, hcell, gtile);
            else
                asum = za ? smorph_bwd_pair2<MK, KH, KW, true, true>(xw, w, a, A, B, rows, pen, gw, bl, btail, hcell, gtile)
                          : smorph_bwd_pair2<MK, KH, KW, true, false>(xw, w, a, A, B, rows, pen, gw, bl, btail, hcell, gtile);
            if constexpr (!PACK) lds_add(&bl[K * NC], (Acc)asum);
            if constexpr (MK == MK_SMOOTH)
            {
                const float bterm = btA + btB;
                if constexpr (PACK)
                    lds_add(&btail[32], (Acc)bterm);
                else
                    lds_add(&bl[(K + 1) * NC], (Acc)bterm);
            }
            if (o + 1 < o_end) stage_weights(o + 1, buf ^ 1);
            __syncthreads();
            // Partial of value k (tap k < K, K alpha, K + 1 beta) of pair o into this workgroup's slot.
            auto put = [&](int k, Acc v) {
                if (lds_partials)
                    partials[(o - o_begin) * (K + NB) + k] += (float)v;  // one owner per entry
                else if (k < K)
                    global_add(&part_w[((int64_t)o * g.Cw + wi) * K + k], (float)v);
                else if (k == K)
                    global_add(&part_a[pair_index(o)], (float)v);
                else
                    global_add(&part_b[o], (float)v);
            };
            if constexpr (PACK)
            {
                // Sum the 16 copies of each value (4 threads per value, 4 adjacent copies each, a
                // butterfly over the 4) into this workgroup's slot: the packed groups, then the tail.
                // The thread count is a multiple of 4.
                constexpr int NG = PackedBins<K>::groups;
                for (int j = threadIdx.x; j < NG * 16 + (1 + NB) * 4; j += BLOCK)
                {
                    double4* q = reinterpret_cast<double4*>(&bins[j * 4]);
                    const double4 c4 = *q;
                    *q = make_double4(0.0, 0.0, 0.0, 0.0);
                    Acc v = (c4.x + c4.y) + (c4.z + c4.w);
                    v += __shfl_xor(v, 1, 4);
                    v += __shfl_xor(v, 2, 4);
                    // Emission index: in the groups, or the tail's K - 1 (the last tap), K (alpha) and
                    // K + 1 (beta).
                    const int e = j < NG * 16 ? (j >> 4) * 4 + smorph_pack_value((j >> 2) & 3) : K - 1 + ((j - NG * 16) >> 2);
                    if ((j & 3) == 0 && e < K + NB)
                    {
                        // Emission e < K is tap (KH - 1 - e / KW) KW + e % KW; the others keep their index.
                        put(e < K ? (KH - 1 - e / KW) * KW + e % KW : e, v);
                    }
                }
                __syncthreads();
                continue;
            }
            // Sum the NC copies of each bin (8 threads per bin, NC / 8 adjacent copies each, a butterfly
            // over the 8) into this workgroup's slot, as the one-row kernel does.
            constexpr int PER = NC / 8;
            for (int j = threadIdx.x; j < (K + NB) * 8; j += BLOCK)
            {
                Acc v;
                if constexpr (PER == 4)
                {
                    double4* q = reinterpret_cast<double4*>(&bins[j * 4]);
                    const double4 c4 = *q;
                    *q = make_double4(0.0, 0.0, 0.0, 0.0);
                    v = (c4.x + c4.y) + (c4.z + c4.w);
                }
                else
                {
                    double2* q = reinterpret_cast<double2*>(&bins[j * 2]);
                    const double2 c2 = *q;
                    *q = make_double2(0.0, 0.0);
                    v = c2.x + c2.y;
                }
#pragma unroll
                for (int d = 4; d >= 1; d /= 2) v += __shfl_xor(v, d, 8);
                if ((j & 7) == 0) put(j >> 3, v);
            }
            __syncthreads();
        }
        for (int idx = threadIdx.x; idx < ROWS * COLS; idx += BLOCK)
        {
            const int ly = idx / COLS, lx = idx - ly * COLS;
            const int y = y0 + ly, x = x0 + lx;
            if (y < 0 || y >= g.H || x < 0 || x >= g.W) continue;
            const float v = (float)gtile[idx];
            if (v != 0.0f) global_add(&gplane[(int64_t)y * g.W + x], v);
        }
    }
    if (lds_partials)
    {
        __syncthreads();
        const int n = (o_end - o_begin) * (K + NB);
        for (int j = threadIdx.x; j < n; j += BLOCK)
        {
            const int ol = j / (K + NB), k = j - ol * (K + NB), o = o_begin + ol;
            if (k < K)
                part_w[((int64_t)o * g.Cw + wi) * K + k] = partials[j];
            else if (k == K)
                part_a[pair_index(o)] = partials[j];
            else
                part_b[o] = partials[j];
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Launch
// ------------------------------------------------------------------------------------------------

template <int KS, bool SAVE>
static hipError_t fwd_size(int mk, bool stats, const SmorphFwdParams<float>& p, hipStream_t stream)
{
    const unsigned blocks = (unsigned)((int64_t)p.g.B * p.t.nty * p.t.ntx * p.g.Cout);
    if (stats)
    {
        if (mk == MK_MAX)
            smorph_fwd_static<MK_MAX, KS, KS, true, false><<<blocks, BLOCK, 0, stream>>>(p);
        else
            smorph_fwd_static<MK_MIN, KS, KS, true, false><<<blocks, BLOCK, 0, stream>>>(p);
        return hipGetLastError();
    }
    switch (mk)
    {
        case MK_SUM: smorph_fwd_static<MK_SUM, KS, KS, false, SAVE><<<blocks, BLOCK, 0, stream>>>(p); break;
        case MK_MAX: smorph_fwd_static<MK_MAX, KS, KS, false, SAVE><<<blocks, BLOCK, 0, stream>>>(p); break;
        case MK_MIN: smorph_fwd_static<MK_MIN, KS, KS, false, SAVE><<<blocks, BLOCK, 0, stream>>>(p); break;
        case MK_SMOOTH: smorph_fwd_static<MK_SMOOTH, KS, KS, false, SAVE><<<blocks, BLOCK, 0, stream>>>(p); break;
        default: smorph_fwd_static<MK_IDENT, KS, KS, false, SAVE><<<blocks, BLOCK, 0, stream>>>(p); break;
    }
    return hipGetLastError();
}

template <bool SAVE>
static hipError_t fwd_dispatch(int mk, bool stats, const SmorphFwdParams<float>& p, hipStream_t stream)
{
    switch (p.g.KH)
    {
        case 3: return fwd_size<3, SAVE>(mk, stats, p, stream);
        case 5: return fwd_size<5, SAVE>(mk, stats, p, stream);
        case 7: return fwd_size<7, SAVE>(mk, stats, p, stream);
        default: return fwd_size<11, SAVE>(mk, stats, p, stream);
    }
}

hipError_t launch_smorph_fwd_static(int mk, bool stats, const SmorphFwdParams<float>& p, hipStream_t stream)
{
    if (stats && p.pstats) return hipErrorInvalidValue;
    return p.pstats ? fwd_dispatch<true>(mk, stats, p, stream) : fwd_dispatch<false>(mk, stats, p, stream);
}

template <int KS>
static hipError_t bwd_size(int mk, const SmorphBwdParams<float>& p, hipStream_t stream)
{
    const unsigned blocks = (unsigned)((int64_t)p.g.B * p.g.Cin * p.nstrips);
    switch (mk)
    {
        case MK_SUM: smorph_bwd_static<MK_SUM, KS, KS><<<blocks, BLOCK, 0, stream>>>(p); break;
        case MK_MAX: smorph_bwd_static<MK_MAX, KS, KS><<<blocks, BLOCK, 0, stream>>>(p); break;
        case MK_MIN: smorph_bwd_static<MK_MIN, KS, KS><<<blocks, BLOCK, 0, stream>>>(p); break;
        case MK_SMOOTH: smorph_bwd_static<MK_SMOOTH, KS, KS><<<blocks, BLOCK, 0, stream>>>(p); break;
        default: smorph_bwd_static<MK_IDENT, KS, KS><<<blocks, BLOCK, 0, stream>>>(p); break;
    }
    return hipGetLastError();
}

template <int KS>
static hipError_t bwd2_size(int mk, const SmorphBwdParams<float>& p, hipStream_t stream)
{
    const unsigned blocks = (unsigned)((int64_t)p.g.B * p.g.Cin * p.nstrips);
    switch (mk)
    {
        case MK_SUM: smorph_bwd_saved2<MK_SUM, KS, KS><<<blocks, BLOCK, 0, stream>>>(p); break;
        case MK_MAX: smorph_bwd_saved2<MK_MAX, KS, KS><<<blocks, BLOCK, 0, stream>>>(p); break;
        case MK_MIN: smorph_bwd_saved2<MK_MIN, KS, KS><<<blocks, BLOCK, 0, stream>>>(p); break;
        case MK_SMOOTH: smorph_bwd_saved2<MK_SMOOTH, KS, KS><<<blocks, BLOCK, 0, stream>>>(p); break;
        default: smorph_bwd_saved2<MK_IDENT, KS, KS><<<blocks, BLOCK, 0, stream>>>(p); break;
    }
    return hipGetLastError();
}

hipError_t launch_smorph_bwd_static(int mk, const SmorphBwdParams<float>& p, hipStream_t stream)
{
    // From saved statistics: the two-row kernel (64 x 8 tiles); recomputing: the one-row kernel.
    if (p.t.rh != (p.pstats ? 2 : 1)) return hipErrorInvalidValue;
    switch (p.g.KH)
    {
        case 3: return p.pstats ? bwd2_size<3>(mk, p, stream) : bwd_size<3>(mk, p, stream);
        case 5: return p.pstats ? bwd2_size<5>(mk, p, stream) : bwd_size<5>(mk, p, stream);
        case 7: return p.pstats ? bwd2_size<7>(mk, p, stream) : bwd_size<7>(mk, p, stream);
        default: return p.pstats ? bwd2_size<11>(mk, p, stream) : bwd_size<11>(mk, p, stream);
    }
}

// MAX / MIN merge target and winner counts from the saved statistics: target[b, o, pixel] =
// smorph_merge_target of the merged output, counts[b, o, pixel] = the number of input channels i
// whose W / S lies within 1e-6 of it (what the counting forward pass computes,
// smorph_cpu_kernels.hxx:507-518, 622-627), one thread per output pixel.
__global__ __launch_bounds__(BLOCK) void smorph_counts_saved(const float* __restrict__ outp, const float* __restrict__ out,
                                                             float* __restrict__ counts, float* __restrict__ target, int64_t n_out, int cin,
                                                             int64_t plane)
{
    const int64_t j = (int64_t)blockIdx.x * BLOCK + threadIdx.x;
    if (j >= n_out) return;
    const int64_t bo = j / plane, pix = j - bo * plane;
    const float* q = outp + bo * cin * plane + pix;
    const float t = smorph_merge_target(out[j], q[0]);
    float m = 0.0f;
    for (int i = 0; i < cin; ++i)
        if (is_winner(q[(int64_t)i * plane], t)) m = m + 1.0f;
    counts[j] = m;
    target[j] = t;
}

hipError_t launch_smorph_counts_saved(const float* outp, const float* out, float* counts, float* target, const Geom& g, hipStream_t stream)
{
    const int64_t n_out = (int64_t)g.B * g.Cout * g.plane();
    if (n_out == 0) return hipSuccess;
    const unsigned blocks = (unsigned)((n_out + BLOCK - 1) / BLOCK);
    smorph_counts_saved<<<blocks, BLOCK, 0, stream>>>(outp, out, counts, target, n_out, g.Cin, g.plane());
    return hipGetLastError();
}

}  // namespace mca
