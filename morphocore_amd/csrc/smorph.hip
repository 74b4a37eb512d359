// Smorph forward and backward for gfx950 (reference semantics: smorph_cpu_kernels.hxx:14-229,
// 387-638; smorph.cpp:20-111).
//
// Per channel pair (o, i) and output pixel, over the taps that read an in-image pixel:
//   v_k = x_k + w_k, ref = max v (alpha >= 0) or min v, e_k = exp(alpha (v_k - ref)),
//   S = sum e_k, W = sum e_k v_k, out_pair = W * (1 / S), merged over input channels.
// A tap is in the image by its position (the staged tile holds 0 outside), so an in-image NaN takes
// part as in the reference: it never wins the ref scan (strict comparison), and its exponential is
// NaN, which reaches S, W and the gradients.
//
// SMOOTH merge (smorph_scm, smorph_cpu_kernels.hxx:231-266): the forward writes every pair output
// c_i; smorph_soft_merge_kernel then takes ref = the extremum of the c_i (channel 0 first, strict),
// q_i = exp(beta (c_i - ref)), out = (sum q_i c_i) * (1 / sum q_i). The backward routes, per pair,
// g_i = g (p_i + beta p_i (c_i - out)) with p_i = q_i / sum q_i, recomputed from the forward's ref and
// 1 / sum, and sums grad_beta = sum p_i (c_i - ref)(c_i - out) g.
//
// Forward (smorph_fwd_kernel): one workgroup per (batch element, output channel, tile) walks the
// input channels with the tile staged in LDS. The same kernel in STATS mode counts, for MAX / MIN
// merges, how many channel pairs lie within 1e-6 of the merged output (the backward's winners).
//
// Backward (smorph_bwd_kernel): one workgroup per (batch element, input channel, strip of tiles)
// walks every output channel, recomputes the pair's ref, S and W, and routes
//   c_k = p_k (1 + alpha (v_k - out)) g,  p_k = e_k / S,
// to an LDS copy of the tile's grad_input, to lane-striped LDS bins of grad_weight and to the
// pair's grad_alpha (sum of p_k (v_k - ref)(v_k - out) g); the bins become this workgroup's partial
// slot, summed over slots in a fixed order afterwards.
#include <algorithm>

#include "smorph_common.hpp"

namespace mca
{

// Whether tap (kh, kw) of the output pixel whose first tap reads input row `iy` and column `ix`
// (iy = h + KH / 2, ix = w + KW / 2) reads an in-image pixel.
__device__ __forceinline__ bool tap_in_image(int iy, int ix, int kh, int kw, const Geom& g)
{
    return (unsigned)(iy - kh) < (unsigned)g.H && (unsigned)(ix - kw) < (unsigned)g.W;
}

// ref, S and W of one pair for the RH pixels of this lane (rows iy0 + r, column ix in input
// coordinates of the first tap), from the staged tile.
template <typename T, int RH>
__device__ __forceinline__ void smorph_pair_stats(const T* tbase, int pitch, const T* __restrict__ wp, T a, const Geom& g, int iy0, int ix,
                                                  T (&ref)[RH], T (&S)[RH], T (&Wsum)[RH])
{
#pragma clang fp contract(off)  // S = S + e and W fused as the reference rounds them (written as fma)
    const bool dilation_like = a >= T(0);
    const T lo = ExpConsts<T>::min_input;
#pragma unroll
    for (int r = 0; r < RH; ++r) ref[r] = dilation_like ? -std::numeric_limits<T>::infinity() : std::numeric_limits<T>::infinity();
    for (int kh = 0; kh < g.KH; ++kh)
        for (int kw = 0; kw < g.KW; ++kw)
        {
            const T wk = wp[kh * g.KW + kw];
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                const T v = tbase[(r - kh) * pitch - kw] + wk;
                // Strict replacement: a NaN never wins, as in the reference.
                const bool better = dilation_like ? v > ref[r] : v < ref[r];
                if (better && tap_in_image(iy0 + r, ix, kh, kw, g)) ref[r] = v;
            }
        }
#pragma unroll
    for (int r = 0; r < RH; ++r)
    {
        S[r] = T(0);
        Wsum[r] = T(0);
    }
    for (int kh = 0; kh < g.KH; ++kh)
        for (int kw = 0; kw < g.KW; ++kw)
        {
            const T wk = wp[kh * g.KW + kw];
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                const T v = tbase[(r - kh) * pitch - kw] + wk;
                const bool valid = tap_in_image(iy0 + r, ix, kh, kw, g);
                const T e = valid ? exp_ref((v - ref[r]) * a, lo) : T(0);
                S[r] = S[r] + e;
                Wsum[r] = fma(e, valid ? v : T(0), Wsum[r]);
            }
        }
}

template <typename T, int MK, int RH, bool STATS>
__global__ __launch_bounds__(BLOCK) void smorph_fwd_kernel(const SmorphFwdParams<T> p)
{
#pragma clang fp contract(off)  // fused only where the reference fuses (written as fma)
    extern __shared__ __align__(16) unsigned char smem_raw[];
    T* tile = reinterpret_cast<T*>(smem_raw);
    const Geom g = p.g;
    const Tiling t = p.t;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    int work = xcd_work_index(blockIdx.x, gridDim.x);
    const int o = work % g.Cout;
    work /= g.Cout;
    const int tx = work % t.ntx;
    work /= t.ntx;
    const int ty = work % t.nty;
    const int b = work / t.nty;
    const int h0 = ty * t.th, w0 = tx * TILE_W;
    const int K = g.KH * g.KW, ph = g.pad_h(), pw = g.pad_w();
    const int y0 = h0 + ph - (g.KH - 1), x0 = w0 + pw - (g.KW - 1);
    const int64_t plane = g.plane();
    const int wc = w0 + lane;
    // Input coordinates read by tap (0, 0) of this lane's first output row.
    const int iy0 = h0 + wave * RH + ph, ix = wc + pw;

    T m[RH], tgt[RH];
#pragma unroll
    for (int r = 0; r < RH; ++r)
    {
        // STATS mode counts winners from zero; otherwise the merge starts from its identity.
        m[r] = STATS ? T(0) : (MK == MK_MAX ? lowest_of<T>() : (MK == MK_MIN ? max_of<T>() : T(0)));
        tgt[r] = T(0);
        if constexpr (STATS)
        {
            const int h = h0 + wave * RH + r;
            if (h < g.H && wc < g.W) tgt[r] = p.target[((int64_t)b * g.Cout + o) * plane + (int64_t)h * g.W + wc];
        }
    }

    const int i_begin = MK == MK_IDENT ? o : 0;
    const int i_end = MK == MK_IDENT ? o + 1 : g.Cin;
    const T* tbase = tile + (wave * RH + g.KH - 1) * t.pitch + lane + g.KW - 1;
    for (int i = i_begin; i < i_end; ++i)
    {
        __syncthreads();
        stage_tile(tile, p.x + ((int64_t)b * g.Cin + i) * plane, g, t, y0, x0, false, T(0));
        __syncthreads();
        const int pair = MK == MK_IDENT ? o : o * g.Cin + i;
        const T a = p.alpha[pair];
        const T* __restrict__ wp = p.w + ((int64_t)o * g.Cw + (MK == MK_IDENT ? 0 : i)) * K;
        T ref[RH], S[RH], Wsum[RH];
        smorph_pair_stats<T, RH>(tbase, t.pitch, wp, a, g, iy0, ix, ref, S, Wsum);
#pragma unroll
        for (int r = 0; r < RH; ++r)
        {
            const T inv = T(1) / S[r];
            if constexpr (STATS)
            {
                if (i == i_begin) tgt[r] = smorph_merge_target(tgt[r], Wsum[r] * inv);
                if (is_winner(Wsum[r] * inv, tgt[r])) m[r] = m[r] + T(1);
            }
            else if constexpr (MK == MK_MAX)
            {
                const T c = Wsum[r] * inv;
                m[r] = m[r] < c ? c : m[r];
            }
            else if constexpr (MK == MK_MIN)
            {
                const T c = Wsum[r] * inv;
                m[r] = c < m[r] ? c : m[r];
            }
            else if constexpr (MK == MK_SUM)
            {
                m[r] = fma(Wsum[r], inv, m[r]);
            }
            else if constexpr (MK == MK_SMOOTH)
            {
                const int h = h0 + wave * RH + r;
                if (h < g.H && wc < g.W) p.pout[(((int64_t)b * g.Cout + o) * g.Cin + i) * plane + (int64_t)h * g.W + wc] = Wsum[r] * inv;
            }
            else
            {
                m[r] = Wsum[r] * inv;
            }
        }
    }

    if constexpr (MK == MK_SMOOTH) return;  // merged by smorph_soft_merge_kernel
#pragma unroll
    for (int r = 0; r < RH; ++r)
    {
        const int h = h0 + wave * RH + r;
        if (h >= g.H || wc >= g.W) continue;
        T v = m[r];
        if constexpr (MK == MK_SUM && !STATS)
        {
            if (p.average) v = v / (T)g.Cin;
        }
        p.out[((int64_t)b * g.Cout + o) * plane + (int64_t)h * g.W + wc] = v;
        if constexpr (STATS) p.tout[((int64_t)b * g.Cout + o) * plane + (int64_t)h * g.W + wc] = tgt[r];
    }
}

// GGIN: grad_input is summed in global memory (p.gacc, double atomics per routed tap) instead of an LDS
// copy of the tile flushed per tile: for elements whose tile and its double copy exceed the LDS.
template <typename T, int MK, int RH, bool GGIN = false>
__global__ __launch_bounds__(BLOCK) void smorph_bwd_kernel(const SmorphBwdParams<T> p)
{
#pragma clang fp contract(off)  // fused only where the reference fuses (written as fma)
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const Geom g = p.g;
    const Tiling t = p.t;
    const int tile_elems = t.rows * t.pitch;
    const int K = g.KH * g.KW, ph = g.pad_h(), pw = g.pad_w();
    // Bins per copy: the K taps of grad_weight, grad_alpha, and grad_beta for the SMOOTH merge.
    const int nb = K + (MK == MK_SMOOTH ? 2 : 1);
    T* tile = reinterpret_cast<T*>(smem_raw);
    Acc* gtile = reinterpret_cast<Acc*>(smem_raw + align16((size_t)tile_elems * sizeof(T)));
    Acc* bins = GGIN ? gtile : gtile + tile_elems;
    Acc* abins = bins + K * p.ncopy;
    Acc* bbins = abins + p.ncopy;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    int work = xcd_work_index(blockIdx.x, gridDim.x);
    const int strip = work % p.nstrips;
    work /= p.nstrips;
    const int i = work % g.Cin;
    const int b = work / g.Cin;
    const int64_t plane = g.plane();
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * K;
    const int slot = b * p.nstrips + strip;
    T* part_w = p.part_w + (int64_t)slot * wnumel;
    T* part_a = p.part_a + (int64_t)slot * p.npairs;
    const int copy = lane & (p.ncopy - 1);
    const T lo = ExpConsts<T>::min_input;

    for (int j = threadIdx.x; j < nb * p.ncopy; j += BLOCK) bins[j] = Acc(0);

    const int tile_begin = strip * p.tps;
    const int tile_end = min(tile_begin + p.tps, t.ntiles());
    const T* tbase = tile + (wave * RH + g.KH - 1) * t.pitch + lane + g.KW - 1;
    for (int tid = tile_begin; tid < tile_end; ++tid)
    {
        const int ty = tid / t.ntx, tx = tid - ty * t.ntx;
        const int h0 = ty * t.th, w0 = tx * TILE_W;
        const int y0 = h0 + ph - (g.KH - 1), x0 = w0 + pw - (g.KW - 1);
        const int wc = w0 + lane;
        const int iy0 = h0 + wave * RH + ph, ix = wc + pw;
        __syncthreads();
        stage_tile(tile, p.x + ((int64_t)b * g.Cin + i) * plane, g, t, y0, x0, false, T(0));
        if constexpr (!GGIN)
            for (int j = threadIdx.x; j < tile_elems; j += BLOCK) gtile[j] = Acc(0);
        __syncthreads();
        Acc* __restrict__ gacc_plane = GGIN ? p.gacc + ((int64_t)b * g.Cin + i) * plane : nullptr;

        const int o_begin = MK == MK_IDENT ? i : 0;
        const int o_end = MK == MK_IDENT ? i + 1 : g.Cout;
        for (int o = o_begin; o < o_end; ++o)
        {
            const int wi = MK == MK_IDENT ? 0 : i;
            const int pair = MK == MK_IDENT ? o : o * g.Cin + i;
            const T a = p.alpha[pair];
            const T* __restrict__ wp = p.w + ((int64_t)o * g.Cw + wi) * K;
            T ref[RH], S[RH], Wsum[RH], outp[RH], scaled[RH], asum[RH];
            bool in[RH];
            T bsum = T(0);
            smorph_pair_stats<T, RH>(tbase, t.pitch, wp, a, g, iy0, ix, ref, S, Wsum);
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                const int h = h0 + wave * RH + r;
                in[r] = h < g.H && wc < g.W;
                const int64_t oi = ((int64_t)b * g.Cout + o) * plane + (int64_t)h * g.W + wc;
                T gv = in[r] ? p.gout[oi] * p.scale : T(0);
                const T inv = T(1) / S[r];
                outp[r] = Wsum[r] * inv;
                if constexpr (MK == MK_MAX || MK == MK_MIN)
                {
                    if (in[r])
                    {
                        const T cnt = p.counts[oi];
                        gv = gv / (cnt > T(0) ? cnt : T(1));
                        if (!is_winner(outp[r], p.out[oi])) gv = T(0);
                    }
                }
                if constexpr (MK == MK_SMOOTH)
                {
                    // Channel i's share of the soft merge, from the forward's ref and 1 / sum.
                    if (in[r])
                    {
                        const T bt = p.beta[o];
                        const T sref = p.sstats[oi], sinv = p.sstats[(int64_t)g.B * g.Cout * plane + oi], fin = p.out[oi];
                        const T c = outp[r];
                        const T pp = exp_ref((c - sref) * bt, lo) * sinv;
                        bsum = bsum + pp * (c - sref) * (c - fin) * gv;
                        gv = gv * fma(bt * pp, c - fin, pp);
                    }
                }
                scaled[r] = gv * inv;
                asum[r] = T(0);
            }
            for (int kh = 0; kh < g.KH; ++kh)
                for (int kw = 0; kw < g.KW; ++kw)
                {
                    const int k = kh * g.KW + kw;
                    const T wk = wp[k];
#pragma unroll
                    for (int r = 0; r < RH; ++r)
                    {
                        // Every in-image tap of an in-image pixel routes, also with a zero gradient
                        // (so that a NaN of the pair reaches the gradients, as in the reference).
                        if (!in[r] || !tap_in_image(iy0 + r, ix, kh, kw, g)) continue;
                        const T v = tbase[(r - kh) * t.pitch - kw] + wk;
                        // The routing's exponential: the hardware one in float32 (the sums above,
                        // and so the output, use the reference's).
                        T e;
                        if constexpr (sizeof(T) == 4)
                            e = exp_route((v - ref[r]) * a);
                        else
                            e = exp_ref((v - ref[r]) * a, lo);
                        const T pg = e * scaled[r];
                        const T centered = v - outp[r];
                        // c = pg (1 + a centered) and the alpha term pg (v - ref) centered share pg centered.
                        const T q = pg * centered;
                        const T c = fma(a, q, pg);
                        if constexpr (GGIN)
                            global_add(&gacc_plane[(int64_t)(iy0 + r - kh) * g.W + (ix - kw)], (Acc)c);
                        else
                            lds_add(&gtile[(wave * RH + r + g.KH - 1 - kh) * t.pitch + lane + g.KW - 1 - kw], (Acc)c);
                        lds_add(&bins[k * p.ncopy + copy], (Acc)c);
                        asum[r] = fma(q, v - ref[r], asum[r]);
                    }
                }
            T as = T(0);
#pragma unroll
            for (int r = 0; r < RH; ++r) as += asum[r];
            if (as != T(0)) lds_add(&abins[copy], (Acc)as);
            if constexpr (MK == MK_SMOOTH)
                if (bsum != T(0)) lds_add(&bbins[copy], (Acc)bsum);
            __syncthreads();
            for (int j = threadIdx.x; j < nb; j += BLOCK)
            {
                Acc s = Acc(0);
                for (int c = 0; c < p.ncopy; ++c)
                {
                    s += bins[j * p.ncopy + c];
                    bins[j * p.ncopy + c] = Acc(0);
                }
                if (j < K)
                    part_w[((int64_t)o * g.Cw + wi) * K + j] += (T)s;
                else if (j == K)
                    part_a[pair] += (T)s;
                else
                    p.part_b[((int64_t)slot * g.Cin + i) * g.Cout + o] += (T)s;
            }
            __syncthreads();
        }

        if constexpr (GGIN) continue;  // nothing staged: grad_input is already in global memory
        T* gplane = p.gin + ((int64_t)b * g.Cin + i) * plane;
        for (int ly = wave; ly < t.rows; ly += NWAVES)
        {
            const int iy = y0 + ly;
            if (iy < 0 || iy >= g.H) continue;
            for (int lx = lane; lx < t.cols; lx += WAVE)
            {
                const int gx = x0 + lx;
                if (gx < 0 || gx >= g.W) continue;
                const T v = (T)gtile[ly * t.pitch + lx];
                if (v != T(0)) global_add(&gplane[(int64_t)iy * g.W + gx], v);
            }
        }
    }
}

// SMOOTH merge of the pair outputs c_i of one (batch element, output channel, pixel) per thread
// (smorph_soft_merge, smorph_cpu_kernels.hxx:231-266): ref = c_0, replaced by each later channel that
// is strictly greater (beta >= 0) or smaller; q_i = exp((c_i - ref) beta); sum = sum q_i and
// weighted = sum q_i c_i (fused) in channel order; out = weighted * (1 / sum). `sstats` (or null)
// receives ref, then 1 / sum, [B, Cout, H, W] each, for the backward. The c_i of one output channel
// are Cin planes apart, so consecutive threads read consecutive pixels of each plane.
// CREG > 0 (Cin <= CREG, checked by the launcher): the c_i are read once, into registers, and both
// passes run from there (the two-pass form reads them from memory twice: 4.2 ms at configs[2]'s shape,
// 8.6 GB of pair outputs per pass).
template <typename T, int CREG>
__global__ __launch_bounds__(BLOCK) void smorph_soft_merge_kernel(const T* __restrict__ pout, const T* __restrict__ beta, T* __restrict__ out,
                                                                  T* __restrict__ sstats, Geom g)
{
#pragma clang fp contract(off)
    const int64_t plane = g.plane();
    const int64_t n = (int64_t)g.B * g.Cout * plane;
    const T lo = ExpConsts<T>::min_input;
    for (int64_t j = (int64_t)blockIdx.x * BLOCK + threadIdx.x; j < n; j += (int64_t)gridDim.x * BLOCK)
    {
        const int64_t bo = j / plane;
        const int64_t pix = j - bo * plane;
        const T bt = beta[bo % g.Cout];
        const T* __restrict__ c = pout + bo * g.Cin * plane + pix;
        if constexpr (CREG > 0)
        {
            T cv[CREG];
#pragma unroll
            for (int i = 0; i < CREG; ++i) cv[i] = i < g.Cin ? c[(int64_t)i * plane] : T(0);
            T ref = cv[0];
#pragma unroll
            for (int i = 1; i < CREG; ++i)
                if (i < g.Cin) ref = (bt >= T(0) ? cv[i] > ref : cv[i] < ref) ? cv[i] : ref;
            T sum = T(0), weighted = T(0);
#pragma unroll
            for (int i = 0; i < CREG; ++i)
                if (i < g.Cin)
                {
                    const T q = exp_ref((cv[i] - ref) * bt, lo);
                    sum = sum + q;
                    weighted = fma(q, cv[i], weighted);
                }
            const T inv = T(1) / sum;
            out[j] = weighted * inv;
            if (sstats)
            {
                sstats[j] = ref;
                sstats[n + j] = inv;
            }
            continue;
        }
        T ref = c[0];
        if (bt >= T(0))
        {
            for (int i = 1; i < g.Cin; ++i)
            {
                const T ci = c[(int64_t)i * plane];
                ref = ci > ref ? ci : ref;
            }
        }
        else
        {
            for (int i = 1; i < g.Cin; ++i)
            {
                const T ci = c[(int64_t)i * plane];
                ref = ci < ref ? ci : ref;
            }
        }
        T sum = T(0), weighted = T(0);
        for (int i = 0; i < g.Cin; ++i)
        {
            const T ci = c[(int64_t)i * plane];
            const T q = exp_ref((ci - ref) * bt, lo);
            sum = sum + q;
            weighted = fma(q, ci, weighted);
        }
        const T inv = T(1) / sum;
        out[j] = weighted * inv;
        if (sstats)
        {
            sstats[j] = ref;
            sstats[n + j] = inv;
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Launch
// ------------------------------------------------------------------------------------------------

struct SmorphBwdPlan
{
    Tiling t;
    int nstrips;
    int tps;
    int ncopy;
    int npairs;
    bool ggin;  // generic kernel with grad_input summed in global memory (smorph_bwd_kernel<..., true>)
    size_t part_w_bytes, part_a_bytes, part_b_bytes, counts_bytes, gacc_bytes;
    size_t lds;
};

// Rows per wave of the generic forward: the default while its tile fits the tuned LDS budget, else one
// (a shorter tile, for large elements).
template <typename T>
static int smorph_fwd_rh(const Geom& g)
{
    const Tiling t = make_tiling(g, rows_per_wave<T>());
    return (size_t)t.rows * t.pitch * sizeof(T) <= LDS_LIMIT ? rows_per_wave<T>() : 1;
}

// `saved`: the backward from saved statistics, whose static kernel takes two output rows per wave.
// Its tiles are taller, but the rounding of tiles per strip can still give it more strips (slots)
// than the one-row plan (4 x 64 x 100 x 100: 26 against 25), so the workspace is sized for both.
template <typename T>
static SmorphBwdPlan plan_smorph_bwd(int merge, const Geom& g, bool saved = false)
{
    SmorphBwdPlan s{};
    // The static kernels (smorph_static.hip) use one output row per wave (two from saved statistics)
    // and static LDS.
    const bool stat = smorph_static_supported<T>(g);
    int rh = stat ? (saved ? 2 : 1) : rows_per_wave<T>();
    s.ncopy = 16;
    if (!stat)
    {
        // The generic kernel: tile, its double grad_input copy, and ncopy copies of the bins (K taps,
        // alpha, beta for SMOOTH). The first of these that fits: the default rows per wave, then one
        // row per wave (a shorter tile), within the tuned budget, then within the device's LDS, then
        // grad_input summed in global memory (no copy of the tile); each with as many bin copies as
        // fit (fewer copies: more same-address LDS adds).
        const size_t nbins = (size_t)g.taps() + (merge == MERGE_SMOOTH ? 2 : 1);
        const size_t dev = device_lds_limit();
        const size_t budgets[2] = {LDS_LIMIT < dev ? LDS_LIMIT : dev, dev};
        bool fit = false;
        for (int attempt = 0; attempt < 5 && !fit; ++attempt)
        {
            const size_t budget = budgets[attempt < 2 ? 0 : 1];
            const bool ggin = attempt == 4;
            rh = (attempt == 0 || attempt == 2) ? rows_per_wave<T>() : 1;
            const Tiling t = make_tiling(g, rh);
            const size_t cells = (size_t)t.rows * t.pitch;
            const size_t fixed = align16(cells * sizeof(T)) + (ggin ? 0 : cells * sizeof(Acc));
            int ncopy = 16;
            while (ncopy > 1 && fixed + nbins * ncopy * sizeof(Acc) > budget) ncopy /= 2;
            s.ncopy = ncopy;
            s.ggin = ggin;
            s.lds = fixed + nbins * ncopy * sizeof(Acc);
            fit = s.lds <= budget;
        }
    }
    s.t = make_tiling(g, rh);
    s.npairs = merge == MERGE_IDENTITY ? g.Cout : g.Cout * g.Cin;
    const int64_t units = std::max<int64_t>(1, (int64_t)g.B * g.Cin);  // (an empty problem: one strip)
    const int ntiles = s.t.ntiles();
    int64_t nstrips = ((stat ? 8192 : 2048) + units - 1) / units;
    if (nstrips > ntiles) nstrips = ntiles;
    if (nstrips < 1) nstrips = 1;
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * g.taps();
    while (nstrips > 1 && (size_t)g.B * nstrips * (wnumel + s.npairs) * sizeof(T) > ((size_t)256 << 20)) nstrips = (nstrips + 1) / 2;
    s.tps = std::max(1, (int)((ntiles + nstrips - 1) / nstrips));
    s.nstrips = (int)((ntiles + s.tps - 1) / s.tps);
    const size_t nslots = (size_t)g.B * s.nstrips;
    s.part_w_bytes = nslots * wnumel * sizeof(T);
    s.part_a_bytes = nslots * s.npairs * sizeof(T);
    // SMOOTH: grad_beta partials [slot][Cin][Cout], as many values as the grad_alpha ones.
    s.part_b_bytes = merge == MERGE_SMOOTH ? s.part_a_bytes : 0;
    // MAX / MIN: winner counts, then the merge target, per output pixel.
    s.counts_bytes = (merge == MERGE_MAX || merge == MERGE_MIN) ? 2 * (size_t)g.B * g.Cout * g.plane() * sizeof(T) : 0;
    // grad_input summed in global memory: a double buffer, rounded into grad_input afterwards (float
    // tensors; double ones sum into grad_input itself).
    s.gacc_bytes = (s.ggin && sizeof(T) != sizeof(Acc)) ? (size_t)g.B * g.Cin * g.plane() * sizeof(Acc) : 0;
    return s;
}

template <typename T>
size_t smorph_lds(int merge, const Geom& g, bool backward)
{
    if (backward) return plan_smorph_bwd<T>(merge, g).lds;
    if (smorph_static_supported<T>(g)) return 0;  // static LDS
    const Tiling t = make_tiling(g, smorph_fwd_rh<T>(g));
    return (size_t)t.rows * t.pitch * sizeof(T);
}

// Workspace bytes of one backward plan: slot partials, MAX / MIN counts and target, reduction scratch.
template <typename T>
static size_t smorph_plan_workspace(const SmorphBwdPlan& s, const Geom& g)
{
    const int nslots = g.B * s.nstrips;
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * g.taps();
    const size_t red = reduce_slots_scratch<T>(nslots, wnumel > s.npairs ? wnumel : s.npairs);
    // SMOOTH: grad_beta sums nslots * Cin partial rows of Cout values.
    const size_t red_b = s.part_b_bytes ? reduce_slots_scratch<T>(nslots * g.Cin, g.Cout) : 0;
    return align_up(s.part_w_bytes) + align_up(s.part_a_bytes) + align_up(s.part_b_bytes) + align_up(s.counts_bytes) +
           align_up(red > red_b ? red : red_b) + align_up(s.gacc_bytes);
}

// Enough for either backward (recomputing or from saved statistics): the caller sizes the workspace
// before it knows which one runs.
template <typename T>
size_t smorph_backward_workspace(int merge, const Geom& g)
{
    const size_t a = smorph_plan_workspace<T>(plan_smorph_bwd<T>(merge, g, false), g);
    const size_t b = smorph_static_supported<T>(g) ? smorph_plan_workspace<T>(plan_smorph_bwd<T>(merge, g, true), g) : 0;
    return a > b ? a : b;
}

// The generic backward kernel of a plan: the default rows per wave or one, grad_input summed in an LDS
// copy of the tile or in global memory.
template <typename T, int MK>
static hipError_t launch_smorph_bwd_generic(const SmorphBwdPlan& s, const SmorphBwdParams<T>& p, hipStream_t stream)
{
    constexpr int RH = rows_per_wave<T>();
    const unsigned blocks = (unsigned)((int64_t)p.g.B * p.g.Cin * s.nstrips);
    if (s.ggin)
        smorph_bwd_kernel<T, MK, 1, true><<<blocks, BLOCK, s.lds, stream>>>(p);
    else if (s.t.rh == 1)
        smorph_bwd_kernel<T, MK, 1, false><<<blocks, BLOCK, s.lds, stream>>>(p);
    else
        smorph_bwd_kernel<T, MK, RH, false><<<blocks, BLOCK, s.lds, stream>>>(p);
    return hipGetLastError();
}

// Where the global-memory grad_input sum of a plan goes: grad_input itself for double tensors, the
// workspace buffer (zero-filled here, rounded into grad_input by finish_gacc) for float ones; null
// when the plan sums it in LDS.
template <typename T>
static hipError_t prepare_gacc(const SmorphBwdPlan& s, const Geom& g, T* grad_in, Acc* buffer, Acc** gacc, hipStream_t stream)
{
    *gacc = nullptr;
    if (!s.ggin) return hipSuccess;
    if constexpr (sizeof(T) == sizeof(Acc))
    {
        *gacc = reinterpret_cast<Acc*>(grad_in);  // zero-filled by the caller
        return hipSuccess;
    }
    else
    {
        *gacc = buffer;
        return fill_async<Acc>(buffer, (int64_t)g.B * g.Cin * g.plane(), Acc(0), stream);
    }
}

template <typename T>
static hipError_t finish_gacc(const SmorphBwdPlan& s, const Geom& g, const Acc* buffer, T* grad_in, hipStream_t stream)
{
    if constexpr (sizeof(T) != sizeof(Acc))
        if (s.ggin) return round_async<T>(buffer, grad_in, (int64_t)g.B * g.Cin * g.plane(), stream);
    return hipSuccess;
}

template <typename T, int MK, bool STATS>
static hipError_t launch_smorph_fwd(const SmorphFwdParams<T>& p, hipStream_t stream)
{
    if constexpr (sizeof(T) == 4)
        if (smorph_static_supported<T>(p.g)) return launch_smorph_fwd_static(MK, STATS, p, stream);
    constexpr int RH = rows_per_wave<T>();
    const int64_t blocks = (int64_t)p.g.B * p.t.nty * p.t.ntx * p.g.Cout;
    const size_t lds = (size_t)p.t.rows * p.t.pitch * sizeof(T);
    if (p.t.rh == 1)
        smorph_fwd_kernel<T, MK, 1, STATS><<<(unsigned)blocks, BLOCK, lds, stream>>>(p);
    else
        smorph_fwd_kernel<T, MK, RH, STATS><<<(unsigned)blocks, BLOCK, lds, stream>>>(p);
    return hipGetLastError();
}

int64_t smorph_stats_values(int merge, const Geom& g) { return smorph_stats_count<float>(merge, g); }

bool smorph_stats_supported(const Geom& g) { return smorph_static_supported<float>(g); }

template <typename T>
hipError_t smorph_forward(int merge, const T* x, const T* w, const T* alpha, T* out, const Geom& g, hipStream_t stream, float* stats)
{
    if (stats && !smorph_static_supported<T>(g)) return hipErrorInvalidValue;
    if ((int64_t)g.B * g.Cout * g.plane() == 0) return hipSuccess;
    if (g.Cin == 0)
        return fill_async<T>(out, (int64_t)g.B * g.Cout * g.plane(), empty_merge_value<T>(merge), stream);  // no channel pairs
    SmorphFwdParams<T> p{};
    p.x = x;
    p.w = w;
    p.alpha = alpha;
    p.out = out;
    p.target = nullptr;
    p.pstats = stats;
    p.nstat = smorph_stats_count<T>(merge, g);
    p.g = g;
    // The static kernels (smorph_static.hip) put one output row on each wave.
    p.t = make_tiling(g, smorph_static_supported<T>(g) ? 1 : smorph_fwd_rh<T>(g));
    p.average = merge == MERGE_AVERAGE;
    switch (merge)
    {
        case MERGE_ADD:
        case MERGE_AVERAGE: return launch_smorph_fwd<T, MK_SUM, false>(p, stream);
        case MERGE_MAX: return launch_smorph_fwd<T, MK_MAX, false>(p, stream);
        case MERGE_MIN: return launch_smorph_fwd<T, MK_MIN, false>(p, stream);
        case MERGE_IDENTITY: return launch_smorph_fwd<T, MK_IDENT, false>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

template <typename T>
hipError_t smorph_backward(int merge, const T* x, const T* w, const T* alpha, const T* out, const T* grad_out, T* grad_in, T* grad_w,
                           T* grad_alpha, const Geom& g, void* workspace, size_t workspace_bytes, hipStream_t stream, const float* stats)
{
    hipError_t err;
    if (workspace_bytes < smorph_backward_workspace<T>(merge, g)) return hipErrorInvalidValue;
    if (stats && !smorph_static_supported<T>(g)) return hipErrorInvalidValue;
    const int64_t nstat = smorph_stats_count<T>(merge, g);
    const SmorphBwdPlan s = plan_smorph_bwd<T>(merge, g, stats != nullptr);
    // The layout below is this plan's; never lay it out past the buffer.
    if (workspace_bytes < smorph_plan_workspace<T>(s, g)) return hipErrorInvalidValue;
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * g.taps();
    if ((err = fill_async<T>(grad_in, (int64_t)g.B * g.Cin * g.plane(), T(0), stream)) != hipSuccess) return err;
    if ((int64_t)g.B * g.Cout * g.plane() == 0 || g.Cin == 0)
    {
        if ((err = fill_async<T>(grad_w, wnumel, T(0), stream)) != hipSuccess) return err;
        return fill_async<T>(grad_alpha, s.npairs, T(0), stream);
    }
    unsigned char* ws = reinterpret_cast<unsigned char*>(workspace);
    T* part_w = reinterpret_cast<T*>(ws);
    T* part_a = reinterpret_cast<T*>(ws + align_up(s.part_w_bytes));
    T* counts = reinterpret_cast<T*>(ws + align_up(s.part_w_bytes) + align_up(s.part_a_bytes));
    T* target = counts + (int64_t)g.B * g.Cout * g.plane();
    Acc* gbuf = reinterpret_cast<Acc*>(ws + align_up(s.part_w_bytes) + align_up(s.part_a_bytes) + align_up(s.counts_bytes));
    T* scratch = reinterpret_cast<T*>(ws + align_up(s.part_w_bytes) + align_up(s.part_a_bytes) + align_up(s.counts_bytes) +
                                      align_up(s.gacc_bytes));
    const int nslots = g.B * s.nstrips;
    // The static kernels that keep their partials in LDS store every slot entry themselves.
    if (!(smorph_static_supported<T>(g) && smorph_bwd_lds_partials(g, merge == MERGE_IDENTITY)))
    {
        if ((err = fill_async<T>(part_w, (int64_t)nslots * wnumel, T(0), stream)) != hipSuccess) return err;
        if ((err = fill_async<T>(part_a, (int64_t)nslots * s.npairs, T(0), stream)) != hipSuccess) return err;
    }

    if (stats && (merge == MERGE_MAX || merge == MERGE_MIN))
    {
        if constexpr (sizeof(T) == 4)
            if ((err = launch_smorph_counts_saved(stats + 2 * nstat, out, counts, target, g, stream)) != hipSuccess) return err;
    }
    else if (merge == MERGE_MAX || merge == MERGE_MIN)
    {
        SmorphFwdParams<T> f{};
        f.x = x;
        f.w = w;
        f.alpha = alpha;
        f.out = counts;
        f.tout = target;
        f.target = out;
        f.g = g;
        f.t = make_tiling(g, smorph_static_supported<T>(g) ? 1 : smorph_fwd_rh<T>(g));
        f.average = 0;
        err = merge == MERGE_MAX ? launch_smorph_fwd<T, MK_MAX, true>(f, stream) : launch_smorph_fwd<T, MK_MIN, true>(f, stream);
        if (err != hipSuccess) return err;
    }

    SmorphBwdParams<T> p{};
    p.x = x;
    p.w = w;
    p.alpha = alpha;
    // MAX / MIN compare the pair outputs with the merge target (the forward's output unless channel
    // 0's pair output is NaN).
    p.out = (merge == MERGE_MAX || merge == MERGE_MIN) ? target : out;
    p.counts = counts;
    p.gout = grad_out;
    p.gin = grad_in;
    p.part_w = part_w;
    p.part_a = part_a;
    p.pstats = stats;
    p.nstat = nstat;
    p.g = g;
    p.t = s.t;
    p.nstrips = s.nstrips;
    p.tps = s.tps;
    p.ncopy = s.ncopy;
    p.npairs = s.npairs;
    p.scale = merge == MERGE_AVERAGE ? T(1) / (T)g.Cin : T(1);
    const int mk = merge == MERGE_MAX ? MK_MAX : (merge == MERGE_MIN ? MK_MIN : (merge == MERGE_IDENTITY ? MK_IDENT : MK_SUM));
    if constexpr (sizeof(T) == 4)
    {
        if (smorph_static_supported<T>(g))
        {
            if ((err = launch_smorph_bwd_static(mk, p, stream)) != hipSuccess) return err;
            if ((err = reduce_slots_async<T>(part_w, nslots, wnumel, grad_w, scratch, stream)) != hipSuccess) return err;
            return reduce_slots_async<T>(part_a, nslots, s.npairs, grad_alpha, scratch, stream);
        }
    }
    Acc* gacc = nullptr;
    if ((err = prepare_gacc<T>(s, g, grad_in, gbuf, &gacc, stream)) != hipSuccess) return err;
    p.gacc = gacc;
    switch (merge)
    {
        case MERGE_ADD:
        case MERGE_AVERAGE: err = launch_smorph_bwd_generic<T, MK_SUM>(s, p, stream); break;
        case MERGE_MAX: err = launch_smorph_bwd_generic<T, MK_MAX>(s, p, stream); break;
        case MERGE_MIN: err = launch_smorph_bwd_generic<T, MK_MIN>(s, p, stream); break;
        case MERGE_IDENTITY: err = launch_smorph_bwd_generic<T, MK_IDENT>(s, p, stream); break;
        default: return hipErrorInvalidValue;
    }
    if (err != hipSuccess) return err;
    if ((err = finish_gacc<T>(s, g, gbuf, grad_in, stream)) != hipSuccess) return err;
    if ((err = reduce_slots_async<T>(part_w, nslots, wnumel, grad_w, scratch, stream)) != hipSuccess) return err;
    return reduce_slots_async<T>(part_a, nslots, s.npairs, grad_alpha, scratch, stream);
}

// The smorph kernels' exponential, elementwise (a test probe of its bits).
template <typename T>
__global__ __launch_bounds__(BLOCK) void exp_probe_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t n)
{
    for (int64_t j = (int64_t)blockIdx.x * BLOCK + threadIdx.x; j < n; j += (int64_t)gridDim.x * BLOCK) y[j] = exp_ref(x[j]);
}

template <typename T>
hipError_t exp_probe(const T* x, T* y, int64_t n, hipStream_t stream)
{
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + BLOCK - 1) / BLOCK;
    exp_probe_kernel<T><<<(unsigned)(blocks > 8192 ? 8192 : blocks), BLOCK, 0, stream>>>(x, y, n);
    return hipGetLastError();
}

template hipError_t exp_probe<float>(const float*, float*, int64_t, hipStream_t);
template hipError_t exp_probe<double>(const double*, double*, int64_t, hipStream_t);

// ------------------------------------------------------------------------------------------------
// SMOOTH merge (smorph_scm): the generic kernels for every size and both types.
// ------------------------------------------------------------------------------------------------

template <typename T>
size_t smorph_scm_forward_workspace(const Geom& g)
{
    return align_up((size_t)g.B * g.Cout * g.Cin * g.plane() * sizeof(T));
}

template <typename T>
size_t smorph_scm_backward_workspace(const Geom& g)
{
    return smorph_backward_workspace<T>(MERGE_SMOOTH, g);
}

template <typename T>
size_t smorph_scm_lds(const Geom& g, bool backward)
{
    if (backward) return plan_smorph_bwd<T>(MERGE_SMOOTH, g).lds;
    if (smorph_static_supported<T>(g)) return 0;  // static LDS
    const Tiling t = make_tiling(g, smorph_fwd_rh<T>(g));
    return (size_t)t.rows * t.pitch * sizeof(T);
}

static unsigned elementwise_grid(int64_t n)
{
    const int64_t blocks = (n + BLOCK - 1) / BLOCK;
    return (unsigned)(blocks < 1 ? 1 : (blocks > 8192 ? 8192 : blocks));
}

template <typename T>
hipError_t smorph_scm_forward(const T* x, const T* w, const T* alpha, const T* beta, T* out, T* sstats, const Geom& g, void* workspace,
                              size_t workspace_bytes, hipStream_t stream, float* pstats)
{
    if (pstats && !(sizeof(T) == 4 && smorph_static_supported<T>(g))) return hipErrorInvalidValue;
    if (!pstats && workspace_bytes < smorph_scm_forward_workspace<T>(g)) return hipErrorInvalidValue;
    const int64_t n = (int64_t)g.B * g.Cout * g.plane();
    if (n == 0) return hipSuccess;
    SmorphFwdParams<T> p{};
    p.x = x;
    p.w = w;
    p.alpha = alpha;
    p.g = g;
    if constexpr (sizeof(T) == 4)
    {
        // Saving: the W / S array holds the pair outputs, [B, Cout, Cin, H, W] as the workspace would.
        p.pstats = pstats;
        p.nstat = smorph_stats_count<T>(MERGE_SMOOTH, g);
    }
    p.pout = pstats ? reinterpret_cast<T*>(pstats + 2 * p.nstat) : reinterpret_cast<T*>(workspace);
    // The float32 static kernels (one row per wave) write the pair outputs where they exist.
    p.t = make_tiling(g, smorph_static_supported<T>(g) ? 1 : smorph_fwd_rh<T>(g));
    hipError_t err = launch_smorph_fwd<T, MK_SMOOTH, false>(p, stream);
    if (err != hipSuccess) return err;
    if (sizeof(T) == 4 && g.Cin <= 16)
        smorph_soft_merge_kernel<T, 16><<<elementwise_grid(n), BLOCK, 0, stream>>>(p.pout, beta, out, sstats, g);
    else if (sizeof(T) == 4 && g.Cin <= 64)
        smorph_soft_merge_kernel<T, 64><<<elementwise_grid(n), BLOCK, 0, stream>>>(p.pout, beta, out, sstats, g);
    else
        smorph_soft_merge_kernel<T, 0><<<elementwise_grid(n), BLOCK, 0, stream>>>(p.pout, beta, out, sstats, g);
    return hipGetLastError();
}

template <typename T>
hipError_t smorph_scm_backward(const T* x, const T* w, const T* alpha, const T* beta, const T* out, const T* sstats, const T* grad_out,
                               T* grad_in, T* grad_w, T* grad_alpha, T* grad_beta, const Geom& g, void* workspace, size_t workspace_bytes,
                               hipStream_t stream, const float* pstats)
{
    hipError_t err;
    if (pstats && !(sizeof(T) == 4 && smorph_static_supported<T>(g))) return hipErrorInvalidValue;
    if (workspace_bytes < smorph_scm_backward_workspace<T>(g)) return hipErrorInvalidValue;
    const SmorphBwdPlan s = plan_smorph_bwd<T>(MERGE_SMOOTH, g, pstats != nullptr);
    // The layout below is this plan's; never lay it out past the buffer.
    if (workspace_bytes < smorph_plan_workspace<T>(s, g)) return hipErrorInvalidValue;
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * g.taps();
    if ((err = fill_async<T>(grad_in, (int64_t)g.B * g.Cin * g.plane(), T(0), stream)) != hipSuccess) return err;
    if ((int64_t)g.B * g.Cout * g.plane() == 0 || g.Cin == 0)
    {
        if ((err = fill_async<T>(grad_w, wnumel, T(0), stream)) != hipSuccess) return err;
        if ((err = fill_async<T>(grad_alpha, s.npairs, T(0), stream)) != hipSuccess) return err;
        return fill_async<T>(grad_beta, g.Cout, T(0), stream);
    }
    unsigned char* ws = reinterpret_cast<unsigned char*>(workspace);
    T* part_w = reinterpret_cast<T*>(ws);
    T* part_a = reinterpret_cast<T*>(ws + align_up(s.part_w_bytes));
    T* part_b = reinterpret_cast<T*>(ws + align_up(s.part_w_bytes) + align_up(s.part_a_bytes));
    Acc* gbuf = reinterpret_cast<Acc*>(ws + align_up(s.part_w_bytes) + align_up(s.part_a_bytes) + align_up(s.part_b_bytes));
    T* scratch = reinterpret_cast<T*>(ws + align_up(s.part_w_bytes) + align_up(s.part_a_bytes) + align_up(s.part_b_bytes) +
                                      align_up(s.gacc_bytes));
    const int nslots = g.B * s.nstrips;
    const bool stat = smorph_static_supported<T>(g);
    // The static kernel that keeps its partials in LDS stores every slot entry itself.
    if (!(stat && smorph_bwd_lds_partials(g, false, true)))
    {
        if ((err = fill_async<T>(part_w, (int64_t)nslots * wnumel, T(0), stream)) != hipSuccess) return err;
        if ((err = fill_async<T>(part_a, (int64_t)nslots * s.npairs, T(0), stream)) != hipSuccess) return err;
        if ((err = fill_async<T>(part_b, (int64_t)nslots * g.Cin * g.Cout, T(0), stream)) != hipSuccess) return err;
    }

    SmorphBwdParams<T> p{};
    p.x = x;
    p.w = w;
    p.alpha = alpha;
    p.out = out;
    p.gout = grad_out;
    p.gin = grad_in;
    p.part_w = part_w;
    p.part_a = part_a;
    p.beta = beta;
    p.sstats = sstats;
    p.part_b = part_b;
    p.g = g;
    p.t = s.t;
    p.nstrips = s.nstrips;
    p.tps = s.tps;
    p.ncopy = s.ncopy;
    p.npairs = s.npairs;
    p.scale = T(1);
    bool launched = false;
    if constexpr (sizeof(T) == 4)
        if (stat)
        {
            // The float32 static kernels: from the saved pair statistics (two rows per wave), or
            // recomputing them (one row per wave).
            p.pstats = pstats;
            p.nstat = smorph_stats_count<T>(MERGE_SMOOTH, g);
            if ((err = launch_smorph_bwd_static(MK_SMOOTH, p, stream)) != hipSuccess) return err;
            launched = true;
        }
    if (!launched)
    {
        Acc* gacc = nullptr;
        if ((err = prepare_gacc<T>(s, g, grad_in, gbuf, &gacc, stream)) != hipSuccess) return err;
        p.gacc = gacc;
        if ((err = launch_smorph_bwd_generic<T, MK_SMOOTH>(s, p, stream)) != hipSuccess) return err;
        if ((err = finish_gacc<T>(s, g, gbuf, grad_in, stream)) != hipSuccess) return err;
    }
    if ((err = reduce_slots_async<T>(part_w, nslots, wnumel, grad_w, scratch, stream)) != hipSuccess) return err;
    if ((err = reduce_slots_async<T>(part_a, nslots, s.npairs, grad_alpha, scratch, stream)) != hipSuccess) return err;
    // grad_beta[o]: the partial rows [slot][i] summed in (slot, i) order.
    return reduce_slots_async<T>(part_b, nslots * g.Cin, g.Cout, grad_beta, scratch, stream);
}

#define MCA_INSTANTIATE_SCM(T)                                                                                                           \
    template size_t smorph_scm_forward_workspace<T>(const Geom&);                                                                        \
    template size_t smorph_scm_backward_workspace<T>(const Geom&);                                                                       \
    template size_t smorph_scm_lds<T>(const Geom&, bool);                                                                                \
    template hipError_t smorph_scm_forward<T>(const T*, const T*, const T*, const T*, T*, T*, const Geom&, void*, size_t, hipStream_t,  \
                                              float*);                                                                               \
    template hipError_t smorph_scm_backward<T>(const T*, const T*, const T*, const T*, const T*, const T*, const T*, T*, T*, T*, T*,   \
                                               const Geom&, void*, size_t, hipStream_t, const float*);

MCA_INSTANTIATE_SCM(float)
MCA_INSTANTIATE_SCM(double)

#define MCA_INSTANTIATE_SMORPH(T)                                                                                                   \
    template hipError_t smorph_forward<T>(int, const T*, const T*, const T*, T*, const Geom&, hipStream_t, float*);                \
    template size_t smorph_lds<T>(int, const Geom&, bool);                                                                          \
    template size_t smorph_backward_workspace<T>(int, const Geom&);                                                                 \
    template hipError_t smorph_backward<T>(int, const T*, const T*, const T*, const T*, const T*, T*, T*, T*, const Geom&, void*, \
                                           size_t, hipStream_t, const float*);

MCA_INSTANTIATE_SMORPH(float)
MCA_INSTANTIATE_SMORPH(double)

}  // namespace mca
