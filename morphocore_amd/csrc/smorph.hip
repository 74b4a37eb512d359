// Smorph forward and backward for gfx950 (reference semantics: smorph_cpu_kernels.hxx:14-229,
// 387-638; smorph.cpp:20-111).
//
// Per channel pair (o, i) and output pixel, over the taps that read an in-image pixel:
//   v_k = x_k + w_k, ref = max v (alpha >= 0) or min v, e_k = exp(alpha (v_k - ref)),
//   S = sum e_k, W = sum e_k v_k, out_pair = W * (1 / S), merged over input channels.
// Out-of-image pixels are staged in LDS as NaN: they never win the ref scan, and the exp pass
// selects them away.
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
#include "smorph_common.hpp"

namespace mca
{

// ref, S and W of one pair for the RH pixels of this lane, from the staged tile.
template <typename T, int RH>
__device__ __forceinline__ void smorph_pair_stats(const T* tbase, int pitch, const T* __restrict__ wp, T a, int KH, int KW, T (&ref)[RH],
                                                  T (&S)[RH], T (&Wsum)[RH])
{
    const bool dilation_like = a >= T(0);
#pragma unroll
    for (int r = 0; r < RH; ++r) ref[r] = dilation_like ? -std::numeric_limits<T>::infinity() : std::numeric_limits<T>::infinity();
    if (dilation_like)
    {
        for (int kh = 0; kh < KH; ++kh)
            for (int kw = 0; kw < KW; ++kw)
            {
                const T wk = wp[kh * KW + kw];
#pragma unroll
                for (int r = 0; r < RH; ++r) ref[r] = fmax(ref[r], tbase[(r - kh) * pitch - kw] + wk);
            }
    }
    else
    {
        for (int kh = 0; kh < KH; ++kh)
            for (int kw = 0; kw < KW; ++kw)
            {
                const T wk = wp[kh * KW + kw];
#pragma unroll
                for (int r = 0; r < RH; ++r) ref[r] = fmin(ref[r], tbase[(r - kh) * pitch - kw] + wk);
            }
    }
#pragma unroll
    for (int r = 0; r < RH; ++r)
    {
        S[r] = T(0);
        Wsum[r] = T(0);
    }
    for (int kh = 0; kh < KH; ++kh)
        for (int kw = 0; kw < KW; ++kw)
        {
            const T wk = wp[kh * KW + kw];
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                const T v = tbase[(r - kh) * pitch - kw] + wk;
                const bool valid = v == v;
                const T e = valid ? exp_t((v - ref[r]) * a) : T(0);
                S[r] = S[r] + e;
                Wsum[r] = fma(e, valid ? v : T(0), Wsum[r]);
            }
        }
}

template <typename T, int MK, int RH, bool STATS>
__global__ __launch_bounds__(BLOCK) void smorph_fwd_kernel(const SmorphFwdParams<T> p)
{
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
    const T nan = std::numeric_limits<T>::quiet_NaN();
    const int wc = w0 + lane;

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
        stage_tile(tile, p.x + ((int64_t)b * g.Cin + i) * plane, g, t, y0, x0, false, nan);
        __syncthreads();
        const int pair = MK == MK_IDENT ? o : o * g.Cin + i;
        const T a = p.alpha[pair];
        const T* __restrict__ wp = p.w + ((int64_t)o * g.Cw + (MK == MK_IDENT ? 0 : i)) * K;
        T ref[RH], S[RH], Wsum[RH];
        smorph_pair_stats<T, RH>(tbase, t.pitch, wp, a, g.KH, g.KW, ref, S, Wsum);
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
            else
            {
                m[r] = Wsum[r] * inv;
            }
        }
    }

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

template <typename T, int MK, int RH>
__global__ __launch_bounds__(BLOCK) void smorph_bwd_kernel(const SmorphBwdParams<T> p)
{
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const Geom g = p.g;
    const Tiling t = p.t;
    const int tile_elems = t.rows * t.pitch;
    const int K = g.KH * g.KW, ph = g.pad_h(), pw = g.pad_w();
    T* tile = reinterpret_cast<T*>(smem_raw);
    Acc* gtile = reinterpret_cast<Acc*>(smem_raw + align16((size_t)tile_elems * sizeof(T)));
    Acc* bins = gtile + tile_elems;
    Acc* abins = bins + K * p.ncopy;
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
    const T nan = std::numeric_limits<T>::quiet_NaN();

    for (int j = threadIdx.x; j < (K + 1) * p.ncopy; j += BLOCK) bins[j] = Acc(0);

    const int tile_begin = strip * p.tps;
    const int tile_end = min(tile_begin + p.tps, t.ntiles());
    const T* tbase = tile + (wave * RH + g.KH - 1) * t.pitch + lane + g.KW - 1;
    for (int tid = tile_begin; tid < tile_end; ++tid)
    {
        const int ty = tid / t.ntx, tx = tid - ty * t.ntx;
        const int h0 = ty * t.th, w0 = tx * TILE_W;
        const int y0 = h0 + ph - (g.KH - 1), x0 = w0 + pw - (g.KW - 1);
        const int wc = w0 + lane;
        __syncthreads();
        stage_tile(tile, p.x + ((int64_t)b * g.Cin + i) * plane, g, t, y0, x0, false, nan);
        for (int j = threadIdx.x; j < tile_elems; j += BLOCK) gtile[j] = Acc(0);
        __syncthreads();

        const int o_begin = MK == MK_IDENT ? i : 0;
        const int o_end = MK == MK_IDENT ? i + 1 : g.Cout;
        for (int o = o_begin; o < o_end; ++o)
        {
            const int wi = MK == MK_IDENT ? 0 : i;
            const int pair = MK == MK_IDENT ? o : o * g.Cin + i;
            const T a = p.alpha[pair];
            const T* __restrict__ wp = p.w + ((int64_t)o * g.Cw + wi) * K;
            T ref[RH], S[RH], Wsum[RH], outp[RH], scaled[RH], asum[RH];
            smorph_pair_stats<T, RH>(tbase, t.pitch, wp, a, g.KH, g.KW, ref, S, Wsum);
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                const int h = h0 + wave * RH + r;
                const bool in = h < g.H && wc < g.W;
                const int64_t oi = ((int64_t)b * g.Cout + o) * plane + (int64_t)h * g.W + wc;
                T gv = in ? p.gout[oi] * p.scale : T(0);
                const T inv = T(1) / S[r];
                outp[r] = Wsum[r] * inv;
                if constexpr (MK == MK_MAX || MK == MK_MIN)
                {
                    if (in)
                    {
                        const T cnt = p.counts[oi];
                        gv = gv / (cnt > T(0) ? cnt : T(1));
                        if (!is_winner(outp[r], p.out[oi])) gv = T(0);
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
                        if (scaled[r] == T(0)) continue;
                        const T v = tbase[(r - kh) * t.pitch - kw] + wk;
                        if (!(v == v)) continue;
                        const T e = exp_t((v - ref[r]) * a);
                        const T pg = e * scaled[r];
                        const T centered = v - outp[r];
                        const T c = fma(a * pg, centered, pg);
                        lds_add(&gtile[(wave * RH + r + g.KH - 1 - kh) * t.pitch + lane + g.KW - 1 - kw], (Acc)c);
                        lds_add(&bins[k * p.ncopy + copy], (Acc)c);
                        asum[r] = asum[r] + pg * (v - ref[r]) * centered;
                    }
                }
            T as = T(0);
#pragma unroll
            for (int r = 0; r < RH; ++r) as += asum[r];
            if (as != T(0)) lds_add(&abins[copy], (Acc)as);
            __syncthreads();
            for (int j = threadIdx.x; j <= K; j += BLOCK)
            {
                Acc s = Acc(0);
                for (int c = 0; c < p.ncopy; ++c)
                {
                    s += bins[j * p.ncopy + c];
                    bins[j * p.ncopy + c] = Acc(0);
                }
                if (j < K)
                    part_w[((int64_t)o * g.Cw + wi) * K + j] += (T)s;
                else
                    part_a[pair] += (T)s;
            }
            __syncthreads();
        }

        T* gplane = p.gin + ((int64_t)b * g.Cin + i) * plane;
        for (int ly = wave; ly < t.rows; ly += NWAVES)
        {
            const int iy = y0 + ly;
            if (iy < 0 || iy >= g.H) continue;
            for (int lx = lane; lx < t.cols; lx += WAVE)
            {
                const int ix = x0 + lx;
                if (ix < 0 || ix >= g.W) continue;
                const T v = (T)gtile[ly * t.pitch + lx];
                if (v != T(0)) global_add(&gplane[(int64_t)iy * g.W + ix], v);
            }
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
    size_t part_w_bytes, part_a_bytes, counts_bytes;
    size_t lds;
};

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
    s.t = make_tiling(g, stat ? (saved ? 2 : 1) : rows_per_wave<T>());
    s.ncopy = 16;
    s.npairs = merge == MERGE_IDENTITY ? g.Cout : g.Cout * g.Cin;
    const int64_t units = (int64_t)g.B * g.Cin;
    const int ntiles = s.t.ntiles();
    int64_t nstrips = ((stat ? 8192 : 2048) + units - 1) / units;
    if (nstrips > ntiles) nstrips = ntiles;
    if (nstrips < 1) nstrips = 1;
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * g.taps();
    while (nstrips > 1 && (size_t)g.B * nstrips * (wnumel + s.npairs) * sizeof(T) > ((size_t)256 << 20)) nstrips = (nstrips + 1) / 2;
    s.tps = (int)((ntiles + nstrips - 1) / nstrips);
    s.nstrips = (int)((ntiles + s.tps - 1) / s.tps);
    const size_t nslots = (size_t)g.B * s.nstrips;
    s.part_w_bytes = nslots * wnumel * sizeof(T);
    s.part_a_bytes = nslots * s.npairs * sizeof(T);
    // MAX / MIN: winner counts, then the merge target, per output pixel.
    s.counts_bytes = (merge == MERGE_MAX || merge == MERGE_MIN) ? 2 * (size_t)g.B * g.Cout * g.plane() * sizeof(T) : 0;
    s.lds = stat ? 0
                 : align16((size_t)s.t.rows * s.t.pitch * sizeof(T)) + ((size_t)s.t.rows * s.t.pitch + (size_t)(g.taps() + 1) * s.ncopy) * sizeof(Acc);
    return s;
}

template <typename T>
size_t smorph_lds(int merge, const Geom& g, bool backward)
{
    if (backward) return plan_smorph_bwd<T>(merge, g).lds;
    if (smorph_static_supported<T>(g)) return 0;  // static LDS
    const Tiling t = make_tiling(g, rows_per_wave<T>());
    return (size_t)t.rows * t.pitch * sizeof(T);
}

// Workspace bytes of one backward plan: slot partials, MAX / MIN counts and target, reduction scratch.
template <typename T>
static size_t smorph_plan_workspace(const SmorphBwdPlan& s, const Geom& g)
{
    const int nslots = g.B * s.nstrips;
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * g.taps();
    return align_up(s.part_w_bytes) + align_up(s.part_a_bytes) + align_up(s.counts_bytes) +
           align_up(reduce_slots_scratch<T>(nslots, wnumel > s.npairs ? wnumel : s.npairs));
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

template <typename T, int MK, bool STATS>
static hipError_t launch_smorph_fwd(const SmorphFwdParams<T>& p, hipStream_t stream)
{
    if constexpr (sizeof(T) == 4)
        if (smorph_static_supported<T>(p.g)) return launch_smorph_fwd_static(MK, STATS, p, stream);
    constexpr int RH = rows_per_wave<T>();
    const int64_t blocks = (int64_t)p.g.B * p.t.nty * p.t.ntx * p.g.Cout;
    const size_t lds = (size_t)p.t.rows * p.t.pitch * sizeof(T);
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
    p.t = make_tiling(g, smorph_static_supported<T>(g) ? 1 : rows_per_wave<T>());
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
    if ((int64_t)g.B * g.Cout * g.plane() == 0)
    {
        if ((err = fill_async<T>(grad_w, wnumel, T(0), stream)) != hipSuccess) return err;
        return fill_async<T>(grad_alpha, s.npairs, T(0), stream);
    }
    unsigned char* ws = reinterpret_cast<unsigned char*>(workspace);
    T* part_w = reinterpret_cast<T*>(ws);
    T* part_a = reinterpret_cast<T*>(ws + align_up(s.part_w_bytes));
    T* counts = reinterpret_cast<T*>(ws + align_up(s.part_w_bytes) + align_up(s.part_a_bytes));
    T* target = counts + (int64_t)g.B * g.Cout * g.plane();
    T* scratch = reinterpret_cast<T*>(ws + align_up(s.part_w_bytes) + align_up(s.part_a_bytes) + align_up(s.counts_bytes));
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
        f.t = make_tiling(g, smorph_static_supported<T>(g) ? 1 : rows_per_wave<T>());
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
    constexpr int RH = rows_per_wave<T>();
    const unsigned blocks = (unsigned)((int64_t)g.B * g.Cin * s.nstrips);
    switch (merge)
    {
        case MERGE_ADD:
        case MERGE_AVERAGE: smorph_bwd_kernel<T, MK_SUM, RH><<<blocks, BLOCK, s.lds, stream>>>(p); break;
        case MERGE_MAX: smorph_bwd_kernel<T, MK_MAX, RH><<<blocks, BLOCK, s.lds, stream>>>(p); break;
        case MERGE_MIN: smorph_bwd_kernel<T, MK_MIN, RH><<<blocks, BLOCK, s.lds, stream>>>(p); break;
        case MERGE_IDENTITY: smorph_bwd_kernel<T, MK_IDENT, RH><<<blocks, BLOCK, s.lds, stream>>>(p); break;
        default: return hipErrorInvalidValue;
    }
    if ((err = hipGetLastError()) != hipSuccess) return err;
    if ((err = reduce_slots_async<T>(part_w, nslots, wnumel, grad_w, scratch, stream)) != hipSuccess) return err;
    return reduce_slots_async<T>(part_a, nslots, s.npairs, grad_alpha, scratch, stream);
}

#define MCA_INSTANTIATE_SMORPH(T)                                                                                                   \
    template hipError_t smorph_forward<T>(int, const T*, const T*, const T*, T*, const Geom&, hipStream_t, float*);                \
    template size_t smorph_lds<T>(int, const Geom&, bool);                                                                          \
    template size_t smorph_backward_workspace<T>(int, const Geom&);                                                                 \
    template hipError_t smorph_backward<T>(int, const T*, const T*, const T*, const T*, const T*, T*, T*, T*, const Geom&, void*, \
                                           size_t, hipStream_t, const float*);

MCA_INSTANTIATE_SMORPH(float)
MCA_INSTANTIATE_SMORPH(double)

}  // namespace mca
