// Dilation / erosion forward and backward for gfx950.
//
// Forward (morpho_fwd_kernel): a workgroup owns one output tile of one batch element for OB output
// channels and walks the input channels in order. Each input plane's tile plus halo is staged in
// LDS once and reused by the OB output channels; the structuring element values are wave-uniform
// (scalar loads). The per-pair extremum uses the NaN-ignoring max/min, the channel merge follows the
// reference's order and comparisons exactly (morpho_op_cpu_kernels.hxx:364-395), and the winning tap
// of a MAX / MIN merge is found afterwards by one rescan of the winning channel (first tap equal to
// the winning value), which also fixes the sign of a zero result.
//
// Backward, MAX / MIN (morpho_bwd_scatter_kernel): one workgroup per (output channel, pixel chunk)
// scatters each output gradient to its packed (channel, tap): grad_input by global float atomics,
// grad_weight into LDS bins that are written out as this workgroup's partial, then summed over the
// chunks in a fixed order (reduce_slots_kernel).
//
// Backward, ADD / AVERAGE / IDENTITY (morpho_bwd_pairs_kernel): one workgroup per (batch element,
// input channel, strip of tiles) stages the input tile once and walks every output channel,
// recomputing each pair's first extremal tap and routing the gradient into an LDS copy of the tile's
// grad_input (flushed once per tile) and into lane-striped LDS bins of grad_weight (written once per
// output channel into the workgroup's own partial slot, then summed over slots in a fixed order).
#include <stdexcept>

#include "launch.hpp"

namespace mca
{

template <typename T>
struct FwdParams
{
    const T* __restrict__ x;
    const T* __restrict__ w;
    T* __restrict__ out;
    int32_t* __restrict__ idx;
    Geom g;
    Tiling t;
    int nog;
    int replicate;
    int average;
    T fill;
};

template <typename T, int OP, int MK, int OB, int RH, bool SAVE>
__global__ __launch_bounds__(BLOCK) void morpho_fwd_kernel(const FwdParams<T> p)
{
    using Tr = OpTraits<OP, T>;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    T* tile = reinterpret_cast<T*>(smem_raw);
    const Geom g = p.g;
    const Tiling t = p.t;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    int work = xcd_work_index(blockIdx.x, gridDim.x);
    const int og = work % p.nog;
    work /= p.nog;
    const int tx = work % t.ntx;
    work /= t.ntx;
    const int ty = work % t.nty;
    const int b = work / t.nty;
    const int h0 = ty * t.th, w0 = tx * TILE_W, o0 = og * OB;
    const int K = g.KH * g.KW, ph = g.pad_h(), pw = g.pad_w();
    const int y0 = h0 + ph - (g.KH - 1), x0 = w0 + pw - (g.KW - 1);
    const int64_t plane = g.plane();
    const T* __restrict__ wb = p.w + (int64_t)b * g.wbs;

    T acc[OB][RH], best[OB][RH], winbest[OB][RH];
    int win[OB][RH];
#pragma unroll
    for (int ob = 0; ob < OB; ++ob)
#pragma unroll
        for (int r = 0; r < RH; ++r)
        {
            acc[ob][r] = MK == MK_MAX ? lowest_of<T>() : (MK == MK_MIN ? max_of<T>() : T(0));
            winbest[ob][r] = Tr::init();
            win[ob][r] = 0;
        }

    const int i_begin = MK == MK_IDENT ? o0 : 0;
    const int i_end = MK == MK_IDENT ? o0 + 1 : g.Cin;
    for (int i = i_begin; i < i_end; ++i)
    {
        __syncthreads();
        stage_tile(tile, p.x + ((int64_t)b * g.Cin + i) * plane, g, t, y0, x0, p.replicate != 0, p.fill);
        __syncthreads();

        const T* wi[OB];
#pragma unroll
        for (int ob = 0; ob < OB; ++ob)
        {
            const int o = min(o0 + ob, g.Cout - 1);
            wi[ob] = wb + ((int64_t)o * g.Cw + (MK == MK_IDENT ? 0 : i)) * K;
        }
#pragma unroll
        for (int ob = 0; ob < OB; ++ob)
#pragma unroll
            for (int r = 0; r < RH; ++r) best[ob][r] = Tr::init();

        const T* tbase = tile + (wave * RH + g.KH - 1) * t.pitch + lane + g.KW - 1;
        for (int kh = 0; kh < g.KH; ++kh)
        {
            const T* trow = tbase - kh * t.pitch;
            for (int kw = 0; kw < g.KW; ++kw)
            {
                T wk[OB];
#pragma unroll
                for (int ob = 0; ob < OB; ++ob) wk[ob] = wi[ob][kh * g.KW + kw];
#pragma unroll
                for (int r = 0; r < RH; ++r)
                {
                    const T xv = trow[r * t.pitch - kw];
#pragma unroll
                    for (int ob = 0; ob < OB; ++ob) best[ob][r] = Tr::pick(best[ob][r], Tr::combine(xv, wk[ob]));
                }
            }
        }

        // Channel merge in input-channel order (morpho_merge_policy.hpp:10-86).
#pragma unroll
        for (int ob = 0; ob < OB; ++ob)
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                const T bv = best[ob][r];
                if constexpr (MK == MK_SUM)
                {
                    acc[ob][r] = acc[ob][r] + bv;
                }
                else if constexpr (MK == MK_MAX)
                {
                    if (i == 0 || bv > acc[ob][r])
                    {
                        win[ob][r] = i;
                        winbest[ob][r] = bv;
                    }
                    acc[ob][r] = acc[ob][r] < bv ? bv : acc[ob][r];
                }
                else if constexpr (MK == MK_MIN)
                {
                    if (i == 0 || bv < acc[ob][r])
                    {
                        win[ob][r] = i;
                        winbest[ob][r] = bv;
                    }
                    acc[ob][r] = bv < acc[ob][r] ? bv : acc[ob][r];
                }
                else
                {
                    acc[ob][r] = bv;
                    win[ob][r] = i;
                    winbest[ob][r] = bv;
                }
            }
    }

#pragma unroll
    for (int ob = 0; ob < OB; ++ob)
#pragma unroll
        for (int r = 0; r < RH; ++r)
        {
            const int o = o0 + ob, h = h0 + wave * RH + r, wc = w0 + lane;
            if (o >= g.Cout || h >= g.H || wc >= g.W) continue;
            T v = acc[ob][r];
            if constexpr (MK == MK_SUM)
            {
                if (p.average) v = v / (T)g.Cin;
            }
            int32_t packed = 0;
            if constexpr (MK != MK_SUM)
            {
                // The first tap of the winning channel that reaches the winning value is the tap the
                // strict-improvement scan keeps; its own value carries the sign of a zero result.
                if ((SAVE || v == T(0)) && i_end > i_begin)
                {
                    const int c = win[ob][r];
                    const T target = winbest[ob][r];
                    const T* __restrict__ wp = wb + ((int64_t)o * g.Cw + (MK == MK_IDENT ? 0 : c)) * K;
                    const T* __restrict__ xp = p.x + ((int64_t)b * g.Cin + c) * plane;
                    int karg = 0;
                    if (target != Tr::init())
                    {
                        for (int k = 0; k < K; ++k)
                        {
                            const int kh = k / g.KW, kw = k - kh * g.KW;
                            const T xv = read_padded(xp, g.H, g.W, h + ph - kh, wc + pw - kw, p.replicate != 0, p.fill);
                            const T val = Tr::combine(xv, wp[k]);
                            if (val == target)
                            {
                                karg = k;
                                if (v == T(0)) v = val;
                                break;
                            }
                        }
                    }
                    packed = (int32_t)((c << 16) | karg);
                }
            }
            const int64_t oi = ((int64_t)b * g.Cout + o) * plane + (int64_t)h * g.W + wc;
            p.out[oi] = v;
            if constexpr (SAVE) p.idx[oi] = packed;
        }
}

template <typename T>
struct ScatterParams
{
    const int32_t* __restrict__ idx;
    const T* __restrict__ gout;
    T* __restrict__ gin;
    T* __restrict__ part;
    Geom g;
    int nchunks;
    int lds_bins;
    int64_t chunk;
};

template <typename T, int OP>
__global__ __launch_bounds__(BLOCK) void morpho_bwd_scatter_kernel(const ScatterParams<T> p)
{
    extern __shared__ __align__(16) unsigned char smem_raw[];
    T* bins = reinterpret_cast<T*>(smem_raw);
    const Geom g = p.g;
    const int work = xcd_work_index(blockIdx.x, gridDim.x);
    const int chunk = work % p.nchunks;
    const int o = work / p.nchunks;
    const int K = g.KH * g.KW, ph = g.pad_h(), pw = g.pad_w();
    const int64_t nb = (int64_t)g.Cin * K;
    const int64_t plane = g.plane();
    T* part = p.part + ((int64_t)chunk * g.Cout + o) * nb;
    if (p.lds_bins)
    {
        for (int64_t j = threadIdx.x; j < nb; j += BLOCK) bins[j] = T(0);
        __syncthreads();
    }
    const int64_t total = (int64_t)g.B * plane;
    const int64_t n_begin = (int64_t)chunk * p.chunk;
    const int64_t n_end = min(n_begin + p.chunk, total);
    const T sign = (T)OpTraits<OP, T>::sign;
    for (int64_t n = n_begin + threadIdx.x; n < n_end; n += BLOCK)
    {
        const int64_t b = n / plane;
        const int64_t pix = n - b * plane;
        const int h = (int)(pix / g.W), wc = (int)(pix - (int64_t)h * g.W);
        const int64_t gi = (b * g.Cout + o) * plane + pix;
        const T gv = p.gout[gi];
        if (gv == T(0)) continue;
        const int32_t packed = p.idx[gi];
        const int c = packed >> 16, k = packed & 0xFFFF;
        const int kh = k / g.KW, kw = k - kh * g.KW;
        const int iy = h + ph - kh, ix = wc + pw - kw;
        if (iy >= 0 && iy < g.H && ix >= 0 && ix < g.W) global_add(&p.gin[(b * g.Cin + c) * plane + (int64_t)iy * g.W + ix], gv);
        if (p.lds_bins)
            lds_add(&bins[(int64_t)c * K + k], sign * gv);
        else
            global_add(&part[(int64_t)c * K + k], sign * gv);
    }
    if (p.lds_bins)
    {
        __syncthreads();
        for (int64_t j = threadIdx.x; j < nb; j += BLOCK) part[j] = bins[j];
    }
}

template <typename T>
struct PairsParams
{
    const T* __restrict__ x;
    const T* __restrict__ w;
    const T* __restrict__ gout;
    T* __restrict__ gin;
    T* __restrict__ part;
    Geom g;
    Tiling t;
    int nstrips;
    int tps;  // tiles per strip
    int replicate;
    int ncopy;
    T fill;
    T scale;
};

template <typename T, int OP, int RH, bool IDENT>
__global__ __launch_bounds__(BLOCK) void morpho_bwd_pairs_kernel(const PairsParams<T> p)
{
    using Tr = OpTraits<OP, T>;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const Geom g = p.g;
    const Tiling t = p.t;
    const int tile_elems = t.rows * t.pitch;
    T* tile = reinterpret_cast<T*>(smem_raw);
    T* gtile = tile + tile_elems;
    T* bins = gtile + tile_elems;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    int work = xcd_work_index(blockIdx.x, gridDim.x);
    const int strip = work % p.nstrips;
    work /= p.nstrips;
    const int i = work % g.Cin;
    const int b = work / g.Cin;
    const int K = g.KH * g.KW, ph = g.pad_h(), pw = g.pad_w();
    const int64_t plane = g.plane();
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * K;
    const T* __restrict__ wb = p.w + (int64_t)b * g.wbs;
    T* part = p.part + ((int64_t)b * p.nstrips + strip) * wnumel;
    const T sign = (T)Tr::sign;
    const int copy = lane & (p.ncopy - 1);

    for (int j = threadIdx.x; j < K * p.ncopy; j += BLOCK) bins[j] = T(0);

    const int tile_begin = strip * p.tps;
    const int tile_end = min(tile_begin + p.tps, t.ntiles());
    for (int tid = tile_begin; tid < tile_end; ++tid)
    {
        const int ty = tid / t.ntx, tx = tid - ty * t.ntx;
        const int h0 = ty * t.th, w0 = tx * TILE_W;
        const int y0 = h0 + ph - (g.KH - 1), x0 = w0 + pw - (g.KW - 1);
        __syncthreads();
        stage_tile(tile, p.x + ((int64_t)b * g.Cin + i) * plane, g, t, y0, x0, p.replicate != 0, p.fill);
        for (int j = threadIdx.x; j < tile_elems; j += BLOCK) gtile[j] = T(0);
        __syncthreads();

        const int o_begin = IDENT ? i : 0;
        const int o_end = IDENT ? i + 1 : g.Cout;
        const int wc = w0 + lane;
        const T* tbase = tile + (wave * RH + g.KH - 1) * t.pitch + lane + g.KW - 1;
        for (int o = o_begin; o < o_end; ++o)
        {
            const int wi = IDENT ? 0 : i;
            const T* __restrict__ wp = wb + ((int64_t)o * g.Cw + wi) * K;
            T gr[RH], best[RH];
            int arg[RH];
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                const int h = h0 + wave * RH + r;
                gr[r] = (h < g.H && wc < g.W) ? p.gout[((int64_t)b * g.Cout + o) * plane + (int64_t)h * g.W + wc] * p.scale : T(0);
                best[r] = Tr::init();
                arg[r] = 0;
            }
            for (int kh = 0; kh < g.KH; ++kh)
            {
                const T* trow = tbase - kh * t.pitch;
                for (int kw = 0; kw < g.KW; ++kw)
                {
                    const T wk = wp[kh * g.KW + kw];
                    const int k = kh * g.KW + kw;
#pragma unroll
                    for (int r = 0; r < RH; ++r)
                    {
                        const T v = Tr::combine(trow[r * t.pitch - kw], wk);
                        if (Tr::better(v, best[r]))
                        {
                            best[r] = v;
                            arg[r] = k;
                        }
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                if (gr[r] == T(0)) continue;
                const int h = h0 + wave * RH + r;
                const int kh = arg[r] / g.KW, kw = arg[r] - kh * g.KW;
                const int iy = h + ph - kh, ix = wc + pw - kw;
                if (iy >= 0 && iy < g.H && ix >= 0 && ix < g.W) lds_add(&gtile[(wave * RH + r + g.KH - 1 - kh) * t.pitch + lane + g.KW - 1 - kw], gr[r]);
                lds_add(&bins[arg[r] * p.ncopy + copy], sign * gr[r]);
            }
            __syncthreads();
            for (int j = threadIdx.x; j < K; j += BLOCK)
            {
                T s = T(0);
                for (int c = 0; c < p.ncopy; ++c)
                {
                    s += bins[j * p.ncopy + c];
                    bins[j * p.ncopy + c] = T(0);
                }
                part[((int64_t)o * g.Cw + wi) * K + j] += s;
            }
            __syncthreads();
        }

        // This tile's grad_input contributions, including the halo shared with neighbouring tiles.
        T* gplane = p.gin + ((int64_t)b * g.Cin + i) * plane;
        for (int ly = wave; ly < t.rows; ly += NWAVES)
        {
            const int iy = y0 + ly;
            if (iy < 0 || iy >= g.H) continue;
            for (int lx = lane; lx < t.cols; lx += WAVE)
            {
                const int ix = x0 + lx;
                if (ix < 0 || ix >= g.W) continue;
                const T v = gtile[ly * t.pitch + lx];
                if (v != T(0)) global_add(&gplane[(int64_t)iy * g.W + ix], v);
            }
        }
    }
}

template <typename T>
__global__ __launch_bounds__(BLOCK) void fill_kernel(T* __restrict__ p, int64_t n, T v)
{
    for (int64_t j = (int64_t)blockIdx.x * BLOCK + threadIdx.x; j < n; j += (int64_t)gridDim.x * BLOCK) p[j] = v;
}

template <typename T>
__global__ __launch_bounds__(BLOCK) void reduce_slots_kernel(const T* __restrict__ part, int nslots, int64_t n, T* __restrict__ out)
{
    for (int64_t j = (int64_t)blockIdx.x * BLOCK + threadIdx.x; j < n; j += (int64_t)gridDim.x * BLOCK)
    {
        T s = T(0);
        for (int slot = 0; slot < nslots; ++slot) s += part[(int64_t)slot * n + j];
        out[j] = s;
    }
}

static int grid_for(int64_t n)
{
    const int64_t blocks = (n + BLOCK - 1) / BLOCK;
    return (int)(blocks < 8192 ? (blocks < 1 ? 1 : blocks) : 8192);
}

template <typename T>
hipError_t fill_async(T* p, int64_t n, T v, hipStream_t stream)
{
    if (n <= 0) return hipSuccess;
    fill_kernel<T><<<grid_for(n), BLOCK, 0, stream>>>(p, n, v);
    return hipGetLastError();
}

template <typename T>
hipError_t reduce_slots_async(const T* part, int nslots, int64_t n, T* out, hipStream_t stream)
{
    if (n <= 0) return hipSuccess;
    reduce_slots_kernel<T><<<grid_for(n), BLOCK, 0, stream>>>(part, nslots, n, out);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------
// Forward launch
// ------------------------------------------------------------------------------------------------

template <typename T>
size_t morpho_forward_lds(const Geom& g)
{
    const Tiling t = make_tiling(g, rows_per_wave<T>());
    return (size_t)t.rows * t.pitch * sizeof(T);
}

template <typename T, int OP, int MK, int OB, bool SAVE>
static hipError_t launch_fwd(const FwdParams<T>& p, hipStream_t stream)
{
    constexpr int RH = rows_per_wave<T>();
    const int64_t blocks = (int64_t)p.g.B * p.t.nty * p.t.ntx * p.nog;
    const size_t lds = (size_t)p.t.rows * p.t.pitch * sizeof(T);
    morpho_fwd_kernel<T, OP, MK, OB, RH, SAVE><<<(unsigned)blocks, BLOCK, lds, stream>>>(p);
    return hipGetLastError();
}

template <typename T, int OP>
static hipError_t forward_op(int merge, FwdParams<T> p, hipStream_t stream)
{
    const bool save = p.idx != nullptr;
    const bool group4 = p.g.Cout >= 4 && merge != MERGE_IDENTITY;
    p.nog = merge == MERGE_IDENTITY ? p.g.Cout : (group4 ? (p.g.Cout + 3) / 4 : p.g.Cout);
    switch (merge)
    {
        case MERGE_ADD:
        case MERGE_AVERAGE:
            p.average = merge == MERGE_AVERAGE;
            return group4 ? launch_fwd<T, OP, MK_SUM, 4, false>(p, stream) : launch_fwd<T, OP, MK_SUM, 1, false>(p, stream);
        case MERGE_MAX:
            if (save) return group4 ? launch_fwd<T, OP, MK_MAX, 4, true>(p, stream) : launch_fwd<T, OP, MK_MAX, 1, true>(p, stream);
            return group4 ? launch_fwd<T, OP, MK_MAX, 4, false>(p, stream) : launch_fwd<T, OP, MK_MAX, 1, false>(p, stream);
        case MERGE_MIN:
            if (save) return group4 ? launch_fwd<T, OP, MK_MIN, 4, true>(p, stream) : launch_fwd<T, OP, MK_MIN, 1, true>(p, stream);
            return group4 ? launch_fwd<T, OP, MK_MIN, 4, false>(p, stream) : launch_fwd<T, OP, MK_MIN, 1, false>(p, stream);
        case MERGE_IDENTITY: return launch_fwd<T, OP, MK_IDENT, 1, false>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

template <typename T>
hipError_t morpho_forward(int op, int merge, bool replicate, T fill, const T* x, const T* w, T* out, int32_t* indices, const Geom& g,
                          hipStream_t stream)
{
    if ((int64_t)g.B * g.Cout * g.plane() == 0) return hipSuccess;
    FwdParams<T> p{};
    p.x = x;
    p.w = w;
    p.out = out;
    p.idx = indices;
    p.g = g;
    p.t = make_tiling(g, rows_per_wave<T>());
    p.replicate = replicate ? 1 : 0;
    p.fill = fill;
    p.average = 0;
    return op == DILATION ? forward_op<T, DILATION>(merge, p, stream) : forward_op<T, EROSION>(merge, p, stream);
}

// ------------------------------------------------------------------------------------------------
// Backward launch
// ------------------------------------------------------------------------------------------------

struct ScatterPlan
{
    int nchunks;
    int64_t chunk;
    bool lds_bins;
    size_t part_bytes;
    size_t lds;
};

template <typename T>
static ScatterPlan plan_scatter(const Geom& g)
{
    ScatterPlan s{};
    const int64_t total = (int64_t)g.B * g.plane();
    const int64_t wnumel = (int64_t)g.Cout * g.Cin * g.taps();
    int64_t nchunks = (4096 + g.Cout - 1) / g.Cout;
    const int64_t max_chunks = (total + BLOCK - 1) / BLOCK;
    if (nchunks > max_chunks) nchunks = max_chunks;
    // Keep the partials within 256 MiB.
    while (nchunks > 1 && (size_t)nchunks * wnumel * sizeof(T) > ((size_t)256 << 20)) nchunks /= 2;
    if (nchunks < 1) nchunks = 1;
    s.nchunks = (int)nchunks;
    s.chunk = (total + nchunks - 1) / nchunks;
    const size_t bins = (size_t)g.Cin * g.taps() * sizeof(T);
    s.lds_bins = bins <= (size_t)48 * 1024;
    s.lds = s.lds_bins ? bins : 0;
    s.part_bytes = (size_t)nchunks * wnumel * sizeof(T);
    return s;
}

struct PairsPlan
{
    Tiling t;
    int nstrips;
    int tps;
    int ncopy;
    size_t part_bytes;
    size_t lds;
};

template <typename T>
static PairsPlan plan_pairs(int merge, const Geom& g)
{
    PairsPlan s{};
    s.t = make_tiling(g, rows_per_wave<T>());
    s.ncopy = 16;
    const int64_t units = (int64_t)g.B * g.Cin;
    const int ntiles = s.t.ntiles();
    int64_t nstrips = (2048 + units - 1) / units;
    if (nstrips > ntiles) nstrips = ntiles;
    if (nstrips < 1) nstrips = 1;
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * g.taps();
    while (nstrips > 1 && (size_t)g.B * nstrips * wnumel * sizeof(T) > ((size_t)256 << 20)) nstrips = (nstrips + 1) / 2;
    s.tps = (int)((ntiles + nstrips - 1) / nstrips);
    s.nstrips = (int)((ntiles + s.tps - 1) / s.tps);
    s.part_bytes = (size_t)g.B * s.nstrips * wnumel * sizeof(T);
    s.lds = (2 * (size_t)s.t.rows * s.t.pitch + (size_t)g.taps() * s.ncopy) * sizeof(T);
    (void)merge;
    return s;
}

template <typename T>
size_t morpho_backward_lds(int merge, const Geom& g)
{
    if (merge == MERGE_MAX || merge == MERGE_MIN) return morpho_forward_lds<T>(g);
    return plan_pairs<T>(merge, g).lds;
}

template <typename T>
size_t morpho_backward_workspace(int merge, bool has_indices, const Geom& g)
{
    if (merge == MERGE_MAX || merge == MERGE_MIN)
    {
        size_t bytes = align_up(plan_scatter<T>(g).part_bytes);
        if (!has_indices)
        {
            const size_t n = (size_t)g.B * g.Cout * g.plane();
            bytes += align_up(n * sizeof(int32_t)) + align_up(n * sizeof(T));
        }
        return bytes;
    }
    return align_up(plan_pairs<T>(merge, g).part_bytes);
}

template <typename T, int OP>
static hipError_t backward_op(int merge, bool replicate, T fill, const T* x, const T* w, const int32_t* indices, const T* grad_out,
                              T* grad_in, T* grad_w, const Geom& g, unsigned char* ws, hipStream_t stream)
{
    hipError_t err;
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * g.taps();
    if ((err = fill_async<T>(grad_in, (int64_t)g.B * g.Cin * g.plane(), T(0), stream)) != hipSuccess) return err;
    if ((int64_t)g.B * g.Cout * g.plane() == 0) return fill_async<T>(grad_w, wnumel, T(0), stream);

    if (merge == MERGE_MAX || merge == MERGE_MIN)
    {
        const ScatterPlan s = plan_scatter<T>(g);
        T* part = reinterpret_cast<T*>(ws);
        ws += align_up(s.part_bytes);
        if (!indices)
        {
            // Winners were not saved by the forward: regenerate them.
            const size_t n = (size_t)g.B * g.Cout * g.plane();
            int32_t* idx = reinterpret_cast<int32_t*>(ws);
            T* tmp_out = reinterpret_cast<T*>(ws + align_up(n * sizeof(int32_t)));
            if ((err = morpho_forward<T>(OP, merge, replicate, fill, x, w, tmp_out, idx, g, stream)) != hipSuccess) return err;
            indices = idx;
        }
        if (!s.lds_bins)
            if ((err = fill_async<T>(part, (int64_t)s.nchunks * wnumel, T(0), stream)) != hipSuccess) return err;
        ScatterParams<T> p{};
        p.idx = indices;
        p.gout = grad_out;
        p.gin = grad_in;
        p.part = part;
        p.g = g;
        p.nchunks = s.nchunks;
        p.lds_bins = s.lds_bins ? 1 : 0;
        p.chunk = s.chunk;
        morpho_bwd_scatter_kernel<T, OP><<<(unsigned)((int64_t)s.nchunks * g.Cout), BLOCK, s.lds, stream>>>(p);
        if ((err = hipGetLastError()) != hipSuccess) return err;
        return reduce_slots_async<T>(part, s.nchunks, wnumel, grad_w, stream);
    }

    const PairsPlan s = plan_pairs<T>(merge, g);
    T* part = reinterpret_cast<T*>(ws);
    const int nslots = g.B * s.nstrips;
    if ((err = fill_async<T>(part, (int64_t)nslots * wnumel, T(0), stream)) != hipSuccess) return err;
    PairsParams<T> p{};
    p.x = x;
    p.w = w;
    p.gout = grad_out;
    p.gin = grad_in;
    p.part = part;
    p.g = g;
    p.t = s.t;
    p.nstrips = s.nstrips;
    p.tps = s.tps;
    p.replicate = replicate ? 1 : 0;
    p.ncopy = s.ncopy;
    p.fill = fill;
    p.scale = merge == MERGE_AVERAGE ? T(1) / (T)g.Cin : T(1);
    constexpr int RH = rows_per_wave<T>();
    const unsigned blocks = (unsigned)((int64_t)g.B * g.Cin * s.nstrips);
    if (merge == MERGE_IDENTITY)
        morpho_bwd_pairs_kernel<T, OP, RH, true><<<blocks, BLOCK, s.lds, stream>>>(p);
    else
        morpho_bwd_pairs_kernel<T, OP, RH, false><<<blocks, BLOCK, s.lds, stream>>>(p);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    return reduce_slots_async<T>(part, nslots, wnumel, grad_w, stream);
}

template <typename T>
hipError_t morpho_backward(int op, int merge, bool replicate, T fill, const T* x, const T* w, const int32_t* indices, const T* grad_out,
                           T* grad_in, T* grad_w, const Geom& g, void* workspace, size_t workspace_bytes, hipStream_t stream)
{
    if (workspace_bytes < morpho_backward_workspace<T>(merge, indices != nullptr, g)) return hipErrorInvalidValue;
    unsigned char* ws = reinterpret_cast<unsigned char*>(workspace);
    return op == DILATION ? backward_op<T, DILATION>(merge, replicate, fill, x, w, indices, grad_out, grad_in, grad_w, g, ws, stream)
                          : backward_op<T, EROSION>(merge, replicate, fill, x, w, indices, grad_out, grad_in, grad_w, g, ws, stream);
}

#define MCA_INSTANTIATE(T)                                                                                                              \
    template hipError_t morpho_forward<T>(int, int, bool, T, const T*, const T*, T*, int32_t*, const Geom&, hipStream_t);              \
    template size_t morpho_forward_lds<T>(const Geom&);                                                                                 \
    template size_t morpho_backward_workspace<T>(int, bool, const Geom&);                                                               \
    template size_t morpho_backward_lds<T>(int, const Geom&);                                                                           \
    template hipError_t morpho_backward<T>(int, int, bool, T, const T*, const T*, const int32_t*, const T*, T*, T*, const Geom&, void*, \
                                           size_t, hipStream_t);                                                                        \
    template hipError_t fill_async<T>(T*, int64_t, T, hipStream_t);                                                                     \
    template hipError_t reduce_slots_async<T>(const T*, int, int64_t, T*, hipStream_t);

MCA_INSTANTIATE(float)
MCA_INSTANTIATE(double)

}  // namespace mca
