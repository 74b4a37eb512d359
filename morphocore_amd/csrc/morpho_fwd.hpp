// Dilation / erosion forward for gfx950.
//
// A workgroup owns one output tile (64 columns x 4*RH rows) of one batch element for OB output
// channels, and walks the input channels in order. Each input plane's tile plus its halo is staged
// in LDS once and shared by the OB output channels; the structuring element values are
// wave-uniform (scalar loads). Three modes:
//   VALUE  the per-pair extremum with the NaN-ignoring max/min (v_max3 / v_min3: ~1.5 VALU ops per
//          tap), merged over input channels in the reference's order and comparisons;
//   TAPS   (ADD / AVERAGE / IDENTITY, when the backward pass will need them) the strict first-tap
//          scan of every pair in the reference's tap order (kh, then kw), writing each pair's tap;
//   PACKED (MAX / MIN) VALUE plus the packed (channel << 16 | tap) winner of every output pixel.
// The winning tap of a MAX / MIN merge is found by one rescan of the winning channel (the first tap
// equal to the winning value, which is the tap the strict scan keeps), which also restores the sign
// of a zero result (the NaN-ignoring max does not order -0 and +0). The static kernels of 5x5 and
// larger elements rescan channel by channel from LDS, after sorting the workgroup's pixels by winning
// channel; the others rescan each pixel from global memory.
//
// The static kernel (morpho_fwd_static) is compiled for the structuring-element sizes of the common
// layers, holds each thread's input window in registers and double-buffers the LDS tile; the
// generic kernel (morpho_fwd_generic) takes any size at runtime.
#pragma once

#include <type_traits>

#include "launch.hpp"

namespace mca
{

enum FwdMode : int
{
    FWD_VALUE = 0,
    FWD_TAPS = 1,
    FWD_PACKED = 2
};

template <typename ST>
struct FwdParams
{
    const ST* __restrict__ x;
    const ST* __restrict__ w;
    ST* __restrict__ out;
    void* __restrict__ idx;
    Geom g;
    Tiling t;
    int nog;
    int chans;  // static kernel, IDENTITY: consecutive channels per workgroup (else 1)
    int replicate;
    int average;
    compute_t<ST> fill;
};

struct FwdWork
{
    int b, og, tx, ty;
};

__device__ __forceinline__ FwdWork decode_fwd(int nog, const Tiling& t)
{
    int work = xcd_work_index(blockIdx.x, gridDim.x);
    FwdWork w;
    w.og = work % nog;
    work /= nog;
    w.tx = work % t.ntx;
    work /= t.ntx;
    w.ty = work % t.nty;
    w.b = work / t.nty;
    return w;
}

template <typename T, int MK>
__device__ __forceinline__ T merge_init()
{
    return MK == MK_MAX ? lowest_of<T>() : (MK == MK_MIN ? max_of<T>() : T(0));
}

// Channel merge of one pair result `bv` of input channel i (morpho_merge_policy.hpp:10-86,
// morpho_op_cpu_kernels.hxx:364-395): ADD sums in channel order; MAX / MIN keep channel 0 as the
// provisional winner and replace it only by a strictly better channel.
template <typename T, int MK>
__device__ __forceinline__ void merge_pair(T bv, int i, T& acc, int& win)
{
    if constexpr (MK == MK_SUM)
    {
        acc = acc + bv;
    }
    else if constexpr (MK == MK_MAX)
    {
        if (i == 0 || bv > acc) win = i;
        acc = acc < bv ? bv : acc;
    }
    else if constexpr (MK == MK_MIN)
    {
        if (i == 0 || bv < acc) win = i;
        acc = bv < acc ? bv : acc;
    }
    else
    {
        acc = bv;
        win = i;
    }
}

// Finalises and stores one output pixel; for MAX / MIN / IDENTITY rescans the winning channel when
// its tap is needed (PACKED) or when the result is zero (sign of the first zero tap). The merged
// value is the winning channel's extremum, so it is the value to look for, unless it is the merge's
// clamp (lowest() / max()): then channel 0 won without a strictly better channel after it, and its
// extremum may lie beyond the clamp (an infinite tap), so that extremum is recomputed and looked for.
template <typename ST, int OP, int MK, int MODE>
__device__ __forceinline__ void store_output(const FwdParams<ST>& p, int b, int o, int h, int wc, int i_count, compute_t<ST> acc, int win)
{
    using T = compute_t<ST>;
    using Tr = OpTraits<OP, T>;
    const Geom& g = p.g;
    T v = acc;
    if constexpr (MK == MK_SUM)
    {
        if (p.average) v = v / (T)g.Cin;
    }
    int32_t packed = 0;
    if constexpr (MK != MK_SUM)
    {
        if ((MODE == FWD_PACKED || v == T(0)) && i_count > 0)
        {
            const int K = g.KH * g.KW, ph = g.KH / 2, pw = g.KW / 2;
            const int c = win;
            const ST* __restrict__ wp = p.w + (int64_t)b * g.wbs + ((int64_t)o * g.Cw + (MK == MK_IDENT ? 0 : c)) * K;
            const ST* __restrict__ xp = p.x + ((int64_t)b * g.Cin + c) * g.plane();
            int karg = 0;
            T target = acc;
            if constexpr (MK == MK_MAX || MK == MK_MIN)
            {
                if (acc == merge_init<T, MK>())
                {
                    target = Tr::init();
                    for (int kh = 0; kh < g.KH; ++kh)
                        for (int kw = 0; kw < g.KW; ++kw)
                        {
                            const int y = h + ph - kh, x = wc + pw - kw;
                            const T raw = (T)xp[(int64_t)clampi(y, 0, g.H - 1) * g.W + clampi(x, 0, g.W - 1)];
                            const bool inb = y >= 0 && y < g.H && x >= 0 && x < g.W;
                            target = Tr::pick(target, Tr::combine(inb || p.replicate ? raw : p.fill, (T)wp[kh * g.KW + kw]));
                        }
                }
            }
            if (target != Tr::init())
            {
                // Taps in chunks of 4 whose loads are all in flight together (the rescan is a chain of
                // dependent global loads otherwise); the first equal tap of the first chunk holding
                // one wins.
                constexpr int CH = 4;
                int kh0 = 0, kw0 = 0, found = -1;
                T fval = T(0);
                for (int k0 = 0; k0 < K && found < 0; k0 += CH)
                {
                    T val[CH];
                    int kh = kh0, kw = kw0;
#pragma unroll
                    for (int j = 0; j < CH; ++j)
                    {
                        // read_padded with an unconditional (clamped, in-bounds) load
                        const int kk = min(k0 + j, K - 1);
                        const int y = h + ph - kh, x = wc + pw - kw;
                        const T raw = (T)xp[(int64_t)clampi(y, 0, g.H - 1) * g.W + clampi(x, 0, g.W - 1)];
                        const bool inb = y >= 0 && y < g.H && x >= 0 && x < g.W;
                        val[j] = Tr::combine(inb || p.replicate ? raw : p.fill, (T)wp[kk]);
                        if (++kw == g.KW)
                        {
                            kw = 0;
                            ++kh;
                        }
                    }
                    kh0 = kh;
                    kw0 = kw;
#pragma unroll
                    for (int j = CH - 1; j >= 0; --j)
                    {
                        const bool hit = k0 + j < K && val[j] == target;
                        found = hit ? k0 + j : found;
                        fval = hit ? val[j] : fval;
                    }
                }
                if (found >= 0)
                {
                    karg = found;
                    if (v == T(0)) v = fval;
                }
            }
            packed = (int32_t)((c << 16) | karg);
        }
    }
    const int64_t oi = ((int64_t)b * g.Cout + o) * g.plane() + (int64_t)h * g.W + wc;
    p.out[oi] = (ST)v;
    if constexpr (MODE == FWD_PACKED) static_cast<int32_t*>(p.idx)[oi] = packed;
}

// Index of channel pair (o, i)'s tap of output pixel (h, w) in the saved TAPS array.
__device__ __forceinline__ int64_t pair_tap_index(const Geom& g, bool ident, int b, int o, int i, int h, int wc)
{
    const int cpair = ident ? 1 : g.Cin;
    return (((int64_t)b * g.Cout + o) * cpair + (ident ? 0 : i)) * g.plane() + (int64_t)h * g.W + wc;
}

// ------------------------------------------------------------------------------------------------
// Generic kernel: any structuring element, read tap by tap from the LDS tile.
// ------------------------------------------------------------------------------------------------

template <typename ST, int OP, int MK, int OB, int RH, int MODE, typename AT>
__global__ __launch_bounds__(BLOCK) void morpho_fwd_generic(const FwdParams<ST> p)
{
    using T = compute_t<ST>;
    using Tr = OpTraits<OP, T>;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    T* tile = reinterpret_cast<T*>(smem_raw);
    const Geom g = p.g;
    const Tiling t = p.t;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const FwdWork wk = decode_fwd(p.nog, t);
    const int b = wk.b;
    const int h0 = wk.ty * t.th, w0 = wk.tx * TILE_W, o0 = wk.og * OB;
    const int K = g.KH * g.KW, ph = g.pad_h(), pw = g.pad_w();
    const int y0 = h0 + ph - (g.KH - 1), x0 = w0 + pw - (g.KW - 1);
    const int64_t plane = g.plane();
    const ST* __restrict__ wb = p.w + (int64_t)b * g.wbs;
    const int wc = w0 + lane;
    constexpr bool ident = MK == MK_IDENT;

    T acc[OB][RH];
    int win[OB][RH];
#pragma unroll
    for (int ob = 0; ob < OB; ++ob)
#pragma unroll
        for (int r = 0; r < RH; ++r)
        {
            acc[ob][r] = merge_init<T, MK>();
            win[ob][r] = 0;
        }

    const int i_begin = ident ? o0 : 0;
    const int i_end = ident ? o0 + 1 : g.Cin;
    const T* tbase = tile + (wave * RH + g.KH - 1) * t.pitch + lane + g.KW - 1;
    for (int i = i_begin; i < i_end; ++i)
    {
        __syncthreads();
        stage_tile(tile, p.x + ((int64_t)b * g.Cin + i) * plane, g, t, y0, x0, p.replicate != 0, p.fill);
        __syncthreads();

        const ST* wi[OB];
#pragma unroll
        for (int ob = 0; ob < OB; ++ob) wi[ob] = wb + ((int64_t)min(o0 + ob, g.Cout - 1) * g.Cw + (ident ? 0 : i)) * K;

        T best[OB][RH];
        int arg[OB][RH];
#pragma unroll
        for (int ob = 0; ob < OB; ++ob)
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                best[ob][r] = Tr::init();
                arg[ob][r] = 0;
            }
        for (int kh = 0; kh < g.KH; ++kh)
        {
            const T* trow = tbase - kh * t.pitch;
            for (int kw = 0; kw < g.KW; ++kw)
            {
                const int k = kh * g.KW + kw;
                T wv[OB];
#pragma unroll
                for (int ob = 0; ob < OB; ++ob) wv[ob] = (T)wi[ob][k];
#pragma unroll
                for (int r = 0; r < RH; ++r)
                {
                    const T xv = trow[r * t.pitch - kw];
#pragma unroll
                    for (int ob = 0; ob < OB; ++ob)
                    {
                        const T v = Tr::combine(xv, wv[ob]);
                        if constexpr (MODE == FWD_TAPS)
                        {
                            if (Tr::better(v, best[ob][r]))
                            {
                                best[ob][r] = v;
                                arg[ob][r] = k;
                            }
                        }
                        else
                        {
                            best[ob][r] = Tr::pick(best[ob][r], v);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int ob = 0; ob < OB; ++ob)
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                merge_pair<T, MK>(best[ob][r], i, acc[ob][r], win[ob][r]);
                if constexpr (MODE == FWD_TAPS)
                {
                    const int o = o0 + ob, h = h0 + wave * RH + r;
                    if (o < g.Cout && h < g.H && wc < g.W) static_cast<AT*>(p.idx)[pair_tap_index(g, ident, b, o, i, h, wc)] = (AT)arg[ob][r];
                }
            }
    }

#pragma unroll
    for (int ob = 0; ob < OB; ++ob)
#pragma unroll
        for (int r = 0; r < RH; ++r)
        {
            const int o = o0 + ob, h = h0 + wave * RH + r;
            if (o >= g.Cout || h >= g.H || wc >= g.W) continue;
            store_output<ST, OP, MK, MODE>(p, b, o, h, wc, i_end - i_begin, acc[ob][r], win[ob][r]);
        }
}

// ------------------------------------------------------------------------------------------------
// Static kernel: structuring element size known at compile time.
// ------------------------------------------------------------------------------------------------

template <int KH, int KW, int RH>
struct StaticTile
{
    static constexpr int K = KH * KW;
    static constexpr int TH = NWAVES * RH;
    static constexpr int ROWS = TH + KH - 1;
    static constexpr int COLS = TILE_W + KW - 1;
    static constexpr int ELEMS = ROWS * COLS;
    static constexpr int NS = (ELEMS + BLOCK - 1) / BLOCK;  // staged elements per thread
    static constexpr int WR = RH + KH - 1;                  // window rows of one thread
};

// The PACKED winner rescan runs by channel from LDS for elements of at least this many taps and up to
// this many input channels (a bucket start per channel in LDS); smaller elements rescan each pixel from
// global memory, which costs fewer staging passes than it saves.
constexpr int BUCKET_MIN_TAPS = 25;
constexpr int BUCKET_MAX_CIN = 256;

// Structuring-element values of the workgroup's OB output channels for one input channel, staged
// with the input tile and read by every lane at the same LDS address (a broadcast).
template <int OB, int K>
struct StaticWeights
{
    static constexpr int ELEMS = OB * K;
    static constexpr int NW = (ELEMS + BLOCK - 1) / BLOCK;
};

// The channel-sorted winner rescan (bucket_rescan) is held to the channel loop's four waves per SIMD.
template <int MODE, int MK, int OB, int RH, int K>
constexpr bool bucket_rescan()
{
    return MODE == FWD_PACKED && MK != MK_IDENT && OB * RH > 1 && K >= BUCKET_MIN_TAPS;
}

template <typename ST, int OP, int MK, int KH, int KW, int OB, int RH, int MODE>
__global__ __launch_bounds__(BLOCK) __attribute__((amdgpu_waves_per_eu(bucket_rescan<MODE, MK, OB, RH, KH * KW>() ? 4 : 1, 8))) void
morpho_fwd_static(const FwdParams<ST> p)
{
    using T = compute_t<ST>;
    using Tr = OpTraits<OP, T>;
    using S = StaticTile<KH, KW, RH>;
    using SW = StaticWeights<OB, KH * KW>;
    constexpr int K = S::K, COLS = S::COLS, NS = S::NS, WR = S::WR, NW = SW::NW;
    constexpr bool ident = MK == MK_IDENT;
    constexpr bool BUCKET = bucket_rescan<MODE, MK, OB, RH, K>();
    __shared__ T tiles[2][S::ELEMS];
    __shared__ T wts[2][SW::ELEMS];
    // Winner rescan by channel (BUCKET): bucket starts per input channel, then the workgroup's
    // pixel-channel items sorted by winning channel (an item id, replaced by its result).
    __shared__ int rstart[BUCKET ? BUCKET_MAX_CIN + 1 : 1];
    __shared__ uint16_t rbucket[BUCKET ? BLOCK * OB * RH : 1];

    const Geom& g = p.g;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const FwdWork wk = decode_fwd(p.nog, p.t);
    const int b = wk.b;
    const int h0 = wk.ty * S::TH, w0 = wk.tx * TILE_W, o0 = wk.og * (ident ? p.chans : OB);
    const int y0 = h0 + KH / 2 - (KH - 1), x0 = w0 + KW / 2 - (KW - 1);
    const int64_t plane = g.plane();
    const ST* __restrict__ wb = p.w + (int64_t)b * g.wbs;
    const int wc = w0 + lane;

    // Staging plan, the same for every input channel: plane offset of each element this thread
    // stages (-1: the fill value).
    int off[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j)
    {
        const int idx = threadIdx.x + j * BLOCK;
        const int ly = idx / COLS, lx = idx - ly * COLS;
        const int y = y0 + ly, x = x0 + lx;
        if (y >= 0 && y < g.H && x >= 0 && x < g.W)
            off[j] = y * g.W + x;
        else if (p.replicate)
            off[j] = clampi(y, 0, g.H - 1) * g.W + clampi(x, 0, g.W - 1);
        else
            off[j] = -1;
    }
    // Structuring-element rows this thread stages: output channel o0 + ob, tap k (clamped to a
    // valid channel past Cout; those values are never used).
    int woff[NW];
#pragma unroll
    for (int j = 0; j < NW; ++j)
    {
        const int idx = min((int)threadIdx.x + j * BLOCK, SW::ELEMS - 1);
        const int ob = idx / K, k = idx - ob * K;
        woff[j] = ident ? k : (min(o0 + ob, g.Cout - 1) * g.Cw) * K + k;
    }
    const ST* __restrict__ xb = p.x + (int64_t)b * g.Cin * plane;
    T pre[NS], wpre[NW];
    auto load = [&](int i) {
        const ST* __restrict__ pl = xb + (int64_t)i * plane;
#pragma unroll
        for (int j = 0; j < NS; ++j) pre[j] = off[j] >= 0 ? (T)pl[off[j]] : p.fill;
        const ST* __restrict__ wi = wb + (int64_t)i * K;  // IDENTITY: channel i's own element
#pragma unroll
        for (int j = 0; j < NW; ++j) wpre[j] = (T)wi[woff[j]];
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int j = 0; j < NS; ++j)
        {
            const int idx = threadIdx.x + j * BLOCK;
            if (j < NS - 1 || idx < S::ELEMS) tiles[buf][idx] = pre[j];
        }
#pragma unroll
        for (int j = 0; j < NW; ++j)
        {
            const int idx = threadIdx.x + j * BLOCK;
            if (idx < SW::ELEMS) wts[buf][idx] = wpre[j];
        }
    };

    T acc[OB][RH];
    int win[OB][RH];
#pragma unroll
    for (int ob = 0; ob < OB; ++ob)
#pragma unroll
        for (int r = 0; r < RH; ++r)
        {
            acc[ob][r] = merge_init<T, MK>();
            win[ob][r] = 0;
        }

    // IDENTITY walks its p.chans channels as the other merges walk the input channels (next tile
    // prefetched), storing each channel's outputs after its scan.
    const int i_begin = ident ? o0 : 0;
    const int i_end = ident ? min(o0 + p.chans, g.Cout) : g.Cin;
    load(i_begin);
    store(0);
    __syncthreads();
    for (int i = i_begin; i < i_end; ++i)
    {
        const int buf = (i - i_begin) & 1;
        const bool more = i + 1 < i_end;
        if (more) load(i + 1);  // in flight while this channel computes
        const T* tb = &tiles[buf][wave * RH * COLS + lane + KW - 1];

        if constexpr (MODE == FWD_TAPS)
        {
            // The first tap (kh, then kw) reaching the pair's extremum, in two levels: each kernel
            // row folds to its extremum with max3 / min3, and a strict comparison per row finds the
            // first row that holds the overall extremum (every earlier row is strictly worse); the
            // first tap of that row equal to the extremum is then found by a short reverse scan
            // from LDS. A pair that never improves on the start value (all taps -inf / NaN for
            // dilation) keeps tap 0, as the strict scan does.
            T wnd[WR][KW];
#pragma unroll
            for (int rr = 0; rr < WR; ++rr)
#pragma unroll
                for (int kw = 0; kw < KW; ++kw) wnd[rr][kw] = tb[rr * COLS - kw];
            // Up to 5x5 the taps are stored after every pair's scan, so that the scans form one basic
            // block in which the LDS reads of one pair overlap the arithmetic of the others; larger
            // elements store each pair's tap at once (the deferred form needs more registers than
            // leave two waves per SIMD).
            constexpr bool DEFER = K <= 25;
            // Up to 5x5 the first row holding the extremum and its values are selected from the
            // registers that computed them; larger elements read that row again from LDS (a
            // per-lane row: bank conflicts between lanes on different rows).
            constexpr bool SELECT = K <= (sizeof(T) == 4 ? 25 : 9);
            using AT = std::conditional_t<(K <= 256), uint8_t, uint16_t>;
            const int hw = h0 + __builtin_amdgcn_readfirstlane(wave) * RH;  // the wave's first row
            auto store_tap = [&](int ob, int r, int a) {
                const int o = ident ? i : o0 + ob;
                if (o < g.Cout && hw + r < g.H && wc < g.W)
                    (static_cast<AT*>(p.idx) + pair_tap_index(g, ident, b, o, i, hw, w0))[r * g.W + lane] = (AT)a;
            };
            int arg[OB][RH];
#pragma unroll
            for (int ob = 0; ob < OB; ++ob)
            {
                const T* wp = &wts[buf][ob * K];
#pragma unroll
                for (int r = 0; r < RH; ++r)
                {
                    // Row extrema m[kh] (NaN when a whole row is NaN), the pair's extremum from the
                    // start value, then the first row holding it: rows that hold only NaN never
                    // compare equal, and a pair that never improves on the start value keeps tap 0.
                    T m[KH];
                    T v[KH][KW];
#pragma unroll
                    for (int kh = 0; kh < KH; ++kh)
                    {
#pragma unroll
                        for (int kw = 0; kw < KW; ++kw) v[kh][kw] = Tr::combine(wnd[r + KH - 1 - kh][kw], wp[kh * KW + kw]);
                        // A linear chain, which the compiler folds into max3 / min3 pairs.
                        T mm = v[kh][0];
#pragma unroll
                        for (int kw = 1; kw < KW; ++kw) mm = Tr::pick(mm, v[kh][kw]);
                        m[kh] = mm;
                    }
                    T best = Tr::init();
#pragma unroll
                    for (int kh = 0; kh < KH; ++kh) best = Tr::pick(best, m[kh]);
                    int krow = 0, kcol = 0;
                    if constexpr (SELECT)
                    {
                        // The first row holding the extremum, and its tap values, selected from
                        // registers (the last row stands when none holds it: then best is the start
                        // value and the tap is 0 below).
                        krow = KH - 1;
                        T rv[KW];
#pragma unroll
                        for (int kw = 0; kw < KW; ++kw) rv[kw] = v[KH - 1][kw];
#pragma unroll
                        for (int kh = KH - 2; kh >= 0; --kh)
                        {
                            const bool eq = m[kh] == best;
                            krow = eq ? kh : krow;
#pragma unroll
                            for (int kw = 0; kw < KW; ++kw) rv[kw] = eq ? v[kh][kw] : rv[kw];
                        }
#pragma unroll
                        for (int kw = KW - 1; kw >= 0; --kw) kcol = rv[kw] == best ? kw : kcol;
                    }
                    else
                    {
#pragma unroll
                        for (int kh = KH - 1; kh >= 0; --kh) krow = m[kh] == best ? kh : krow;
                        const T* xrow = tb + (r + KH - 1 - krow) * COLS;
                        const T* wrow = wp + krow * KW;
#pragma unroll
                        for (int kw = KW - 1; kw >= 0; --kw) kcol = Tr::combine(xrow[-kw], wrow[kw]) == best ? kw : kcol;
                    }
                    arg[ob][r] = best == Tr::init() ? 0 : krow * KW + kcol;
                    merge_pair<T, MK>(best, i, acc[ob][r], win[ob][r]);
                    if constexpr (!DEFER) store_tap(ob, r, arg[ob][r]);
                }
            }
            if constexpr (DEFER)
            {
                // The asm uses keep the compiler from sinking each pair's column scan into its
                // conditional store.
#pragma unroll
                for (int ob = 0; ob < OB; ++ob)
#pragma unroll
                    for (int r = 0; r < RH; ++r) asm volatile("" ::"v"(arg[ob][r]));
#pragma unroll
                for (int ob = 0; ob < OB; ++ob)
#pragma unroll
                    for (int r = 0; r < RH; ++r) store_tap(ob, r, arg[ob][r]);
            }
        }
        else
        {
            // Values only: the order of the taps does not matter, so one column of the window is
            // live at a time (kw outer) and pairs of taps fold into one max3 / min3.
            T best[OB][RH];
#pragma unroll
            for (int ob = 0; ob < OB; ++ob)
#pragma unroll
                for (int r = 0; r < RH; ++r) best[ob][r] = Tr::init();
#pragma unroll
            for (int kw = 0; kw < KW; ++kw)
            {
                // One column at a time: keeps the scheduler from gathering the LDS reads of every
                // column (window and structuring element) ahead of the arithmetic, which needs more
                // registers than a SIMD has.
                __builtin_amdgcn_sched_barrier(0);
                T col[WR];
#pragma unroll
                for (int rr = 0; rr < WR; ++rr) col[rr] = tb[rr * COLS - kw];
#pragma unroll
                for (int ob = 0; ob < OB; ++ob)
                {
                    const T* wp = &wts[buf][ob * K];
#pragma unroll
                    for (int r = 0; r < RH; ++r)
                    {
                        T m = best[ob][r];
#pragma unroll
                        for (int kh = 0; kh + 1 < KH; kh += 2)
                            m = Tr::pick(m, Tr::pick(Tr::combine(col[r + KH - 1 - kh], wp[kh * KW + kw]),
                                                     Tr::combine(col[r + KH - 2 - kh], wp[(kh + 1) * KW + kw])));
                        if constexpr (KH % 2 == 1) m = Tr::pick(m, Tr::combine(col[r], wp[(KH - 1) * KW + kw]));
                        best[ob][r] = m;
                    }
                }
            }
#pragma unroll
            for (int ob = 0; ob < OB; ++ob)
#pragma unroll
                for (int r = 0; r < RH; ++r)
                {
                    // Pins the column folds before the next tile's LDS store (the compiler would sink
                    // them past it, keeping every column's window and weights live at once).
                    asm volatile("" ::"v"(best[ob][r]));
                    merge_pair<T, MK>(best[ob][r], i, acc[ob][r], win[ob][r]);
                }
        }

        if constexpr (ident)
        {
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                const int h = h0 + wave * RH + r;
                if (h < g.H && wc < g.W) store_output<ST, OP, MK, MODE>(p, b, i, h, wc, 1, acc[0][r], win[0][r]);
            }
        }
        if (more) store(buf ^ 1);
        __syncthreads();
    }

    if constexpr (BUCKET)
    {
        if (g.Cin >= 1 && g.Cin <= BUCKET_MAX_CIN)
        {
            // The winning tap of every output pixel, found channel by channel from LDS instead of one
            // lane at a time from global memory (whose scattered loads, one plane per lane, bound the
            // per-pixel rescan): the items (output channel, pixel) are sorted by winning channel, each
            // winning channel's tile and elements are staged again, and each item's pair is scanned
            // strictly in tap order (kh, then kw). Its first extremal tap is the first tap equal to the
            // merged value, which is that pair's extremum; a zero result takes that tap's sign.
            constexpr int ITEMS = OB * RH;
            const int hw0 = h0 + wave * RH;
            for (int c = threadIdx.x; c < g.Cin; c += BLOCK) rstart[c] = 0;
            __syncthreads();
            // Each item's rank in its channel's bucket, then its bucket position, kept in the upper half of
            // its winner register (NOPOS: nothing to find, tap 0).
            constexpr int NOPOS = 0xffff;
#pragma unroll
            for (int ob = 0; ob < OB; ++ob)
#pragma unroll
                for (int r = 0; r < RH; ++r)
                {
                    const bool need = o0 + ob < g.Cout && hw0 + r < g.H && wc < g.W && acc[ob][r] != Tr::init();
                    const int rank = need ? atomicAdd(&rstart[win[ob][r]], 1) : NOPOS;
                    win[ob][r] |= (int)((unsigned)rank << 16);
                }
            __syncthreads();
            // Bucket starts: an exclusive prefix over the channels' counts, in the first wave.
            if (wave == 0)
            {
                constexpr int PER = BUCKET_MAX_CIN / WAVE;
                int cnt[PER], s = 0;
#pragma unroll
                for (int j = 0; j < PER; ++j)
                {
                    const int c = lane * PER + j;
                    cnt[j] = c < g.Cin ? rstart[c] : 0;
                    s += cnt[j];
                }
                int incl = s;
#pragma unroll
                for (int d = 1; d < WAVE; d <<= 1)
                {
                    const int t = __shfl_up(incl, d);
                    if (lane >= d) incl += t;
                }
                int base = incl - s;
#pragma unroll
                for (int j = 0; j < PER; ++j)
                {
                    const int c = lane * PER + j;
                    if (c < g.Cin) rstart[c] = base;
                    base += cnt[j];
                }
                if (lane == WAVE - 1) rstart[g.Cin] = incl;
            }
            __syncthreads();
#pragma unroll
            for (int ob = 0; ob < OB; ++ob)
#pragma unroll
                for (int r = 0; r < RH; ++r)
                    if (((unsigned)win[ob][r] >> 16) != NOPOS)
                    {
                        const int c = win[ob][r] & 0xffff;
                        const int at = (int)((unsigned)win[ob][r] >> 16) + rstart[c];
                        win[ob][r] = c | (int)((unsigned)at << 16);
                        rbucket[at] = (uint16_t)(threadIdx.x * ITEMS + ob * RH + r);
                    }
            __syncthreads();
            // The winning channels in order, each tile staged behind the previous channel's scans (as
            // the channel loop above).
            auto next_won = [&](int c) {
                while (c < g.Cin && rstart[c + 1] == rstart[c]) ++c;
                return c;
            };
            int c = next_won(0);
            if (c < g.Cin)
            {
                load(c);
                store(0);
                __syncthreads();
                int buf = 0;
                while (c < g.Cin)
                {
                    const int cn = next_won(c + 1);
                    if (cn < g.Cin) load(cn);
                    const int e1 = rstart[c + 1];
                    for (int e = rstart[c] + threadIdx.x; e < e1; e += BLOCK)
                    {
                        const int id = rbucket[e];
                        const int t = id / ITEMS, s = id - t * ITEMS;
                        const int ob = s / RH, r = s - ob * RH;
                        const T* xp = &tiles[buf][((t / WAVE) * RH + r + KH - 1) * COLS + (t % WAVE) + KW - 1];
                        const T* wp = &wts[buf][ob * K];
                        // The first row holding the pair's extremum: each row folds to its extremum
                        // (max3 / min3), and only a strictly better row replaces the provisional one
                        // (a row of NaN never does; one row at a time, which keeps the channel loop's
                        // register budget). Then the first tap of that row equal to the extremum,
                        // whose value carries the sign of a zero.
                        T best = Tr::init();
                        int krow = 0;
#pragma unroll 1
                        for (int kh = 0; kh < KH; ++kh)
                        {
                            T mm = Tr::combine(xp[-kh * COLS], wp[kh * KW]);
#pragma unroll
                            for (int kw = 1; kw < KW; ++kw) mm = Tr::pick(mm, Tr::combine(xp[-kh * COLS - kw], wp[kh * KW + kw]));
                            const bool up = Tr::better(mm, best);
                            best = up ? mm : best;
                            krow = up ? kh : krow;
                        }
                        int kcol = 0;
                        T fval = best;
#pragma unroll
                        for (int kw = KW - 1; kw >= 0; --kw)
                        {
                            const T v = Tr::combine(xp[-krow * COLS - kw], wp[krow * KW + kw]);
                            const bool eq = v == best;
                            kcol = eq ? kw : kcol;
                            fval = eq ? v : fval;
                        }
                        // A pair that never improves on the start value keeps tap 0.
                        const int tap = best == Tr::init() ? 0 : krow * KW + kcol;
                        rbucket[e] = (uint16_t)(tap | (fval == T(0) && signbit(fval) ? 0x8000 : 0));
                    }
                    if (cn < g.Cin) store(buf ^ 1);
                    __syncthreads();
                    buf ^= 1;
                    c = cn;
                }
            }
#pragma unroll
            for (int ob = 0; ob < OB; ++ob)
#pragma unroll
                for (int r = 0; r < RH; ++r)
                {
                    const int o = o0 + ob, h = hw0 + r;
                    if (o >= g.Cout || h >= g.H || wc >= g.W) continue;
                    T v = acc[ob][r];
                    int karg = 0;
                    const int at = (int)((unsigned)win[ob][r] >> 16);
                    if (at != NOPOS)
                    {
                        const int res = rbucket[at];
                        karg = res & 0x7fff;
                        if (v == T(0)) v = (res & 0x8000) ? -T(0) : T(0);
                    }
                    const int64_t oi = ((int64_t)b * g.Cout + o) * plane + (int64_t)h * g.W + wc;
                    p.out[oi] = (ST)v;
                    static_cast<int32_t*>(p.idx)[oi] = (int32_t)(((win[ob][r] & 0xffff) << 16) | karg);
                }
            return;
        }
    }
    if constexpr (!ident)
    {
#pragma unroll
        for (int ob = 0; ob < OB; ++ob)
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                const int o = o0 + ob, h = h0 + wave * RH + r;
                if (o >= g.Cout || h >= g.H || wc >= g.W) continue;
                store_output<ST, OP, MK, MODE>(p, b, o, h, wc, i_end - i_begin, acc[ob][r], win[ob][r]);
            }
    }
}

// ------------------------------------------------------------------------------------------------
// Launch
// ------------------------------------------------------------------------------------------------

// Structuring-element sizes with a compiled static kernel (square sizes of the common layers).
template <typename ST>
static bool has_static(const Geom& g)
{
    using T = compute_t<ST>;
    if (g.KH != g.KW) return false;
    if constexpr (sizeof(T) == 8) return g.KH == 3;
    return g.KH == 3 || g.KH == 5 || g.KH == 7 || g.KH == 11;
}

// Rows per wave of the static kernel: 4 for every size and mode. Fewer registers and more waves beat
// the better LDS reuse of 8 rows (measured on MI355X: 7-27% faster from 3x3 to 11x11, VALUE, PACKED
// and TAPS alike); 2 rows is no faster.
template <typename T, int KH, int MODE>
constexpr int static_rows()
{
    return 4;
}

template <typename ST>
size_t morpho_forward_lds(const Geom& g)
{
    using T = compute_t<ST>;
    if (has_static<ST>(g)) return 0;  // static LDS, sized at compile time (at most ~40 KiB)
    const Tiling t = make_tiling(g, rows_per_wave<T>());
    return (size_t)t.rows * t.pitch * sizeof(T);
}

template <typename ST, int OP, int MK, int OB, int MODE>
static hipError_t launch_generic(FwdParams<ST> p, hipStream_t stream)
{
    using T = compute_t<ST>;
    constexpr int RH = rows_per_wave<T>();
    p.t = make_tiling(p.g, RH);
    const int64_t blocks = (int64_t)p.g.B * p.t.nty * p.t.ntx * p.nog;
    const size_t lds = (size_t)p.t.rows * p.t.pitch * sizeof(T);
    if (pair_tap_bytes(p.g) == 1)
        morpho_fwd_generic<ST, OP, MK, OB, RH, MODE, uint8_t><<<(unsigned)blocks, BLOCK, lds, stream>>>(p);
    else
        morpho_fwd_generic<ST, OP, MK, OB, RH, MODE, uint16_t><<<(unsigned)blocks, BLOCK, lds, stream>>>(p);
    return hipGetLastError();
}

// Below this many workgroups the chip is mostly idle and every workgroup's serial latency (its channel
// loop, the winner rescans of its pixels) is the kernel time: such launches take one row per wave and
// one output channel per workgroup instead, for up to RH * OB times more workgroups.
constexpr int64_t SMALL_GRID = 1024;
constexpr int IDENT_CHANS = 8;

template <typename ST, int OP, int MK, int OB, int MODE, int KS>
static hipError_t launch_static(FwdParams<ST> p, hipStream_t stream)
{
    constexpr int RH = static_rows<compute_t<ST>, KS, MODE>();
    p.t = make_tiling(p.g, RH);
    if constexpr (MK == MK_IDENT)
    {
        // IDENTITY: up to IDENT_CHANS consecutive channels per workgroup, one tile load in flight
        // behind each channel's scan (a single channel per workgroup leaves the loads unhidden).
        p.chans = p.g.Cout < IDENT_CHANS ? p.g.Cout : IDENT_CHANS;
        p.nog = (p.g.Cout + p.chans - 1) / p.chans;
    }
    int64_t blocks = (int64_t)p.g.B * p.t.nty * p.t.ntx * p.nog;
    if constexpr (RH > 1 || OB > 1)
    {
        if (blocks < SMALL_GRID)
        {
            p.t = make_tiling(p.g, 1);
            p.nog = p.g.Cout;
            p.chans = 1;
            blocks = (int64_t)p.g.B * p.t.nty * p.t.ntx * p.nog;
            morpho_fwd_static<ST, OP, MK, KS, KS, 1, 1, MODE><<<(unsigned)blocks, BLOCK, 0, stream>>>(p);
            return hipGetLastError();
        }
    }
    morpho_fwd_static<ST, OP, MK, KS, KS, OB, RH, MODE><<<(unsigned)blocks, BLOCK, 0, stream>>>(p);
    return hipGetLastError();
}

template <typename ST, int OP, int MK, int OB, int MODE>
static hipError_t launch_fwd(const FwdParams<ST>& p, hipStream_t stream)
{
    if (has_static<ST>(p.g))
    {
        if constexpr (sizeof(compute_t<ST>) == 8)
        {
            return launch_static<ST, OP, MK, OB, MODE, 3>(p, stream);
        }
        else
        {
            switch (p.g.KH)
            {
                case 3: return launch_static<ST, OP, MK, OB, MODE, 3>(p, stream);
                case 5: return launch_static<ST, OP, MK, OB, MODE, 5>(p, stream);
                case 7: return launch_static<ST, OP, MK, OB, MODE, 7>(p, stream);
                default: return launch_static<ST, OP, MK, OB, MODE, 11>(p, stream);
            }
        }
    }
    return launch_generic<ST, OP, MK, OB, MODE>(p, stream);
}

template <typename ST, int OP>
static hipError_t forward_op(int merge, FwdParams<ST> p, hipStream_t stream)
{
    const bool save = p.idx != nullptr;
    // Output channels sharing each staged input tile: 4 for the value modes; 2 when every pair's tap
    // is tracked, whose window and accumulators need more registers.
    const bool group4 = p.g.Cout >= 4 && merge != MERGE_IDENTITY;
    const bool group2 = p.g.Cout >= 2 && merge != MERGE_IDENTITY;
    p.nog = merge == MERGE_IDENTITY ? p.g.Cout : (group4 ? (p.g.Cout + 3) / 4 : p.g.Cout);
    switch (merge)
    {
        case MERGE_ADD:
        case MERGE_AVERAGE:
            p.average = merge == MERGE_AVERAGE;
            if (save)
            {
                p.nog = group2 ? (p.g.Cout + 1) / 2 : p.g.Cout;
                return group2 ? launch_fwd<ST, OP, MK_SUM, 2, FWD_TAPS>(p, stream) : launch_fwd<ST, OP, MK_SUM, 1, FWD_TAPS>(p, stream);
            }
            return group4 ? launch_fwd<ST, OP, MK_SUM, 4, FWD_VALUE>(p, stream) : launch_fwd<ST, OP, MK_SUM, 1, FWD_VALUE>(p, stream);
        case MERGE_MAX:
            if (save) return group4 ? launch_fwd<ST, OP, MK_MAX, 4, FWD_PACKED>(p, stream) : launch_fwd<ST, OP, MK_MAX, 1, FWD_PACKED>(p, stream);
            return group4 ? launch_fwd<ST, OP, MK_MAX, 4, FWD_VALUE>(p, stream) : launch_fwd<ST, OP, MK_MAX, 1, FWD_VALUE>(p, stream);
        case MERGE_MIN:
            if (save) return group4 ? launch_fwd<ST, OP, MK_MIN, 4, FWD_PACKED>(p, stream) : launch_fwd<ST, OP, MK_MIN, 1, FWD_PACKED>(p, stream);
            return group4 ? launch_fwd<ST, OP, MK_MIN, 4, FWD_VALUE>(p, stream) : launch_fwd<ST, OP, MK_MIN, 1, FWD_VALUE>(p, stream);
        case MERGE_IDENTITY:
            // 3x3 / 5x5 planes whose width is a multiple of 8: the streaming row-band kernels (float32 /
            // float64; the 16-bit tiles keep their border value in float32).
            if constexpr (std::is_same_v<ST, float> || std::is_same_v<ST, double>)
            {
                const bool aligned = ((uintptr_t)p.x | (uintptr_t)p.out) % 16 == 0 && (uintptr_t)p.idx % 8 == 0;
                if (aligned && ident_bands(p.g, sizeof(ST), false).R > 0)
                    return ident_band_forward<ST>(OP, p.replicate != 0, p.fill, p.x, p.w, p.out, static_cast<uint8_t*>(p.idx), p.g, stream);
            }
            if (save) return launch_fwd<ST, OP, MK_IDENT, 1, FWD_TAPS>(p, stream);
            return launch_fwd<ST, OP, MK_IDENT, 1, FWD_VALUE>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

template <typename ST>
hipError_t morpho_forward(int op, int merge, bool replicate, compute_t<ST> fill, const ST* x, const ST* w, ST* out, void* indices,
                          const Geom& g, hipStream_t stream)
{
    if ((int64_t)g.B * g.Cout * g.plane() == 0) return hipSuccess;
    if (g.Cin == 0 && merge != MERGE_IDENTITY)
    {
        const int64_t n = (int64_t)g.B * g.Cout * g.plane();
        hipError_t err = fill_async<ST>(out, n, empty_merge_value<ST>(merge), stream);
        if (err == hipSuccess && indices && packed_winners(merge)) err = fill_async<int32_t>(static_cast<int32_t*>(indices), n, 0, stream);
        return err;
    }
    FwdParams<ST> p{};
    p.x = x;
    p.w = w;
    p.out = out;
    p.idx = indices;
    p.g = g;
    p.replicate = replicate ? 1 : 0;
    p.fill = fill;
    p.average = 0;
    return op == DILATION ? forward_op<ST, DILATION>(merge, p, stream) : forward_op<ST, EROSION>(merge, p, stream);
}

#define MCA_INSTANTIATE_FWD(ST)                                                                                                        \
    template hipError_t morpho_forward<ST>(int, int, bool, compute_t<ST>, const ST*, const ST*, ST*, void*, const Geom&, hipStream_t); \
    template size_t morpho_forward_lds<ST>(const Geom&);

}  // namespace mca
