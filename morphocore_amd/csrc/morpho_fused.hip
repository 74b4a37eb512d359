// Fused compositions: opening / closing and sigma_layer with per-channel ('identity') merges, each in
// one pass per tile.
//
// Opening is an erosion followed by a dilation of its output, closing the reverse (reference:
// functional/opening.py:96-101, functional/closing.py:96-101; nn/opening.py:104-180 shares one
// structuring element between the stages, which forces the 'identity' merge on both). With both
// merges 'identity', output channel c depends on input channel c only, so one workgroup can take a
// tile of one channel from x to the final output: it stages x with the halo of both stages in LDS,
// computes the first stage's values over the tile plus the second stage's halo into LDS (the
// intermediate image never reaches HBM), pads them as the second stage reads its input, and runs the
// second stage from LDS. HBM traffic per output pixel: x once, the output once, one tap byte per
// stage, against twice x-sized reads and writes for the two separate launches.
//
// Every pixel of each stage is computed exactly as the separate IDENTITY kernels compute it: the
// strict first-tap scan in the reference's tap order (morpho_op_cpu_kernels.hxx:254-263), the first
// extremal tap saved. The backward routes from those taps, one stage after the other (below).
//
// Tiles are (64 - (K - 1)) output columns by 16 rows, so that the intermediate region a tile needs is
// exactly 64 columns wide: one lane per intermediate column and per output column. A workgroup walks up
// to 8 channels of its tile with the next channel's loads in flight; each lane reads its column's
// window rows once from LDS into registers.
#include <algorithm>

#include "launch.hpp"

namespace mca
{

template <typename T>
struct PairFwdParams
{
    const T* __restrict__ x;
    const T* __restrict__ w1;  // first stage [C, 1, K, K] (or per sample, wbs apart), as the operator receives it
    const T* __restrict__ w2;  // second stage
    int64_t wbs;
    T* __restrict__ out;
    uint8_t* __restrict__ taps1;  // [B, C, H, W] or null
    uint8_t* __restrict__ taps2;
    int B, C, H, W;
    int ntx, nty;
    int chans, ncg;  // consecutive channels per workgroup, channel groups
    int replicate;
    T fill1, fill2;  // the border value each stage reads (REPLICATE: unused)
};

// Output rows per wave.
constexpr int PAIR_RH = 4;

template <int K>
struct PairTile
{
    static constexpr int P = K / 2;
    static constexpr int RH = PAIR_RH;
    static constexpr int TH = NWAVES * RH;        // output rows per tile
    static constexpr int OW = TILE_W - (K - 1);   // output columns per tile
    static constexpr int ER = TH + K - 1;         // intermediate rows a tile needs
    static constexpr int RE = (ER + NWAVES - 1) / NWAVES;  // intermediate rows per wave
    static constexpr int XR = ER + K - 1;         // forward: staged input rows
    static constexpr int XC = TILE_W + K - 1;     // forward: staged input columns (backward: output-gradient columns)
    static constexpr int XN = XR * XC;            // staged elements of the larger region
    static constexpr int NX = (XN + BLOCK - 1) / BLOCK;            // per thread
    static constexpr int EN = ER * TILE_W;        // intermediate region
    static constexpr int NE = (EN + BLOCK - 1) / BLOCK;
};

// Value of `v` on lane `src` of the wave (ds_bpermute; double as two halves).
__device__ __forceinline__ float shfl_t(float v, int src) { return __shfl(v, src, WAVE); }
__device__ __forceinline__ double shfl_t(double v, int src) { return __shfl(v, src, WAVE); }

struct PairWork
{
    int b, cg, tx, ty, tile;
};

// Consecutive work items are neighbouring tiles of one channel group (they share halo rows in L2).
__device__ __forceinline__ PairWork decode_pair(int ncg, int ntx, int nty)
{
    int work = xcd_work_index(blockIdx.x, gridDim.x);
    PairWork w;
    w.tx = work % ntx;
    work /= ntx;
    w.ty = work % nty;
    work /= nty;
    w.tile = w.ty * ntx + w.tx;
    w.cg = work % ncg;
    w.b = work / ncg;
    return w;
}

// Strict first-tap scan (reference tap order kh, then kw) of the pixel whose tap (kh, kw) reads
// win[r + K - 1 - kh][K - 1 - kw]: the extremum and its first tap; a pixel that never improves on
// the start value keeps it with tap 0. The running extremum is kept with the NaN-ignoring max / min,
// which equals the strict scan's up to the sign of a zero, so the strict comparison against it picks
// the same first tap; a zero result takes the value of that tap, whose sign is the strict scan's.
template <int OP, typename T, int K, int WR>
__device__ __forceinline__ void pair_scan(const T (&win)[WR][K], int r, const T* wk, T& best, int& arg)
{
    using Tr = OpTraits<OP, T>;
    T m = Tr::init();
    arg = 0;
#pragma unroll
    for (int kh = 0; kh < K; ++kh)
#pragma unroll
        for (int kw = 0; kw < K; ++kw)
        {
            const T v = Tr::combine(win[r + K - 1 - kh][K - 1 - kw], wk[kh * K + kw]);
            arg = Tr::better(v, m) ? kh * K + kw : arg;
            m = Tr::pick(m, v);
        }
    best = m;
    if (m == T(0))
    {
#pragma unroll
        for (int kh = 0; kh < K; ++kh)
#pragma unroll
            for (int kw = 0; kw < K; ++kw)
                if (arg == kh * K + kw) best = Tr::combine(win[r + K - 1 - kh][K - 1 - kw], wk[kh * K + kw]);
    }
}

// Each workgroup walks `chans` consecutive channels of one tile; the next channel's input tile and
// elements are loaded into registers while the current one computes, and staged behind it.
template <typename T, int OP1, int K>
__global__ __launch_bounds__(BLOCK) void morpho_pair_fwd_kernel(const PairFwdParams<T> p)
{
    constexpr int OP2 = OP1 == DILATION ? EROSION : DILATION;
    using S = PairTile<K>;
    constexpr int P = S::P, TH = S::TH, RH = S::RH, OW = S::OW, ER = S::ER, RE = S::RE, XR = S::XR, XC = S::XC, KK = K * K;
    constexpr int XN = S::XN, NX = S::NX;
    __shared__ T xs[2][XN];
    __shared__ T es[S::EN];
    __shared__ T ws[2][2 * KK];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const PairWork wk = decode_pair(p.ncg, p.ntx, p.nty);
    const int H = p.H, W = p.W;
    const int64_t plane = (int64_t)H * W;
    const int h0 = wk.ty * TH, c0 = wk.tx * OW;
    // Origins of the intermediate region (second stage's input window) and of the staged input.
    const int ey0 = h0 + P - (K - 1), ex0 = c0 + P - (K - 1);
    const int xy0 = ey0 + P - (K - 1), xx0 = ex0 + P - (K - 1);
    const int c_begin = wk.cg * p.chans, c_end = min(c_begin + p.chans, p.C);

    // Staging plan, the same for every channel: the clamped in-image offset of each element this
    // thread stages (loaded unconditionally) and whether the fill value replaces it.
    int off[NX];
    bool fill[NX];
#pragma unroll
    for (int j = 0; j < NX; ++j)
    {
        const int idx = min((int)threadIdx.x + j * BLOCK, XN - 1);
        const int ly = idx / XC, lx = idx - ly * XC;
        const int y = xy0 + ly, xx = xx0 + lx;
        off[j] = clampi(y, 0, H - 1) * W + clampi(xx, 0, W - 1);
        fill[j] = !p.replicate && !(y >= 0 && y < H && xx >= 0 && xx < W);
    }
    T pre[NX], wpre = T(0);
    auto load = [&](int c) {
        const T* __restrict__ xp = p.x + ((int64_t)wk.b * p.C + c) * plane;
#pragma unroll
        for (int j = 0; j < NX; ++j) pre[j] = xp[off[j]];
        if (threadIdx.x < 2 * KK)
        {
            const int k = threadIdx.x < KK ? threadIdx.x : threadIdx.x - KK;
            wpre = (threadIdx.x < KK ? p.w1 : p.w2)[(int64_t)wk.b * p.wbs + (int64_t)c * KK + k];
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int j = 0; j < NX; ++j)
        {
            const int idx = threadIdx.x + j * BLOCK;
            if (j < NX - 1 || idx < XN) xs[buf][idx] = fill[j] ? p.fill1 : pre[j];
        }
        if (threadIdx.x < 2 * KK) ws[buf][threadIdx.x] = wpre;
    };

    const int gx1 = ex0 + lane;
    const bool own_col1 = lane >= K - 1 - P && lane < K - 1 - P + OW;
    const int src_lane = clampi(gx1, 0, W - 1) - ex0;  // in [0, 64) whenever the region crosses an edge
    const bool rows_out = ey0 < 0 || ey0 + ER > H;     // the same for the whole workgroup
    const int wc = c0 + lane;
    const int lcol = lane < OW ? lane : OW - 1;  // lanes past the tile read in bounds; their results are dropped
    load(c_begin);
    store(0);
    __syncthreads();
    for (int c = c_begin; c < c_end; ++c)
    {
        const int buf = (c - c_begin) & 1;
        const bool more = c + 1 < c_end;
        if (more) load(c + 1);  // in flight while this channel computes
        const int64_t pbase = ((int64_t)wk.b * p.C + c) * plane;

        // First stage over the intermediate region: lane = column, RE consecutive rows per wave (the
        // last wave's surplus rows recompute its last row; only real rows are stored). Its taps are
        // saved for the tile's own pixels only (every pixel belongs to exactly one tile).
        {
            T wr[KK];
#pragma unroll
            for (int k = 0; k < KK; ++k) wr[k] = ws[buf][k];
            const int r0 = wave * RE;
            T win[RE + K - 1][K];
#pragma unroll
            for (int rr = 0; rr < RE + K - 1; ++rr)
#pragma unroll
                for (int kw = 0; kw < K; ++kw) win[rr][kw] = xs[buf][min(r0 + rr, XR - 1) * XC + lane + kw];
#pragma unroll
            for (int j = 0; j < RE; ++j)
            {
                const int ly = r0 + j;
                T best;
                int arg;
                pair_scan<OP1, T, K>(win, j, wr, best, arg);
                const int gy = ey0 + ly;
                const bool in = gy >= 0 && gy < H && gx1 >= 0 && gx1 < W;
                // REPLICATE: a column outside the image takes the clamped column's value (another lane
                // of the same row); rows outside the image are copied after the pass.
                const T moved = shfl_t(best, src_lane);
                if (ly < ER) es[ly * TILE_W + lane] = p.replicate ? moved : (in ? best : p.fill2);
                if (p.taps1 && in && own_col1 && ly >= K - 1 - P && ly < K - 1 - P + TH)
                    p.taps1[pbase + (int64_t)gy * W + gx1] = (uint8_t)arg;
            }
        }
        __syncthreads();
        if (p.replicate && rows_out)
        {
            // Rows of the intermediate region outside the image read the clamped edge row, which lies
            // in the region whenever the region crosses that edge (its columns already resolved).
            for (int ly = wave; ly < ER; ly += NWAVES)
            {
                const int gy = ey0 + ly;
                if (gy < 0 || gy >= H) es[ly * TILE_W + lane] = es[(clampi(gy, 0, H - 1) - ey0) * TILE_W + lane];
            }
            __syncthreads();
        }

        // Second stage: lane = output column (the first OW lanes), RH rows per wave.
        {
            T wr[KK];
#pragma unroll
            for (int k = 0; k < KK; ++k) wr[k] = ws[buf][KK + k];
            T win[RH + K - 1][K];
#pragma unroll
            for (int rr = 0; rr < RH + K - 1; ++rr)
#pragma unroll
                for (int kw = 0; kw < K; ++kw) win[rr][kw] = es[(wave * RH + rr) * TILE_W + lcol + kw];
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                const int h = h0 + wave * RH + r;
                T best;
                int arg;
                pair_scan<OP2, T, K>(win, r, wr, best, arg);
                if (lane < OW && h < H && wc < W)
                {
                    const int64_t oi = pbase + (int64_t)h * W + wc;
                    p.out[oi] = best;
                    if (p.taps2) p.taps2[oi] = (uint8_t)arg;
                }
            }
        }
        if (more) store(buf ^ 1);
        // The next channel's first stage rewrites es, and reads the staged buffer.
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------------
// sigma_layer with the 'identity' merge: the erosion and the dilation of one input in one pass.
// ------------------------------------------------------------------------------------------------
//
// The reference's sigma_layer (functional/sigma_layer.py:73-83) blends an erosion and a dilation of one
// input by the same structuring element, soft = sigmoid(mean(alpha)) per output channel:
// out = erosion * (1 - soft) + dilation * soft. With the 'identity' merge both are per channel, so one
// workgroup computes both from one staged tile (each lane's window registers feed the two scans),
// forms the blend in registers with the roundings of torch's three elementwise operations, in their
// order, and writes only the output and one tap byte per operation. The backward routes g (1 - soft)
// through the erosion's taps and g soft through the dilation's into grad_input, gathered per pixel in
// tap order as the separate gather kernels do, and sums g * erosion and g * dilation per channel (the
// gradient of soft) from the two values re-read at their taps. Output tiles are 64 x 16; both
// operations read one border value (geodesic padding: NaN, which never wins either operation, as the
// +inf / -inf of their own fills never does).

template <typename T>
struct SigmaParams
{
    const T* __restrict__ x;
    const T* __restrict__ we;  // erosion element as the erosion operator receives it (flipped)
    const T* __restrict__ wd;  // dilation element
    int64_t wbs;
    const T* __restrict__ soft;  // [C]
    T* __restrict__ out;
    uint8_t* __restrict__ tapse;  // [B, C, H, W]; forward: or null
    uint8_t* __restrict__ tapsd;
    const T* __restrict__ gout;  // backward
    T* __restrict__ gin;
    T* __restrict__ part_we;  // [B * tiles][C][K * K]
    T* __restrict__ part_wd;
    T* __restrict__ part_s;  // [B * tiles][2][C]: sum of g * erosion, sum of g * dilation
    int B, C, H, W;
    int ntx, nty, chans, ncg;
    int replicate;
    T fill;
};

template <int K>
struct SigmaTile
{
    static constexpr int P = K / 2;
    static constexpr int RH = PAIR_RH;
    static constexpr int TH = NWAVES * RH;
    static constexpr int XR = TH + K - 1, XC = TILE_W + K - 1, XN = XR * XC;
    static constexpr int NX = (XN + BLOCK - 1) / BLOCK;
};

// out = e (1 - soft) + d soft as torch evaluates it: 1 - soft, each product and the sum rounded.
template <typename T>
__device__ __forceinline__ T sigma_blend(T e, T d, T oms, T s)
{
#pragma clang fp contract(off)
    const T a = e * oms;
    const T b = d * s;
    return a + b;
}

template <typename T, int K>
__global__ __launch_bounds__(BLOCK) void morpho_sigma_fwd_kernel(const SigmaParams<T> p)
{
    using S = SigmaTile<K>;
    constexpr int P = S::P, RH = S::RH, TH = S::TH, XC = S::XC, XN = S::XN, NX = S::NX, KK = K * K;
    __shared__ T xs[2][XN];
    __shared__ T ws[2][2 * KK + 1];  // erosion element, dilation element, soft
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const PairWork wk = decode_pair(p.ncg, p.ntx, p.nty);
    const int H = p.H, W = p.W;
    const int64_t plane = (int64_t)H * W;
    const int h0 = wk.ty * TH, c0 = wk.tx * TILE_W;
    const int y0 = h0 - P, x0 = c0 - P;
    const int c_begin = wk.cg * p.chans, c_end = min(c_begin + p.chans, p.C);

    int off[NX];
    bool fill[NX];
#pragma unroll
    for (int j = 0; j < NX; ++j)
    {
        const int idx = min((int)threadIdx.x + j * BLOCK, XN - 1);
        const int ly = idx / XC, lx = idx - ly * XC;
        const int y = y0 + ly, xx = x0 + lx;
        off[j] = clampi(y, 0, H - 1) * W + clampi(xx, 0, W - 1);
        fill[j] = !p.replicate && !(y >= 0 && y < H && xx >= 0 && xx < W);
    }
    T pre[NX], wpre = T(0);
    auto load = [&](int c) {
        const T* __restrict__ xp = p.x + ((int64_t)wk.b * p.C + c) * plane;
#pragma unroll
        for (int j = 0; j < NX; ++j) pre[j] = xp[off[j]];
        const int t = threadIdx.x;
        if (t < 2 * KK)
            wpre = (t < KK ? p.we : p.wd)[(int64_t)wk.b * p.wbs + (int64_t)c * KK + (t < KK ? t : t - KK)];
        else if (t == 2 * KK)
            wpre = p.soft[c];
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int j = 0; j < NX; ++j)
        {
            const int idx = threadIdx.x + j * BLOCK;
            if (j < NX - 1 || idx < XN) xs[buf][idx] = fill[j] ? p.fill : pre[j];
        }
        if (threadIdx.x <= 2 * KK) ws[buf][threadIdx.x] = wpre;
    };

    const int wc = c0 + lane;
    load(c_begin);
    store(0);
    __syncthreads();
    for (int c = c_begin; c < c_end; ++c)
    {
        const int buf = (c - c_begin) & 1;
        const bool more = c + 1 < c_end;
        if (more) load(c + 1);  // in flight while this channel computes
        const int64_t pbase = ((int64_t)wk.b * p.C + c) * plane;
        T wer[KK], wdr[KK];
#pragma unroll
        for (int k = 0; k < KK; ++k)
        {
            wer[k] = ws[buf][k];
            wdr[k] = ws[buf][KK + k];
        }
        const T s = ws[buf][2 * KK];
        const T oms = T(1) - s;
        T win[RH + K - 1][K];
#pragma unroll
        for (int rr = 0; rr < RH + K - 1; ++rr)
#pragma unroll
            for (int kw = 0; kw < K; ++kw) win[rr][kw] = xs[buf][(wave * RH + rr) * XC + lane + kw];
#pragma unroll
        for (int r = 0; r < RH; ++r)
        {
            const int h = h0 + wave * RH + r;
            T e, d;
            int te, td;
            pair_scan<EROSION, T, K>(win, r, wer, e, te);
            pair_scan<DILATION, T, K>(win, r, wdr, d, td);
            if (h < H && wc < W)
            {
                const int64_t oi = pbase + (int64_t)h * W + wc;
                p.out[oi] = sigma_blend(e, d, oms, s);
                if (p.tapse)
                {
                    p.tapse[oi] = (uint8_t)te;
                    p.tapsd[oi] = (uint8_t)td;
                }
            }
        }
        if (more) store(buf ^ 1);
        __syncthreads();
    }
}

// Value the forward's scan of operation OP produced at a pixel, from its saved tap: the tap's
// combination, or the start value when no tap improved on it (then the saved tap is 0).
template <int OP, typename T>
__device__ __forceinline__ T sigma_tap_value(T xv, T wv)
{
    using Tr = OpTraits<OP, T>;
    const T v = Tr::combine(xv, wv);
    return Tr::better(v, Tr::init()) ? v : Tr::init();
}

template <typename T, int K>
__global__ __launch_bounds__(BLOCK) void morpho_sigma_bwd_kernel(const SigmaParams<T> p)
{
    using S = SigmaTile<K>;
    constexpr int P = S::P, RH = S::RH, TH = S::TH, XC = S::XC, XN = S::XN, NX = S::NX, KK = K * K;
    constexpr int NC = 32;  // lane-striped copies of each weight-gradient bin
    __shared__ T xs[XN];
    __shared__ T gs[XN];
    __shared__ int8_t tes[XN];
    __shared__ int8_t tds[XN];
    __shared__ T ws[2 * KK + 1];
    __shared__ __align__(16) Acc bins[2 * KK * NC];
    __shared__ Acc red[2 * NWAVES];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const PairWork wk = decode_pair(p.ncg, p.ntx, p.nty);
    const int H = p.H, W = p.W;
    const int64_t plane = (int64_t)H * W;
    const int h0 = wk.ty * TH, c0 = wk.tx * TILE_W;
    // One region serves both: the input window of the tile's own pixels (recomputing their values)
    // and the pixels whose taps may read the tile's inputs (the gather).
    const int y0 = h0 - P, x0 = c0 - P;
    const int c_begin = wk.cg * p.chans, c_end = min(c_begin + p.chans, p.C);

    int off[NX];
    bool in[NX];
#pragma unroll
    for (int j = 0; j < NX; ++j)
    {
        const int idx = min((int)threadIdx.x + j * BLOCK, XN - 1);
        const int ly = idx / XC, lx = idx - ly * XC;
        const int y = y0 + ly, xx = x0 + lx;
        off[j] = clampi(y, 0, H - 1) * W + clampi(xx, 0, W - 1);
        in[j] = y >= 0 && y < H && xx >= 0 && xx < W;
    }
    T px[NX], pg[NX], wpre = T(0);
    int pte[NX], ptd[NX];
    auto load = [&](int c) {
        const int64_t pb = ((int64_t)wk.b * p.C + c) * plane;
#pragma unroll
        for (int j = 0; j < NX; ++j)
        {
            px[j] = p.x[pb + off[j]];
            pg[j] = p.gout[pb + off[j]];
            pte[j] = p.tapse[pb + off[j]];
            ptd[j] = p.tapsd[pb + off[j]];
        }
        const int t = threadIdx.x;
        if (t < 2 * KK)
            wpre = (t < KK ? p.we : p.wd)[(int64_t)wk.b * p.wbs + (int64_t)c * KK + (t < KK ? t : t - KK)];
        else if (t == 2 * KK)
            wpre = p.soft[c];
    };
    auto store = [&]() {
#pragma unroll
        for (int j = 0; j < NX; ++j)
        {
            const int idx = threadIdx.x + j * BLOCK;
            if (j < NX - 1 || idx < XN)
            {
                xs[idx] = in[j] || p.replicate ? px[j] : p.fill;
                gs[idx] = in[j] ? pg[j] : T(0);
                tes[idx] = in[j] ? (int8_t)pte[j] : (int8_t)-1;
                tds[idx] = in[j] ? (int8_t)ptd[j] : (int8_t)-1;
            }
        }
        if (threadIdx.x <= 2 * KK) ws[threadIdx.x] = wpre;
    };

    for (int j = threadIdx.x; j < 2 * KK * NC; j += BLOCK) bins[j] = Acc(0);
    Acc* ble = bins + (lane & (NC - 1));
    Acc* bld = bins + KK * NC + (lane & (NC - 1));
    const int wc = c0 + lane;
    const int64_t slot = (int64_t)wk.b * p.ntx * p.nty + wk.tile;
    load(c_begin);
    store();
    __syncthreads();
    for (int c = c_begin; c < c_end; ++c)
    {
        const bool more = c + 1 < c_end;
        if (more) load(c + 1);  // in flight while this channel computes
        const T s = ws[2 * KK];
        const T oms = T(1) - s;

        // The tile's own pixels: both values re-read at their taps, the sums of g * value, and the
        // elements' gradients (-g (1 - soft) for the erosion, g soft for the dilation).
        Acc se = Acc(0), sd = Acc(0);
#pragma unroll
        for (int r = 0; r < RH; ++r)
        {
            const int lr = wave * RH + r;
            const int oi = (lr + P) * XC + lane + P;
            const int te = tes[oi], td = tds[oi];
            if (te >= 0)
            {
                const T g = gs[oi];
                const int ke = te / K, kd = td / K;
                const T e = sigma_tap_value<EROSION, T>(xs[(lr + K - 1 - ke) * XC + lane + K - 1 - (te - ke * K)], ws[te]);
                const T d = sigma_tap_value<DILATION, T>(xs[(lr + K - 1 - kd) * XC + lane + K - 1 - (td - kd * K)], ws[KK + td]);
                se += (Acc)(g * e);
                sd += (Acc)(g * d);
                lds_add(&ble[te * NC], -(Acc)(g * oms));
                lds_add(&bld[td * NC], (Acc)(g * s));
            }
        }
        // grad_input: pixel q collects g (1 - soft) of the pixels e = q + (kh - P, kw - P) whose erosion
        // tap k read it and g soft of those whose dilation tap did, each summed in tap order and
        // rounded, then added (the two branches of the composition's autograd).
        {
            T gw[RH + K - 1][K];
            int tw[RH + K - 1][K], dw[RH + K - 1][K];
#pragma unroll
            for (int rr = 0; rr < RH + K - 1; ++rr)
#pragma unroll
                for (int kw = 0; kw < K; ++kw)
                {
                    const int i = (wave * RH + rr) * XC + lane + kw;
                    gw[rr][kw] = gs[i];
                    tw[rr][kw] = tes[i];
                    dw[rr][kw] = tds[i];
                }
            T* __restrict__ gin = p.gin + ((int64_t)wk.b * p.C + c) * plane;
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                Acc ae = Acc(0), ad = Acc(0);
#pragma unroll
                for (int kh = 0; kh < K; ++kh)
#pragma unroll
                    for (int kw = 0; kw < K; ++kw)
                    {
                        const T g = gw[r + kh][kw];
                        ae += tw[r + kh][kw] == kh * K + kw ? (Acc)(g * oms) : Acc(0);
                        ad += dw[r + kh][kw] == kh * K + kw ? (Acc)(g * s) : Acc(0);
                    }
                const int h = h0 + wave * RH + r;
                if (h < H && wc < W) gin[(int64_t)h * W + wc] = (T)ae + (T)ad;
            }
        }
        // Per-channel sums over the workgroup in a fixed order: the wave's lanes, then the waves.
#pragma unroll
        for (int d = WAVE / 2; d >= 1; d /= 2)
        {
            se += __shfl_xor(se, d, WAVE);
            sd += __shfl_xor(sd, d, WAVE);
        }
        if (lane == 0)
        {
            red[2 * wave] = se;
            red[2 * wave + 1] = sd;
        }
        __syncthreads();
        if (threadIdx.x < 2)
        {
            Acc v = Acc(0);
#pragma unroll
            for (int w = 0; w < NWAVES; ++w) v += red[2 * w + threadIdx.x];
            p.part_s[(slot * 2 + threadIdx.x) * p.C + c] = (T)v;
        }
        for (int j = threadIdx.x; j < 2 * KK; j += BLOCK)
        {
            Acc* q = bins + (int64_t)j * NC;
            Acc v = Acc(0);
#pragma unroll
            for (int n = 0; n < NC; ++n)
            {
                v += q[n];
                q[n] = Acc(0);
            }
            const int st = j / KK, k = j - st * KK;
            (st == 0 ? p.part_we : p.part_wd)[(slot * p.C + c) * KK + k] = (T)v;
        }
        // Staging the next channel overwrites every buffer this one read; its adds need the cleared
        // bins.
        __syncthreads();
        if (more)
        {
            store();
            __syncthreads();
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Launch
// ------------------------------------------------------------------------------------------------

bool morpho_pair_supported(const Geom& g) { return g.KH == g.KW && (g.KH == 3 || g.KH == 5 || g.KH == 7); }

static void pair_tiles(const Geom& g, int& ntx, int& nty)
{
    const int ow = TILE_W - (g.KW - 1), th = NWAVES * PAIR_RH;
    ntx = (g.W + ow - 1) / ow;
    nty = (g.H + th - 1) / th;
}

// Up to 8 consecutive channels per workgroup (one tile load in flight behind each channel's work),
// fewer when that would leave fewer than 2048 workgroups.
static void pair_channels(const Geom& g, int tiles, int& chans, int& ncg)
{
    chans = 8;
    while (chans > 1 && (int64_t)g.B * tiles * ((g.Cout + chans - 1) / chans) < 2048) chans /= 2;
    ncg = (g.Cout + chans - 1) / chans;
}

// The backward runs the two stages' IDENTITY backwards from the saved taps, second stage first (the
// gather kernels of morpho_bwd.hip for 3x3 and 5x5: each pixel of the intermediate gradient and of
// grad_input written once, in tap order): a fused backward, which must recompute the intermediate
// gradient over every tile's halo with a compare per tap and pixel, measured slower than the two
// gathers it replaces. Workspace: the intermediate gradient, then the larger of the two stages'.
static Geom pair_stage_geom(const Geom& g)
{
    Geom s = g;
    s.Cin = s.Cout;
    s.Cw = 1;
    s.wbs = 0;
    return s;
}

template <typename T>
size_t morpho_pair_backward_workspace(const Geom& g)
{
    const Geom s = pair_stage_geom(g);
    return align_up((size_t)s.B * s.Cout * s.plane() * sizeof(T)) + morpho_backward_workspace<T>(MERGE_IDENTITY, true, s);
}

template <typename T, int OP1>
static hipError_t pair_fwd_launch(const PairFwdParams<T>& p, int K, int64_t blocks, hipStream_t stream)
{
    switch (K)
    {
        case 3: morpho_pair_fwd_kernel<T, OP1, 3><<<(unsigned)blocks, BLOCK, 0, stream>>>(p); break;
        case 5: morpho_pair_fwd_kernel<T, OP1, 5><<<(unsigned)blocks, BLOCK, 0, stream>>>(p); break;
        default: morpho_pair_fwd_kernel<T, OP1, 7><<<(unsigned)blocks, BLOCK, 0, stream>>>(p); break;
    }
    return hipGetLastError();
}

template <typename T>
hipError_t morpho_pair_forward(int first_op, bool replicate, T fill1, T fill2, const T* x, const T* w1, const T* w2, T* out, uint8_t* taps1,
                               uint8_t* taps2, const Geom& g, hipStream_t stream)
{
    if (!morpho_pair_supported(g)) return hipErrorInvalidValue;
    if ((int64_t)g.B * g.Cout * g.plane() == 0) return hipSuccess;
    PairFwdParams<T> p{};
    p.x = x;
    p.w1 = w1;
    p.w2 = w2;
    p.wbs = g.wbs;
    p.out = out;
    p.taps1 = taps1;
    p.taps2 = taps2;
    p.B = g.B;
    p.C = g.Cout;
    p.H = g.H;
    p.W = g.W;
    pair_tiles(g, p.ntx, p.nty);
    pair_channels(g, p.ntx * p.nty, p.chans, p.ncg);
    p.replicate = replicate ? 1 : 0;
    p.fill1 = fill1;
    p.fill2 = fill2;
    const int64_t blocks = (int64_t)g.B * p.ncg * p.ntx * p.nty;
    return first_op == EROSION ? pair_fwd_launch<T, EROSION>(p, g.KH, blocks, stream) : pair_fwd_launch<T, DILATION>(p, g.KH, blocks, stream);
}

template <typename T>
hipError_t morpho_pair_backward(int first_op, const uint8_t* taps1, const uint8_t* taps2, const T* grad_out, T* grad_in, T* grad_w1,
                                T* grad_w2, const Geom& g, void* workspace, size_t workspace_bytes, hipStream_t stream)
{
    if (!morpho_pair_supported(g)) return hipErrorInvalidValue;
    if (workspace_bytes < morpho_pair_backward_workspace<T>(g)) return hipErrorInvalidValue;
    if ((int64_t)g.B * g.Cout * g.plane() == 0)
    {
        // No output (and no input) pixel: both elements' gradients are zero.
        const int64_t nw = (int64_t)g.Cout * g.taps();
        const hipError_t e = fill_async<T>(grad_w1, nw, T(0), stream);
        return e != hipSuccess ? e : fill_async<T>(grad_w2, nw, T(0), stream);
    }
    const Geom s = pair_stage_geom(g);
    const int second_op = first_op == DILATION ? EROSION : DILATION;
    unsigned char* ws = static_cast<unsigned char*>(workspace);
    T* grad_mid = reinterpret_cast<T*>(ws);
    const size_t mid = align_up((size_t)s.B * s.Cout * s.plane() * sizeof(T));
    const size_t rest = workspace_bytes - mid;
    // With saved taps the stages read neither their input nor their element: only the routing.
    hipError_t e = morpho_backward<T>(second_op, MERGE_IDENTITY, false, T(0), nullptr, nullptr, taps2, grad_out, grad_mid, grad_w2, s,
                                      ws + mid, rest, stream);
    if (e != hipSuccess) return e;
    return morpho_backward<T>(first_op, MERGE_IDENTITY, false, T(0), nullptr, nullptr, taps1, grad_mid, grad_in, grad_w1, s, ws + mid, rest,
                              stream);
}

template <typename T, int K>
static void sigma_setup(SigmaParams<T>& p, const Geom& g, int64_t& blocks)
{
    p.B = g.B;
    p.C = g.Cout;
    p.H = g.H;
    p.W = g.W;
    p.wbs = g.wbs;
    p.ntx = (g.W + TILE_W - 1) / TILE_W;
    p.nty = (g.H + SigmaTile<K>::TH - 1) / SigmaTile<K>::TH;
    pair_channels(g, p.ntx * p.nty, p.chans, p.ncg);
    blocks = (int64_t)g.B * p.ncg * p.ntx * p.nty;
}

static int64_t sigma_slots(const Geom& g)
{
    const int th = NWAVES * PAIR_RH;
    return (int64_t)g.B * ((g.W + TILE_W - 1) / TILE_W) * ((g.H + th - 1) / th);
}

template <typename T>
size_t morpho_sigma_backward_workspace(const Geom& g)
{
    const int64_t nslots = sigma_slots(g);
    const int64_t nw = (int64_t)g.Cout * g.taps(), ns = 2 * (int64_t)g.Cout;
    const size_t scratch = std::max(reduce_slots_scratch<T>((int)nslots, nw), reduce_slots_scratch<T>((int)nslots, ns));
    return 2 * align_up((size_t)nslots * nw * sizeof(T)) + align_up((size_t)nslots * ns * sizeof(T)) + align_up(scratch);
}

template <typename T>
hipError_t morpho_sigma_forward(bool replicate, T fill, const T* x, const T* we, const T* wd, const T* soft, T* out, uint8_t* tapse,
                                uint8_t* tapsd, const Geom& g, hipStream_t stream)
{
    if (!morpho_pair_supported(g)) return hipErrorInvalidValue;
    if ((int64_t)g.B * g.Cout * g.plane() == 0) return hipSuccess;
    SigmaParams<T> p{};
    p.x = x;
    p.we = we;
    p.wd = wd;
    p.soft = soft;
    p.out = out;
    p.tapse = tapse;
    p.tapsd = tapsd;
    p.replicate = replicate ? 1 : 0;
    p.fill = fill;
    int64_t blocks = 0;
    switch (g.KH)
    {
        case 3: sigma_setup<T, 3>(p, g, blocks); morpho_sigma_fwd_kernel<T, 3><<<(unsigned)blocks, BLOCK, 0, stream>>>(p); break;
        case 5: sigma_setup<T, 5>(p, g, blocks); morpho_sigma_fwd_kernel<T, 5><<<(unsigned)blocks, BLOCK, 0, stream>>>(p); break;
        default: sigma_setup<T, 7>(p, g, blocks); morpho_sigma_fwd_kernel<T, 7><<<(unsigned)blocks, BLOCK, 0, stream>>>(p); break;
    }
    return hipGetLastError();
}

template <typename T>
hipError_t morpho_sigma_backward(bool replicate, T fill, const T* x, const T* we, const T* wd, const T* soft, const uint8_t* tapse,
                                 const uint8_t* tapsd, const T* grad_out, T* grad_in, T* grad_we, T* grad_wd, T* grad_terms, const Geom& g,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream)
{
    if (!morpho_pair_supported(g)) return hipErrorInvalidValue;
    if (workspace_bytes < morpho_sigma_backward_workspace<T>(g)) return hipErrorInvalidValue;
    const int64_t nw = (int64_t)g.Cout * g.taps(), ns = 2 * (int64_t)g.Cout;
    if ((int64_t)g.B * g.Cout * g.plane() == 0)
    {
        hipError_t e = fill_async<T>(grad_we, nw, T(0), stream);
        if (e == hipSuccess) e = fill_async<T>(grad_wd, nw, T(0), stream);
        return e != hipSuccess ? e : fill_async<T>(grad_terms, ns, T(0), stream);
    }
    const int64_t nslots = sigma_slots(g);
    unsigned char* ws = static_cast<unsigned char*>(workspace);
    SigmaParams<T> p{};
    p.x = x;
    p.we = we;
    p.wd = wd;
    p.soft = soft;
    p.tapse = const_cast<uint8_t*>(tapse);
    p.tapsd = const_cast<uint8_t*>(tapsd);
    p.gout = grad_out;
    p.gin = grad_in;
    const size_t pw = align_up((size_t)nslots * nw * sizeof(T));
    p.part_we = reinterpret_cast<T*>(ws);
    p.part_wd = reinterpret_cast<T*>(ws + pw);
    p.part_s = reinterpret_cast<T*>(ws + 2 * pw);
    T* scratch = reinterpret_cast<T*>(ws + 2 * pw + align_up((size_t)nslots * ns * sizeof(T)));
    p.replicate = replicate ? 1 : 0;
    p.fill = fill;
    int64_t blocks = 0;
    switch (g.KH)
    {
        case 3: sigma_setup<T, 3>(p, g, blocks); morpho_sigma_bwd_kernel<T, 3><<<(unsigned)blocks, BLOCK, 0, stream>>>(p); break;
        case 5: sigma_setup<T, 5>(p, g, blocks); morpho_sigma_bwd_kernel<T, 5><<<(unsigned)blocks, BLOCK, 0, stream>>>(p); break;
        default: sigma_setup<T, 7>(p, g, blocks); morpho_sigma_bwd_kernel<T, 7><<<(unsigned)blocks, BLOCK, 0, stream>>>(p); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if ((e = reduce_slots_async<T>(p.part_we, (int)nslots, nw, grad_we, scratch, stream)) != hipSuccess) return e;
    if ((e = reduce_slots_async<T>(p.part_wd, (int)nslots, nw, grad_wd, scratch, stream)) != hipSuccess) return e;
    return reduce_slots_async<T>(p.part_s, (int)nslots, ns, grad_terms, scratch, stream);
}

#define MCA_INSTANTIATE_PAIR(T)                                                                                                           \
    template size_t morpho_pair_backward_workspace<T>(const Geom&);                                                                        \
    template hipError_t morpho_pair_forward<T>(int, bool, T, T, const T*, const T*, const T*, T*, uint8_t*, uint8_t*, const Geom&,         \
                                               hipStream_t);                                                                               \
    template hipError_t morpho_pair_backward<T>(int, const uint8_t*, const uint8_t*, const T*, T*, T*, T*, const Geom&, void*, size_t,     \
                                                hipStream_t);
MCA_INSTANTIATE_PAIR(float)
MCA_INSTANTIATE_PAIR(double)

#define MCA_INSTANTIATE_SIGMA(T)                                                                                                          \
    template size_t morpho_sigma_backward_workspace<T>(const Geom&);                                                                       \
    template hipError_t morpho_sigma_forward<T>(bool, T, const T*, const T*, const T*, const T*, T*, uint8_t*, uint8_t*, const Geom&,      \
                                                hipStream_t);                                                                              \
    template hipError_t morpho_sigma_backward<T>(bool, T, const T*, const T*, const T*, const T*, const uint8_t*, const uint8_t*, const T*, \
                                                 T*, T*, T*, T*, const Geom&, void*, size_t, hipStream_t);
MCA_INSTANTIATE_SIGMA(float)
MCA_INSTANTIATE_SIGMA(double)

}  // namespace mca
