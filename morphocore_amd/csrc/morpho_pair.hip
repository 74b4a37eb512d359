// Opening and closing with per-channel ('identity') merges, fused into one pass per tile.
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

#define MCA_INSTANTIATE_PAIR(T)                                                                                                           \
    template size_t morpho_pair_backward_workspace<T>(const Geom&);                                                                        \
    template hipError_t morpho_pair_forward<T>(int, bool, T, T, const T*, const T*, const T*, T*, uint8_t*, uint8_t*, const Geom&,         \
                                               hipStream_t);                                                                               \
    template hipError_t morpho_pair_backward<T>(int, const uint8_t*, const uint8_t*, const T*, T*, T*, T*, const Geom&, void*, size_t,     \
                                                hipStream_t);
MCA_INSTANTIATE_PAIR(float)
MCA_INSTANTIATE_PAIR(double)

}  // namespace mca
