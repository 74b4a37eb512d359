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
// extremal tap saved. The backward pass gathers instead of scattering: grad of the intermediate
// image over the tile plus the first stage's halo from the output gradient and the second stage's
// taps, then grad_input from it and the first stage's taps, in the same order and precision as the
// separate gather kernels (double sums rounded once per pixel), and both structuring-element
// gradients in per-tile partial slots summed in a fixed order.
//
// Tiles are (64 - (K - 1)) output columns by 16 rows, so that the intermediate region a tile needs is
// exactly 64 columns wide: one lane per intermediate column and per output column.
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
    int replicate;
    T fill1, fill2;  // the border value each stage reads (REPLICATE: unused)
};

template <typename T>
struct PairBwdParams
{
    const uint8_t* __restrict__ taps1;
    const uint8_t* __restrict__ taps2;
    const T* __restrict__ gout;
    T* __restrict__ gin;
    T* __restrict__ part1;  // [B * tiles][C][K * K] partial weight gradients of each stage
    T* __restrict__ part2;
    int B, C, H, W;
    int ntx, nty;
};

template <int K>
struct PairTile
{
    static constexpr int P = K / 2;
    static constexpr int RH = 4;                  // output rows per wave
    static constexpr int TH = NWAVES * RH;        // output rows per tile
    static constexpr int OW = TILE_W - (K - 1);   // output columns per tile
    static constexpr int ER = TH + K - 1;         // intermediate rows a tile needs
    static constexpr int RE = (ER + NWAVES - 1) / NWAVES;  // intermediate rows per wave
    static constexpr int XR = ER + K - 1;         // forward: staged input rows
    static constexpr int XC = TILE_W + K - 1;     // forward: staged input columns (backward: output-gradient columns)
};

struct PairWork
{
    int b, c, tx, ty, tile;
};

// Consecutive work items are neighbouring tiles of one plane (they share halo rows in L2).
__device__ __forceinline__ PairWork decode_pair(int C, int ntx, int nty)
{
    int work = xcd_work_index(blockIdx.x, gridDim.x);
    PairWork w;
    w.tx = work % ntx;
    work /= ntx;
    w.ty = work % nty;
    work /= nty;
    w.tile = w.ty * ntx + w.tx;
    w.c = work % C;
    w.b = work / C;
    return w;
}

// Strict first-tap scan of one pixel over a K x K window read from LDS at `base` (tap (kh, kw) at
// base[(K - 1 - kh) * pitch + (K - 1 - kw)]): the extremum and its first tap; a pixel that never
// improves on the start value keeps it with tap 0.
template <int OP, typename T, int K>
__device__ __forceinline__ void pair_scan(const T* base, int pitch, const T* wk, T& best, int& arg)
{
    using Tr = OpTraits<OP, T>;
    best = Tr::init();
    arg = 0;
#pragma unroll
    for (int kh = 0; kh < K; ++kh)
#pragma unroll
        for (int kw = 0; kw < K; ++kw)
        {
            const T v = Tr::combine(base[(K - 1 - kh) * pitch + (K - 1 - kw)], wk[kh * K + kw]);
            const bool up = Tr::better(v, best);
            best = up ? v : best;
            arg = up ? kh * K + kw : arg;
        }
}

template <typename T, int OP1, int K>
__global__ __launch_bounds__(BLOCK) void morpho_pair_fwd_kernel(const PairFwdParams<T> p)
{
    constexpr int OP2 = OP1 == DILATION ? EROSION : DILATION;
    using S = PairTile<K>;
    constexpr int P = S::P, TH = S::TH, OW = S::OW, ER = S::ER, RE = S::RE, XR = S::XR, XC = S::XC, KK = K * K;
    __shared__ T xs[XR * XC];
    __shared__ T es[ER * TILE_W];
    __shared__ T ws[2 * KK];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const PairWork wk = decode_pair(p.C, p.ntx, p.nty);
    const int H = p.H, W = p.W;
    const int64_t plane = (int64_t)H * W;
    const int64_t pbase = ((int64_t)wk.b * p.C + wk.c) * plane;
    const int h0 = wk.ty * TH, c0 = wk.tx * OW;
    // Origins of the intermediate region (second stage's input window) and of the staged input.
    const int ey0 = h0 + P - (K - 1), ex0 = c0 + P - (K - 1);
    const int xy0 = ey0 + P - (K - 1), xx0 = ex0 + P - (K - 1);

    const T* __restrict__ xp = p.x + pbase;
    for (int idx = threadIdx.x; idx < XR * XC; idx += BLOCK)
    {
        const int ly = idx / XC, lx = idx - ly * XC;
        const int y = xy0 + ly, xx = xx0 + lx;
        T v;
        if (y >= 0 && y < H && xx >= 0 && xx < W)
            v = xp[(int64_t)y * W + xx];
        else if (p.replicate)
            v = xp[(int64_t)clampi(y, 0, H - 1) * W + clampi(xx, 0, W - 1)];
        else
            v = p.fill1;
        xs[idx] = v;
    }
    if (threadIdx.x < 2 * KK)
    {
        const int s = threadIdx.x / KK, k = threadIdx.x - s * KK;
        const T* wsrc = (s == 0 ? p.w1 : p.w2) + (int64_t)wk.b * p.wbs + (int64_t)wk.c * KK;
        ws[threadIdx.x] = wsrc[k];
    }
    __syncthreads();

    // First stage over the intermediate region: lane = column, RE consecutive rows per wave. Its taps
    // are saved for the tile's own pixels only (every pixel belongs to exactly one tile).
    T w1r[KK];
#pragma unroll
    for (int k = 0; k < KK; ++k) w1r[k] = ws[k];
    const int gx1 = ex0 + lane;
    const bool own_col1 = lane >= K - 1 - P && lane < K - 1 - P + OW;
    for (int j = 0; j < RE; ++j)
    {
        const int ly = wave * RE + j;
        if (ly >= ER) break;
        const int gy = ey0 + ly;
        T best;
        int arg;
        pair_scan<OP1, T, K>(&xs[ly * XC + lane], XC, w1r, best, arg);
        const bool in = gy >= 0 && gy < H && gx1 >= 0 && gx1 < W;
        es[ly * TILE_W + lane] = in ? best : p.fill2;
        if (p.taps1 && in && own_col1 && ly >= K - 1 - P && ly < K - 1 - P + TH) p.taps1[pbase + (int64_t)gy * W + gx1] = (uint8_t)arg;
    }
    __syncthreads();
    if (p.replicate)
    {
        // Out-of-image positions of the intermediate region read the clamped edge pixel, which lies in
        // the region whenever the region crosses that edge.
        for (int idx = threadIdx.x; idx < ER * TILE_W; idx += BLOCK)
        {
            const int ly = idx / TILE_W, lx = idx - ly * TILE_W;
            const int gy = ey0 + ly, gx = ex0 + lx;
            if (gy >= 0 && gy < H && gx >= 0 && gx < W) continue;
            es[idx] = es[(clampi(gy, 0, H - 1) - ey0) * TILE_W + (clampi(gx, 0, W - 1) - ex0)];
        }
        __syncthreads();
    }

    // Second stage: lane = output column (the first OW lanes), RH rows per wave.
    T w2r[KK];
#pragma unroll
    for (int k = 0; k < KK; ++k) w2r[k] = ws[KK + k];
    const int wc = c0 + lane;
    const int lcol = lane < OW ? lane : OW - 1;  // lanes past the tile read in bounds; their results are dropped
#pragma unroll
    for (int r = 0; r < S::RH; ++r)
    {
        const int lr = wave * S::RH + r;
        const int h = h0 + lr;
        T best;
        int arg;
        pair_scan<OP2, T, K>(&es[lr * TILE_W + lcol], TILE_W, w2r, best, arg);
        if (lane < OW && h < H && wc < W)
        {
            const int64_t oi = pbase + (int64_t)h * W + wc;
            p.out[oi] = best;
            if (p.taps2) p.taps2[oi] = (uint8_t)arg;
        }
    }
}

template <typename T, int OP1, int K>
__global__ __launch_bounds__(BLOCK) void morpho_pair_bwd_kernel(const PairBwdParams<T> p)
{
    constexpr int OP2 = OP1 == DILATION ? EROSION : DILATION;
    using S = PairTile<K>;
    constexpr int P = S::P, TH = S::TH, OW = S::OW, ER = S::ER, RE = S::RE, KK = K * K;
    constexpr int SR = ER + K - 1, SC = S::XC;  // staged output-gradient region
    constexpr int NC = 32;                      // lane-striped copies of each weight-gradient bin
    __shared__ T gs[SR * SC];
    __shared__ int8_t ts[SR * SC];
    __shared__ int8_t te[ER * TILE_W];
    __shared__ T ges[ER * TILE_W];
    __shared__ __align__(16) Acc bins[2 * KK * NC];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const PairWork wk = decode_pair(p.C, p.ntx, p.nty);
    const int H = p.H, W = p.W;
    const int64_t plane = (int64_t)H * W;
    const int64_t pbase = ((int64_t)wk.b * p.C + wk.c) * plane;
    const int h0 = wk.ty * TH, c0 = wk.tx * OW;
    // Intermediate pixels whose gradient reaches the tile's inputs, and the output pixels whose
    // gradient reaches those.
    const int ey0 = h0 - P, ex0 = c0 - P;
    const int sy0 = ey0 - P, sx0 = ex0 - P;

    for (int idx = threadIdx.x; idx < SR * SC; idx += BLOCK)
    {
        const int ly = idx / SC, lx = idx - ly * SC;
        const int y = sy0 + ly, xx = sx0 + lx;
        const bool in = y >= 0 && y < H && xx >= 0 && xx < W;
        const int64_t o = pbase + (int64_t)clampi(y, 0, H - 1) * W + clampi(xx, 0, W - 1);
        const T g = p.gout[o];
        const int t = p.taps2[o];
        gs[idx] = in ? g : T(0);
        ts[idx] = in ? (int8_t)t : (int8_t)-1;
    }
    for (int idx = threadIdx.x; idx < ER * TILE_W; idx += BLOCK)
    {
        const int ly = idx / TILE_W, lx = idx - ly * TILE_W;
        const int y = ey0 + ly, xx = ex0 + lx;
        const bool in = y >= 0 && y < H && xx >= 0 && xx < W;
        const int t = p.taps1[pbase + (int64_t)clampi(y, 0, H - 1) * W + clampi(xx, 0, W - 1)];
        te[idx] = in ? (int8_t)t : (int8_t)-1;
    }
    for (int j = threadIdx.x; j < 2 * KK * NC; j += BLOCK) bins[j] = Acc(0);
    __syncthreads();

    const Acc sign1 = (Acc)OpTraits<OP1, T>::sign, sign2 = (Acc)OpTraits<OP2, T>::sign;
    Acc* bl1 = bins + (lane & (NC - 1));
    Acc* bl2 = bins + KK * NC + (lane & (NC - 1));
    // Gradient of the intermediate image: pixel e collects g(s) from the output pixels s = e +
    // (kh - P, kw - P) whose saved tap k = kh * K + kw read it, summed in tap order.
    const bool own_col1 = lane >= P && lane < P + OW;
    for (int j = 0; j < RE; ++j)
    {
        const int ly = wave * RE + j;
        if (ly >= ER) break;
        Acc s = Acc(0);
#pragma unroll
        for (int kh = 0; kh < K; ++kh)
#pragma unroll
            for (int kw = 0; kw < K; ++kw)
            {
                const int si = (ly + kh) * SC + lane + kw;
                s += ts[si] == kh * K + kw ? (Acc)gs[si] : Acc(0);
            }
        const int t = te[ly * TILE_W + lane];
        const T ge = t >= 0 ? (T)s : T(0);
        ges[ly * TILE_W + lane] = ge;
        // First stage's weight gradient from the tile's own intermediate pixels.
        if (t >= 0 && own_col1 && ly >= P && ly < P + TH) lds_add(&bl1[t * NC], sign1 * (Acc)ge);
    }
    // Second stage's weight gradient from the tile's own output pixels.
#pragma unroll
    for (int r = 0; r < S::RH; ++r)
    {
        const int si = (wave * S::RH + r + 2 * P) * SC + lane + 2 * P;
        const int t = ts[si];
        if (lane < OW && t >= 0) lds_add(&bl2[t * NC], sign2 * (Acc)gs[si]);
    }
    __syncthreads();

    // grad_input: pixel q collects the intermediate gradient of e = q + (kh - P, kw - P) whose first
    // stage tap k read it.
    T* __restrict__ gin = p.gin + pbase;
    const int wc = c0 + lane;
    const int lcol = lane < OW ? lane : OW - 1;  // lanes past the tile read in bounds; their results are dropped
#pragma unroll
    for (int r = 0; r < S::RH; ++r)
    {
        const int lr = wave * S::RH + r;
        Acc s = Acc(0);
#pragma unroll
        for (int kh = 0; kh < K; ++kh)
#pragma unroll
            for (int kw = 0; kw < K; ++kw)
            {
                const int ei = (lr + kh) * TILE_W + lcol + kw;
                s += te[ei] == kh * K + kw ? (Acc)ges[ei] : Acc(0);
            }
        const int h = h0 + lr;
        if (lane < OW && h < H && wc < W) gin[(int64_t)h * W + wc] = (T)s;
    }

    // Bins of both stages to this tile's partial slot, copies summed in a fixed order.
    const int64_t slot = ((int64_t)wk.b * p.ntx * p.nty + wk.tile) * p.C + wk.c;
    for (int j = threadIdx.x; j < 2 * KK; j += BLOCK)
    {
        const Acc* q = bins + (int64_t)j * NC;
        Acc v = Acc(0);
#pragma unroll
        for (int n = 0; n < NC; ++n) v += q[n];
        const int s = j / KK, k = j - s * KK;
        (s == 0 ? p.part1 : p.part2)[slot * KK + k] = (T)v;
    }
}

// ------------------------------------------------------------------------------------------------
// Launch
// ------------------------------------------------------------------------------------------------

bool morpho_pair_supported(const Geom& g) { return g.KH == g.KW && (g.KH == 3 || g.KH == 5 || g.KH == 7); }

static void pair_tiles(const Geom& g, int& ntx, int& nty)
{
    const int ow = TILE_W - (g.KW - 1), th = NWAVES * 4;
    ntx = (g.W + ow - 1) / ow;
    nty = (g.H + th - 1) / th;
}

template <typename T>
size_t morpho_pair_backward_workspace(const Geom& g)
{
    int ntx, nty;
    pair_tiles(g, ntx, nty);
    const int64_t nslots = (int64_t)g.B * ntx * nty;
    const int64_t n = (int64_t)g.Cout * g.taps();
    return 2 * align_up((size_t)nslots * n * sizeof(T)) + align_up(reduce_slots_scratch<T>((int)nslots, n));
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
    p.replicate = replicate ? 1 : 0;
    p.fill1 = fill1;
    p.fill2 = fill2;
    const int64_t blocks = (int64_t)g.B * g.Cout * p.ntx * p.nty;
    return first_op == EROSION ? pair_fwd_launch<T, EROSION>(p, g.KH, blocks, stream) : pair_fwd_launch<T, DILATION>(p, g.KH, blocks, stream);
}

template <typename T, int OP1>
static hipError_t pair_bwd_launch(const PairBwdParams<T>& p, int K, int64_t blocks, hipStream_t stream)
{
    switch (K)
    {
        case 3: morpho_pair_bwd_kernel<T, OP1, 3><<<(unsigned)blocks, BLOCK, 0, stream>>>(p); break;
        case 5: morpho_pair_bwd_kernel<T, OP1, 5><<<(unsigned)blocks, BLOCK, 0, stream>>>(p); break;
        default: morpho_pair_bwd_kernel<T, OP1, 7><<<(unsigned)blocks, BLOCK, 0, stream>>>(p); break;
    }
    return hipGetLastError();
}

template <typename T>
hipError_t morpho_pair_backward(int first_op, const uint8_t* taps1, const uint8_t* taps2, const T* grad_out, T* grad_in, T* grad_w1,
                                T* grad_w2, const Geom& g, void* workspace, size_t workspace_bytes, hipStream_t stream)
{
    if (!morpho_pair_supported(g)) return hipErrorInvalidValue;
    if (workspace_bytes < morpho_pair_backward_workspace<T>(g)) return hipErrorInvalidValue;
    const int64_t n = (int64_t)g.Cout * g.taps();
    if ((int64_t)g.B * g.Cout * g.plane() == 0)
    {
        hipError_t e = fill_async<T>(grad_w1, n, T(0), stream);
        return e != hipSuccess ? e : fill_async<T>(grad_w2, n, T(0), stream);
    }
    PairBwdParams<T> p{};
    p.taps1 = taps1;
    p.taps2 = taps2;
    p.gout = grad_out;
    p.gin = grad_in;
    p.B = g.B;
    p.C = g.Cout;
    p.H = g.H;
    p.W = g.W;
    pair_tiles(g, p.ntx, p.nty);
    const int64_t nslots = (int64_t)g.B * p.ntx * p.nty;
    unsigned char* ws = static_cast<unsigned char*>(workspace);
    const size_t part_bytes = align_up((size_t)nslots * n * sizeof(T));
    p.part1 = reinterpret_cast<T*>(ws);
    p.part2 = reinterpret_cast<T*>(ws + part_bytes);
    T* scratch = reinterpret_cast<T*>(ws + 2 * part_bytes);
    const int64_t blocks = (int64_t)g.B * g.Cout * p.ntx * p.nty;
    hipError_t e = first_op == EROSION ? pair_bwd_launch<T, EROSION>(p, g.KH, blocks, stream)
                                       : pair_bwd_launch<T, DILATION>(p, g.KH, blocks, stream);
    if (e != hipSuccess) return e;
    e = reduce_slots_async<T>(p.part1, (int)nslots, n, grad_w1, scratch, stream);
    if (e != hipSuccess) return e;
    return reduce_slots_async<T>(p.part2, (int)nslots, n, grad_w2, scratch, stream);
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
