// Dilation / erosion with the IDENTITY merge (each channel with its own element: configs[3]'s layer),
// 3x3 and 5x5 elements, as streaming kernels over row bands of whole image rows (reference semantics:
// morpho_op_cpu_kernels.hxx:202-296 for the strict first-tap scan, morpho_op_cpu_backward.hxx:90-156
// for the routing). The work is ~1 flop per byte moved, so these kernels are bound by HBM: each
// workgroup takes one band of R rows of one (batch element, channel) plane at its full width, stages
// the band and its (KS / 2)-row halo in LDS with 16-byte non-temporal loads, computes every output of
// the band from LDS and writes 16-byte non-temporal stores. Consecutive workgroups take consecutive
// bands of a plane on one XCD (xcd_work_index), so a band's halo rows are its neighbours' rows, read
// from that XCD's L2.
//
//   ident_band_fwd     out = the pair extremum, TAPS: also the first extremal tap (one byte per pixel)
//   ident_band_gather  grad_input gathered per input pixel from the taps of the outputs that read it,
//                      in tap order, and the band's grad_weight sums (one partial slot per band)
//
// They take planes whose width is a multiple of 8 (whole 16-byte vectors per row for every dtype) and
// whose band fits the LDS (ident_bands); other shapes run the tiled kernels.
#include <type_traits>

#include "launch.hpp"

namespace mca
{

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Elements of the LDS rows left and right of the image columns: 8 for every dtype, so that row
// starts stay 16-byte aligned and the halo columns of a 5x5 element fit.
constexpr int IDENT_HALO = 8;
// Copies of the grad_weight bins in LDS (lane-striped, as the tiled kernels).
constexpr int IDENT_NC = 32;
// 16-byte vectors each thread has in flight while staging a band (a 16-row float64 band of a 112-wide
// plane is 4 per thread).
constexpr int IDENT_NB = 4;

IdentBands ident_bands(const Geom& g, size_t elem_bytes, bool backward)
{
    IdentBands s{0, 0, 0};
    if (g.KH != g.KW || (g.KH != 3 && g.KH != 5) || g.W % 8 != 0 || g.W <= 0 || g.H <= 0 || g.Cw != 1) return s;
    const int P = g.KH / 2;
    const size_t pitch = (size_t)g.W + 2 * IDENT_HALO;
    auto bytes = [&](int R) {
        const size_t rows = (size_t)R + 2 * P;
        return align16(rows * pitch * elem_bytes) + (backward ? align16(rows * pitch) + (size_t)g.taps() * IDENT_NC * sizeof(Acc) : 0);
    };
    // The tallest band of 16, 8 or 4 rows whose LDS leaves room for several workgroups per CU.
    for (int R : {16, 8, 4})
        if (bytes(R) <= (R > 4 ? 40 * 1024 : LDS_LIMIT))
        {
            s.R = R;
            s.nbands = (g.H + R - 1) / R;
            s.lds = bytes(R);
            return s;
        }
    return s;
}

template <typename ST>
struct IdentFwdParams
{
    const ST* __restrict__ x;
    const ST* __restrict__ w;
    ST* __restrict__ out;
    uint8_t* __restrict__ taps;  // null: not saved
    Geom g;
    int R, nbands;
    int replicate;
    ST fill;
};

// One band of one plane: (batch element, channel, band) from the workgroup index, bands fastest.
struct IdentWork
{
    int b, c, h0, hn;
};

__device__ __forceinline__ IdentWork ident_work(const Geom& g, int R, int nbands)
{
    int work = xcd_work_index(blockIdx.x, gridDim.x);
    IdentWork w;
    const int band = work % nbands;
    work /= nbands;
    w.c = work % g.Cout;
    w.b = work / g.Cout;
    w.h0 = band * R;
    w.hn = min(R, g.H - w.h0);
    return w;
}

template <typename ST, int N>
__device__ __forceinline__ void store_bytes(uint8_t* p, const int (&a)[N])
{
    if constexpr (N == 2)
        *reinterpret_cast<uint16_t*>(p) = (uint16_t)(a[0] | (a[1] << 8));
    else
        *reinterpret_cast<uint32_t*>(p) = (uint32_t)(a[0] | (a[1] << 8) | (a[2] << 16) | (a[3] << 24));
}

// Stages `rows` image rows from row y0 of one plane into an LDS tile of row pitch `pitch` (image column
// x at H8 + x): rows outside the image are the clamped row (replicate) or the fill value; then the P
// columns left and right of every staged row (replicate: the row's edge pixel, else the fill value).
// IDENT_NB vectors per thread are in flight at once: every load of a batch is issued (clamped into the
// plane, so unconditionally) before any is waited for.
template <typename ST, int P>
__device__ __forceinline__ void band_stage(ST* tile, const ST* __restrict__ xp, const Geom& g, int pitch, int rows, int y0, bool replicate,
                                           ST fill)
{
    constexpr int V = 16 / sizeof(ST), H8 = IDENT_HALO;
    const int nv = g.W / V;
    u32x4 fillv;
    {
        ST f[V];
#pragma unroll
        for (int e = 0; e < V; ++e) f[e] = fill;
        __builtin_memcpy(&fillv, f, 16);
    }
    const int total = rows * nv;
    for (int j0 = threadIdx.x; j0 < total; j0 += IDENT_NB * BLOCK)
    {
        u32x4 v[IDENT_NB];
#pragma unroll
        for (int u = 0; u < IDENT_NB; ++u)
        {
            const int j = min(j0 + u * BLOCK, total - 1);
            const int lr = j / nv, vi = j - lr * nv;
            v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xp + (int64_t)clampi(y0 + lr, 0, g.H - 1) * g.W) + vi);
        }
        // Keeps the compiler from sinking each load into the conditional store that uses it.
#pragma unroll
        for (int u = 0; u < IDENT_NB; ++u) asm volatile("" : "+v"(v[u]));
#pragma unroll
        for (int u = 0; u < IDENT_NB; ++u)
        {
            const int j = j0 + u * BLOCK;
            if (j >= total) break;
            const int lr = j / nv, vi = j - lr * nv;
            const int y = y0 + lr;
            *reinterpret_cast<u32x4*>(tile + lr * pitch + H8 + vi * V) = ((unsigned)y < (unsigned)g.H || replicate) ? v[u] : fillv;
        }
    }
    for (int j = threadIdx.x; j < rows * 2 * P; j += BLOCK)
    {
        const int lr = j / (2 * P), q = j - lr * (2 * P);
        const bool right = q >= P;
        const int col = right ? g.W + (q - P) : -1 - q;
        ST v = fill;
        if (replicate) v = xp[(int64_t)clampi(y0 + lr, 0, g.H - 1) * g.W + (right ? g.W - 1 : 0)];
        tile[lr * pitch + H8 + col] = v;
    }
}

// V consecutive outputs (image columns x0 ..) of one row from an LDS tile laid out as band_stage's,
// whose row r + 2P - kh holds the input row that the outputs' tap row kh reads: the extremum
// (NaN-ignoring, from the start value) and, for TAPS, the first tap (kh, then kw) equal to it, which is
// the tap the reference's strict scan keeps; a pair that never improves on the start value keeps tap 0.
template <typename ST, int OP, int KS, bool TAPS>
__device__ __forceinline__ void band_scan(const ST* tile, int pitch, int r, int x0, const ST (&wv)[KS * KS], ST (&res)[16 / sizeof(ST)],
                                          int (&arg)[16 / sizeof(ST)])
{
    using Tr = OpTraits<OP, ST>;
    constexpr int P = KS / 2, K = KS * KS, V = 16 / sizeof(ST), H8 = IDENT_HALO;
    // Output (h, w) tap (kh, kw) reads input (h + P - kh, w + P - kw): LDS row r + 2P - kh, column
    // H8 + w + P - kw.
    ST win[KS][V + 2 * P];
#pragma unroll
    for (int kh = 0; kh < KS; ++kh)
#pragma unroll
        for (int cc = 0; cc < V + 2 * P; ++cc) win[kh][cc] = tile[(r + 2 * P - kh) * pitch + H8 + x0 - P + cc];
    auto tap = [&](int e, int k) { return Tr::combine(win[k / KS][e + 2 * P - k % KS], wv[k]); };
    bool zero = false;
#pragma unroll
    for (int e = 0; e < V; ++e)
    {
        ST best = Tr::init();
#pragma unroll
        for (int k = 0; k < K; ++k) best = Tr::pick(best, tap(e, k));
        res[e] = best;
        zero |= best == ST(0);
        if constexpr (TAPS)
        {
            int a = 0;
#pragma unroll
            for (int k = K - 1; k >= 0; --k) a = tap(e, k) == best ? k : a;
            arg[e] = best == Tr::init() ? 0 : a;
        }
    }
    // A zero extremum takes the sign of its first tap (the NaN-ignoring extremum does not order -0 and
    // +0; the strict scan keeps the first): rare, so behind a branch uniform over the active lanes.
    if (__builtin_amdgcn_ballot_w64(zero))
    {
#pragma unroll
        for (int e = 0; e < V; ++e)
        {
            ST first = res[e];
#pragma unroll
            for (int k = K - 1; k >= 0; --k) first = tap(e, k) == res[e] ? tap(e, k) : first;
            res[e] = res[e] == ST(0) ? first : res[e];
        }
    }
}

template <typename ST, int OP, int KS, bool TAPS>
__global__ __launch_bounds__(BLOCK) void ident_band_fwd(const IdentFwdParams<ST> p)
{
    constexpr int P = KS / 2, K = KS * KS, V = 16 / sizeof(ST);
    extern __shared__ __align__(16) unsigned char smem[];
    ST* tile = reinterpret_cast<ST*>(smem);
    const Geom& g = p.g;
    const IdentWork wk = ident_work(g, p.R, p.nbands);
    const int pitch = g.W + 2 * IDENT_HALO, nv = g.W / V;
    const int64_t plane = g.plane();
    const ST* __restrict__ xp = p.x + ((int64_t)wk.b * g.Cin + wk.c) * plane;

    // The band's rows and its P halo rows above and below.
    band_stage<ST, P>(tile, xp, g, pitch, wk.hn + 2 * P, wk.h0 - P, p.replicate != 0, p.fill);
    ST wv[K];
    const ST* __restrict__ wp = p.w + (int64_t)wk.b * g.wbs + (int64_t)wk.c * K;
#pragma unroll
    for (int k = 0; k < K; ++k) wv[k] = wp[k];
    __syncthreads();

    ST* __restrict__ op = p.out + ((int64_t)wk.b * g.Cout + wk.c) * plane;
    for (int j = threadIdx.x; j < wk.hn * nv; j += BLOCK)
    {
        const int r = j / nv, vi = j - r * nv;
        const int x0 = vi * V;
        ST res[V];
        int arg[V];
        band_scan<ST, OP, KS, TAPS>(tile, pitch, r, x0, wv, res, arg);
        const int64_t o = (int64_t)(wk.h0 + r) * g.W + x0;
        u32x4 ov;
        __builtin_memcpy(&ov, res, 16);
        __builtin_nontemporal_store(ov, reinterpret_cast<u32x4*>(op + o));
        if constexpr (TAPS) store_bytes<ST>(p.taps + ((int64_t)wk.b * g.Cout + wk.c) * plane + o, arg);
    }
}

template <typename ST>
hipError_t ident_band_forward(int op, bool replicate, ST fill, const ST* x, const ST* w, ST* out, uint8_t* taps, const Geom& g,
                              hipStream_t stream)
{
    const IdentBands s = ident_bands(g, sizeof(ST), false);
    if (s.R == 0 || g.Cin != g.Cout) return hipErrorInvalidValue;
    IdentFwdParams<ST> p{};
    p.x = x;
    p.w = w;
    p.out = out;
    p.taps = taps;
    p.g = g;
    p.R = s.R;
    p.nbands = s.nbands;
    p.replicate = replicate ? 1 : 0;
    p.fill = fill;
    const unsigned blocks = (unsigned)((int64_t)g.B * g.Cout * s.nbands);
    const bool t = taps != nullptr;
#define MCA_IDENT_FWD(OP, KS, TAPS) ident_band_fwd<ST, OP, KS, TAPS><<<blocks, BLOCK, s.lds, stream>>>(p)
    if (op == DILATION)
    {
        if (g.KH == 3)
            t ? MCA_IDENT_FWD(DILATION, 3, true) : MCA_IDENT_FWD(DILATION, 3, false);
        else
            t ? MCA_IDENT_FWD(DILATION, 5, true) : MCA_IDENT_FWD(DILATION, 5, false);
    }
    else
    {
        if (g.KH == 3)
            t ? MCA_IDENT_FWD(EROSION, 3, true) : MCA_IDENT_FWD(EROSION, 3, false);
        else
            t ? MCA_IDENT_FWD(EROSION, 5, true) : MCA_IDENT_FWD(EROSION, 5, false);
    }
#undef MCA_IDENT_FWD
    return hipGetLastError();
}

template <typename T, typename ST>
struct IdentGatherParams
{
    const ST* __restrict__ gout;
    const uint8_t* __restrict__ taps;
    ST* __restrict__ gin;
    T* __restrict__ part;  // [B * nbands][Cout][K]: the band's grad_weight sums
    Geom g;
    int R, nbands;
};

constexpr uint8_t IDENT_NONE = 0xff;  // a tap byte that matches no tap: outside the image

// Stages `rows` rows from row y0 of an output-gradient plane and of its tap plane into LDS tiles of
// pitch `pitch` (image column x at H8 + x), as band_stage: rows outside the image and the P columns
// left and right of every row hold no gradient (0) and no tap (IDENT_NONE).
template <typename ST, int P>
__device__ __forceinline__ void gather_stage(ST* gs, uint8_t* ts, const ST* __restrict__ gp, const uint8_t* __restrict__ tp, const Geom& g,
                                             int pitch, int rows, int y0)
{
    constexpr int V = 16 / sizeof(ST), H8 = IDENT_HALO;
    using TapBits = std::conditional_t<V == 2, uint16_t, std::conditional_t<V == 4, uint32_t, uint64_t>>;
    const TapBits none = (TapBits)~(TapBits)0;
    const int nv = g.W / V;
    const int total = rows * nv;
    const u32x4 zero = {0u, 0u, 0u, 0u};
    for (int j0 = threadIdx.x; j0 < total; j0 += IDENT_NB * BLOCK)
    {
        u32x4 v[IDENT_NB];
        TapBits t[IDENT_NB];
#pragma unroll
        for (int u = 0; u < IDENT_NB; ++u)
        {
            const int j = min(j0 + u * BLOCK, total - 1);
            const int lr = j / nv, vi = j - lr * nv;
            const int64_t row = (int64_t)clampi(y0 + lr, 0, g.H - 1) * g.W;
            v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gp + row) + vi);
            t[u] = reinterpret_cast<const TapBits*>(tp + row)[vi];
        }
#pragma unroll
        for (int u = 0; u < IDENT_NB; ++u) asm volatile("" : "+v"(v[u]), "+v"(t[u]));
#pragma unroll
        for (int u = 0; u < IDENT_NB; ++u)
        {
            const int j = j0 + u * BLOCK;
            if (j >= total) break;
            const int lr = j / nv, vi = j - lr * nv;
            const bool in = (unsigned)(y0 + lr) < (unsigned)g.H;
            *reinterpret_cast<u32x4*>(gs + lr * pitch + H8 + vi * V) = in ? v[u] : zero;
            *reinterpret_cast<TapBits*>(ts + lr * pitch + H8 + vi * V) = in ? t[u] : none;
        }
    }
    for (int j = threadIdx.x; j < rows * 2 * P; j += BLOCK)
    {
        const int lr = j / (2 * P), q = j - lr * (2 * P);
        const int col = q >= P ? g.W + (q - P) : -1 - q;
        gs[lr * pitch + H8 + col] = ST(0);
        ts[lr * pitch + H8 + col] = IDENT_NONE;
    }
}

// grad_input of V consecutive pixels (image columns x0 ..) of one row, gathered in tap order from the
// output gradients gs and taps ts staged as gather_stage's: input pixel (y, x) receives the gradient of
// output (y - P + kh, x - P + kw) when that output's tap is (kh, kw), at LDS row r + kh, column
// H8 + x - P + kw. With OWN, also the grad_weight terms of the outputs at the pixels' own positions
// (row r + P) into the copy `copy` of the K bins. The window of the V pixels is read first,
// unconditionally (a read inside the selection becomes a branch around each read, one LDS round trip
// after another).
template <typename T, int OP, int KS, typename ST>
__device__ __forceinline__ void gather_vec(const ST* gs, const uint8_t* ts, int pitch, int r, int x0, bool own, Acc* bins, int copy,
                                           ST (&res)[16 / sizeof(ST)])
{
    constexpr int P = KS / 2, K = KS * KS, V = 16 / sizeof(ST), H8 = IDENT_HALO, NC = IDENT_NC;
    uint8_t tw[KS][V + 2 * P];
    T gw[KS][V + 2 * P];
#pragma unroll
    for (int kh = 0; kh < KS; ++kh)
#pragma unroll
        for (int cc = 0; cc < V + 2 * P; ++cc)
        {
            const int idx = (r + kh) * pitch + H8 + x0 - P + cc;
            tw[kh][cc] = ts[idx];
            gw[kh][cc] = (T)gs[idx];
        }
#pragma unroll
    for (int e = 0; e < V; ++e)
    {
        Acc s = Acc(0);
#pragma unroll
        for (int kh = 0; kh < KS; ++kh)
#pragma unroll
            for (int kw = 0; kw < KS; ++kw) s += tw[kh][e + kw] == kh * KS + kw ? (Acc)gw[kh][e + kw] : Acc(0);
        res[e] = (ST)(T)s;
        // grad_weight: the output pixel at the same position (window row P, column e + P).
        const T gv = gw[P][e + P];
        const int k = tw[P][e + P];
        if (own && k < K) lds_add(&bins[k * NC + copy], (Acc)(OP == DILATION ? gv : -gv));
    }
}

// The band's grad_weight bins into its partial slot: 8 threads per tap each add 4 copies, a butterfly
// over the 8 finishes. The caller synchronises the workgroup first.
template <typename T, int K>
__device__ __forceinline__ void flush_bins(const Acc* bins, T* slot)
{
    static_assert(K * 8 <= BLOCK, "one pass over the bins");
    static_assert(IDENT_NC == 32, "four copies per thread");
    if (threadIdx.x < K * 8)
    {
        const Acc* q = bins + threadIdx.x * 4;
        Acc v = (q[0] + q[1]) + (q[2] + q[3]);
#pragma unroll
        for (int d = 4; d >= 1; d /= 2) v += __shfl_xor(v, d, 8);
        if ((threadIdx.x & 7) == 0) slot[threadIdx.x >> 3] = (T)v;
    }
}

// T: the type of the sums and partial slots (float for 16-bit storage), ST: the storage type of the
// gradients.
template <typename T, int OP, int KS, typename ST>
__global__ __launch_bounds__(BLOCK) void ident_band_gather(const IdentGatherParams<T, ST> p)
{
    constexpr int P = KS / 2, K = KS * KS, V = 16 / sizeof(ST), NC = IDENT_NC;
    extern __shared__ __align__(16) unsigned char smem[];
    const Geom& g = p.g;
    const IdentWork wk = ident_work(g, p.R, p.nbands);
    const int pitch = g.W + 2 * IDENT_HALO, nv = g.W / V, rows_max = p.R + 2 * P;
    ST* gs = reinterpret_cast<ST*>(smem);
    uint8_t* ts = smem + align16((size_t)rows_max * pitch * sizeof(ST));
    Acc* bins = reinterpret_cast<Acc*>(ts + align16((size_t)rows_max * pitch));
    const int64_t plane = g.plane();
    const int64_t pl = ((int64_t)wk.b * g.Cout + wk.c) * plane;

    for (int j = threadIdx.x; j < K * NC; j += BLOCK) bins[j] = Acc(0);
    // The band's output rows and the P rows around them: gradient and tap of every output pixel that
    // reads a pixel of the band.
    gather_stage<ST, P>(gs, ts, p.gout + pl, p.taps + pl, g, pitch, wk.hn + 2 * P, wk.h0 - P);
    __syncthreads();

    ST* __restrict__ ip = p.gin + ((int64_t)wk.b * g.Cin + wk.c) * plane;
    const int copy = threadIdx.x & (NC - 1);
    for (int j = threadIdx.x; j < wk.hn * nv; j += BLOCK)
    {
        const int r = j / nv, vi = j - r * nv;
        const int x0 = vi * V;
        ST res[V];
        gather_vec<T, OP, KS, ST>(gs, ts, pitch, r, x0, true, bins, copy, res);
        u32x4 ov;
        __builtin_memcpy(&ov, res, 16);
        __builtin_nontemporal_store(ov, reinterpret_cast<u32x4*>(ip + (int64_t)(wk.h0 + r) * g.W + x0));
    }
    __syncthreads();
    flush_bins<T, K>(bins, p.part + ((int64_t)wk.b * p.nbands + wk.h0 / p.R) * g.Cout * K + (int64_t)wk.c * K);
}

template <typename T, typename ST>
hipError_t ident_band_backward(int op, const uint8_t* taps, const ST* grad_out, ST* grad_in, T* part, const Geom& g, hipStream_t stream)
{
    const IdentBands s = ident_bands(g, sizeof(ST), true);
    if (s.R == 0 || g.Cin != g.Cout || g.taps() > 255) return hipErrorInvalidValue;
    IdentGatherParams<T, ST> p{};
    p.gout = grad_out;
    p.taps = taps;
    p.gin = grad_in;
    p.part = part;
    p.g = g;
    p.R = s.R;
    p.nbands = s.nbands;
    const unsigned blocks = (unsigned)((int64_t)g.B * g.Cout * s.nbands);
    if (op == DILATION)
    {
        if (g.KH == 3)
            ident_band_gather<T, DILATION, 3, ST><<<blocks, BLOCK, s.lds, stream>>>(p);
        else
            ident_band_gather<T, DILATION, 5, ST><<<blocks, BLOCK, s.lds, stream>>>(p);
    }
    else
    {
        if (g.KH == 3)
            ident_band_gather<T, EROSION, 3, ST><<<blocks, BLOCK, s.lds, stream>>>(p);
        else
            ident_band_gather<T, EROSION, 5, ST><<<blocks, BLOCK, s.lds, stream>>>(p);
    }
    return hipGetLastError();
}

template hipError_t ident_band_forward<float>(int, bool, float, const float*, const float*, float*, uint8_t*, const Geom&, hipStream_t);
template hipError_t ident_band_forward<double>(int, bool, double, const double*, const double*, double*, uint8_t*, const Geom&,
                                               hipStream_t);
template hipError_t ident_band_backward<float, float>(int, const uint8_t*, const float*, float*, float*, const Geom&, hipStream_t);
template hipError_t ident_band_backward<double, double>(int, const uint8_t*, const double*, double*, double*, const Geom&, hipStream_t);
template hipError_t ident_band_backward<float, _Float16>(int, const uint8_t*, const _Float16*, _Float16*, float*, const Geom&, hipStream_t);
template hipError_t ident_band_backward<float, __bf16>(int, const uint8_t*, const __bf16*, __bf16*, float*, const Geom&, hipStream_t);

}  // namespace mca
