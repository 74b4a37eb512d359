// Shared definitions of the morphocore_amd HIP kernels (gfx950, wave64).
//
// Layout in HBM: every tensor is a dense row-major NCHW array. x [B, Cin, H, W], the structuring
// element w [Cout, Cw, KH, KW] (Cw = Cin, or 1 for IDENTITY), or one structuring element per batch
// element [B, Cout, Cw, KH, KW] when weight noise is active. Outputs [B, Cout, H, W]; packed indices
// int32 [B, Cout, H, W] holding (channel << 16) | tap.
//
// Tap rule (reference: morpho_op_cpu_kernels.hxx:254-263): output (h, w) with tap (kh, kw) reads the
// input pixel (h + KH/2 - kh, w + KW/2 - kw); the flat tap index is kh * KW + kw.
//
// Every tiled kernel here stages one input plane's tile plus its (KH-1, KW-1) halo in LDS. A block
// is four wave64s; lane l of a wave owns output column w0 + l and the wave owns RH consecutive
// output rows, so the tile is 64 columns by 4 * RH rows and every LDS row read is one contiguous,
// conflict-free 64-lane access.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <limits>
#include <type_traits>

namespace mca
{

// Same integer values as the reference (morpho_op_enum.hpp:17-35, merge_enum.py:4-19).
enum Op : int
{
    DILATION = 0,
    EROSION = 1
};

enum Merge : int
{
    MERGE_MAX = 0,
    MERGE_MIN = 1,
    MERGE_ADD = 2,
    MERGE_AVERAGE = 3,
    MERGE_SMOOTH = 4,
    MERGE_IDENTITY = 5
};

// How the per-pair results of one output pixel are combined, as a kernel template argument.
enum MergeKind : int
{
    MK_SUM = 0,  // ADD and AVERAGE (AVERAGE divides once at the end)
    MK_MAX = 1,
    MK_MIN = 2,
    MK_IDENT = 3,  // output channel c reads input channel c only
    MK_SMOOTH = 4  // smorph's SMOOTH merge (smorph_scm): a soft extremum over the pair outputs
};

constexpr int WAVE = 64;
constexpr int NWAVES = 4;
constexpr int BLOCK = WAVE * NWAVES;
constexpr int TILE_W = WAVE;
// Number of XCDs of an MI355X; the dispatcher hands consecutive workgroups to consecutive XCDs.
constexpr int NUM_XCD = 8;

struct Geom
{
    int B, Cin, Cout, Cw, H, W, KH, KW;
    int64_t wbs;  // elements between the structuring elements of consecutive batch elements, 0 if shared

    __host__ __device__ int taps() const { return KH * KW; }
    __host__ __device__ int pad_h() const { return KH / 2; }
    __host__ __device__ int pad_w() const { return KW / 2; }
    __host__ __device__ int64_t plane() const { return (int64_t)H * W; }
};

// Tiling of the output planes: TILE_W x (NWAVES * rh) tiles, staged with their halo.
struct Tiling
{
    int rh;  // output rows per wave
    int th;  // tile height
    int ntx, nty;
    int rows, cols, pitch;  // staged tile shape (pitch in elements)

    __host__ __device__ int ntiles() const { return ntx * nty; }
};

inline Tiling make_tiling(const Geom& g, int rh)
{
    Tiling t;
    t.rh = rh;
    t.th = NWAVES * rh;
    t.ntx = (g.W + TILE_W - 1) / TILE_W;
    t.nty = (g.H + t.th - 1) / t.th;
    t.rows = t.th + g.KH - 1;
    t.cols = TILE_W + g.KW - 1;
    t.pitch = t.cols;
    return t;
}

// Workgroup index -> work item, so that consecutive work items run on the same XCD (and share its L2):
// workgroup b runs on XCD b % 8, which receives a contiguous range of work items. A bijection for
// any grid size.
__device__ inline int xcd_work_index(int bid, int nblocks)
{
    const int per = nblocks / NUM_XCD;
    const int rem = nblocks % NUM_XCD;
    const int xcd = bid % NUM_XCD;
    const int local = bid / NUM_XCD;
    return xcd * per + (xcd < rem ? xcd : rem) + local;
}

// Dilation and erosion, as per-tap combine, strict improvement and start value
// (reference: morpho_op_policy.hpp:10-64). `pick` is the extremum that ignores NaN operands, equal to
// the strict-improvement scan up to the sign of a zero result.
template <int OP, typename T>
struct OpTraits;

template <typename T>
struct OpTraits<DILATION, T>
{
    static __device__ __forceinline__ T combine(T x, T w) { return x + w; }
    static __device__ __forceinline__ bool better(T a, T b) { return a > b; }
    static __device__ __forceinline__ T pick(T a, T b) { return fmax(a, b); }
    static __host__ __device__ __forceinline__ T init() { return -std::numeric_limits<T>::infinity(); }
    static constexpr int sign = 1;
};

template <typename T>
struct OpTraits<EROSION, T>
{
    static __device__ __forceinline__ T combine(T x, T w) { return x - w; }
    static __device__ __forceinline__ bool better(T a, T b) { return a < b; }
    static __device__ __forceinline__ T pick(T a, T b) { return fmin(a, b); }
    static __host__ __device__ __forceinline__ T init() { return std::numeric_limits<T>::infinity(); }
    static constexpr int sign = -1;
};

__host__ __device__ inline size_t align16(size_t v) { return (v + 15) / 16 * 16; }

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// Value a tap reads at input position (y, x) of `plane`: the pixel, the clamped edge pixel for
// REPLICATE, the fill value otherwise (reference: morpho_padding_policy.hpp:22-74).
template <typename T>
__device__ __forceinline__ T read_padded(const T* __restrict__ plane, int H, int W, int y, int x, bool replicate, T fill)
{
    if (y >= 0 && y < H && x >= 0 && x < W) return plane[(int64_t)y * W + x];
    if (!replicate) return fill;
    return plane[(int64_t)clampi(y, 0, H - 1) * W + clampi(x, 0, W - 1)];
}

// Stage rows [y0, y0 + t.rows) x columns [x0, x0 + t.cols) of `plane` (storage type ST) into `tile`
// (compute type T), out-of-image positions resolved by read_padded. Wave v stages rows v, v + NWAVES,
// ...; lanes stride the columns.
template <typename T, typename ST>
__device__ __forceinline__ void stage_tile(T* tile, const ST* __restrict__ plane, const Geom& g, const Tiling& t, int y0, int x0,
                                           bool replicate, T fill)
{
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    for (int ly = wave; ly < t.rows; ly += NWAVES)
    {
        const int y = y0 + ly;
        const bool row_in = y >= 0 && y < g.H;
        const int yc = clampi(y, 0, g.H - 1);
        for (int lx = lane; lx < t.cols; lx += WAVE)
        {
            const int x = x0 + lx;
            T v;
            if (row_in && x >= 0 && x < g.W)
                v = (T)plane[(int64_t)y * g.W + x];
            else if (replicate)
                v = (T)plane[(int64_t)yc * g.W + clampi(x, 0, g.W - 1)];
            else
                v = fill;
            tile[ly * t.pitch + lx] = v;
        }
    }
}

// Storage types of the dilation / erosion operands: float32 and float64 compute in themselves, float16
// and bfloat16 in float32 (every value converts exactly; a result is rounded once, to nearest even,
// when it is stored).
template <typename ST>
struct ComputeOf
{
    using type = ST;
};
template <>
struct ComputeOf<_Float16>
{
    using type = float;
};
template <>
struct ComputeOf<__bf16>
{
    using type = float;
};
template <typename ST>
using compute_t = typename ComputeOf<ST>::type;

// Gradient accumulators kept in LDS are double, for float and double tensors alike: on gfx950 an
// LDS float64 atomic add (ds_add_f64) issues in ~10 cycles per wave instruction while the float32
// one (ds_add_f32) takes ~190 (measured), and the wider sums are also the more accurate.
using Acc = double;

template <typename T>
__device__ __forceinline__ void lds_add(T* p, T v)
{
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <typename T>
__device__ __forceinline__ void global_add(T* p, T v)
{
    unsafeAtomicAdd(p, v);
}

template <typename T>
__device__ __forceinline__ T lowest_of()
{
    return std::numeric_limits<T>::lowest();
}

template <typename T>
__device__ __forceinline__ T max_of()
{
    return std::numeric_limits<T>::max();
}

}  // namespace mca
