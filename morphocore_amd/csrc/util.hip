// Small helper kernels shared by the launchers: fill (zeroing accumulators without hipMemsetAsync,
// so that the launches stay valid under stream capture) and the fixed-order sum of per-workgroup
// partial slots.
#include <atomic>

#include "launch.hpp"

namespace mca
{

template <typename T>
__global__ __launch_bounds__(BLOCK) void fill_kernel(T* __restrict__ p, int64_t n, T v)
{
    for (int64_t j = (int64_t)blockIdx.x * BLOCK + threadIdx.x; j < n; j += (int64_t)gridDim.x * BLOCK) p[j] = v;
}

// Sum of part[s * n + j] over the slots s0 <= s < s1, in slot order, accumulated in double. The loads
// of REDUCE_GROUP slots are all issued before the first add (in bounds: clamped), so a thread waits
// once per group instead of once per slot; slots past s1 add +0, which leaves the sum unchanged (it
// starts at +0 and can never become -0).
template <typename T>
__device__ __forceinline__ Acc sum_slots(const T* __restrict__ part, int s0, int s1, int64_t n, int64_t j)
{
    Acc s = Acc(0);
    for (int b = s0; b < s1; b += REDUCE_GROUP)
    {
        T v[REDUCE_GROUP];
#pragma unroll
        for (int u = 0; u < REDUCE_GROUP; ++u) v[u] = part[(int64_t)min(b + u, s1 - 1) * n + j];
#pragma unroll
        for (int u = 0; u < REDUCE_GROUP; ++u) s += b + u < s1 ? (Acc)v[u] : Acc(0);
    }
    return s;
}

// out[j] = sum over slots s = 0, 1, ... of part[s * n + j], always in slot order, accumulated in
// double and rounded once.
template <typename T>
__global__ __launch_bounds__(BLOCK) void reduce_slots_kernel(const T* __restrict__ part, int nslots, int64_t n, T* __restrict__ out)
{
    for (int64_t j = (int64_t)blockIdx.x * BLOCK + threadIdx.x; j < n; j += (int64_t)gridDim.x * BLOCK)
        out[j] = (T)sum_slots(part, 0, nslots, n, j);
}

// First stage of a long reduction: group blockIdx.y sums slots [y * REDUCE_GROUP, (y + 1) *
// REDUCE_GROUP) in slot order into tmp[y * n + j]; the groups are then summed in group order.
template <typename T>
__global__ __launch_bounds__(BLOCK) void reduce_groups_kernel(const T* __restrict__ part, int nslots, int64_t n, T* __restrict__ tmp)
{
    const int s0 = blockIdx.y * REDUCE_GROUP;
    const int s1 = min(s0 + REDUCE_GROUP, nslots);
    for (int64_t j = (int64_t)blockIdx.x * BLOCK + threadIdx.x; j < n; j += (int64_t)gridDim.x * BLOCK)
        tmp[(int64_t)blockIdx.y * n + j] = (T)sum_slots(part, s0, s1, n, j);
}

// dst[j] = (T)src[j]: a double accumulator rounded once into its float32 result.
template <typename T>
__global__ __launch_bounds__(BLOCK) void round_kernel(const double* __restrict__ src, T* __restrict__ dst, int64_t n)
{
    for (int64_t j = (int64_t)blockIdx.x * BLOCK + threadIdx.x; j < n; j += (int64_t)gridDim.x * BLOCK) dst[j] = (T)src[j];
}

// acc[j] = (first ? 0 : acc[j]) + part[j] in double: partial sums added in call order, rounded once by
// round_async (or read as double) at the end.
template <typename T>
__global__ __launch_bounds__(BLOCK) void accumulate_kernel(double* __restrict__ acc, const T* __restrict__ part, int64_t n, int first)
{
    for (int64_t j = (int64_t)blockIdx.x * BLOCK + threadIdx.x; j < n; j += (int64_t)gridDim.x * BLOCK)
        acc[j] = (first ? 0.0 : acc[j]) + (double)part[j];
}

// Per-sample structuring elements of weight noise: out[b][j] = w[j] + (u[b][j] * 2 - 1) * scale, with
// the roundings of the four elementwise operations torch evaluates it with (morpho_op_wrap.hxx:55-64),
// in their order, so that the elements are bit for bit the ones the composed expression gives.
template <typename T>
__global__ __launch_bounds__(BLOCK) void noise_sample_kernel(const T* __restrict__ w, const T* __restrict__ u, T scale, T* __restrict__ out,
                                                             int64_t n, int64_t total)
{
#pragma clang fp contract(off)
    for (int64_t j = (int64_t)blockIdx.x * BLOCK + threadIdx.x; j < total; j += (int64_t)gridDim.x * BLOCK)
    {
        const T t = u[j] * T(2);
        const T v = (t - T(1)) * scale;
        out[j] = w[j % n] + v;
    }
}

// dst[j] = src[j] converted: float16 / bfloat16 storage to its float32 compute type (exact) and back
// (rounded to nearest even).
template <typename S, typename D>
__global__ __launch_bounds__(BLOCK) void convert_kernel(const S* __restrict__ src, D* __restrict__ dst, int64_t n)
{
    for (int64_t j = (int64_t)blockIdx.x * BLOCK + threadIdx.x; j < n; j += (int64_t)gridDim.x * BLOCK) dst[j] = (D)(float)src[j];
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
size_t reduce_slots_scratch(int nslots, int64_t n)
{
    return nslots > REDUCE_GROUP ? (size_t)((nslots + REDUCE_GROUP - 1) / REDUCE_GROUP) * (size_t)n * sizeof(T) : 0;
}

template <typename T>
hipError_t reduce_slots_async(const T* part, int nslots, int64_t n, T* out, T* scratch, hipStream_t stream)
{
    if (n <= 0) return hipSuccess;
    if (nslots <= REDUCE_GROUP)
    {
        reduce_slots_kernel<T><<<grid_for(n), BLOCK, 0, stream>>>(part, nslots, n, out);
        return hipGetLastError();
    }
    const int groups = (nslots + REDUCE_GROUP - 1) / REDUCE_GROUP;
    const dim3 grid((unsigned)grid_for(n), (unsigned)groups);
    reduce_groups_kernel<T><<<grid, BLOCK, 0, stream>>>(part, nslots, n, scratch);
    reduce_slots_kernel<T><<<grid_for(n), BLOCK, 0, stream>>>(scratch, groups, n, out);
    return hipGetLastError();
}

size_t device_lds_limit()
{
    constexpr int MAX_DEVICES = 64;
    static std::atomic<int64_t> cached[MAX_DEVICES] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return LDS_LIMIT;
    if (dev < MAX_DEVICES)
    {
        const int64_t c = cached[dev].load(std::memory_order_relaxed);
        if (c > 0) return (size_t)c;
    }
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0) return LDS_LIMIT;
    if (dev < MAX_DEVICES) cached[dev].store(v, std::memory_order_relaxed);
    return (size_t)v;
}

template <typename T>
hipError_t round_async(const double* src, T* dst, int64_t n, hipStream_t stream)
{
    if (n <= 0) return hipSuccess;
    round_kernel<T><<<grid_for(n), BLOCK, 0, stream>>>(src, dst, n);
    return hipGetLastError();
}

template <typename T>
hipError_t accumulate_async(double* acc, const T* part, int64_t n, bool first, hipStream_t stream)
{
    if (n <= 0) return hipSuccess;
    accumulate_kernel<T><<<grid_for(n), BLOCK, 0, stream>>>(acc, part, n, first ? 1 : 0);
    return hipGetLastError();
}

template <typename T>
hipError_t noise_sample_async(const T* w, const T* u, T scale, T* out, int64_t n, int64_t batch, hipStream_t stream)
{
    const int64_t total = n * batch;
    if (total <= 0) return hipSuccess;
    noise_sample_kernel<T><<<grid_for(total), BLOCK, 0, stream>>>(w, u, scale, out, n, total);
    return hipGetLastError();
}

template <typename S, typename D>
hipError_t convert_async(const S* src, D* dst, int64_t n, hipStream_t stream)
{
    if (n <= 0) return hipSuccess;
    convert_kernel<S, D><<<grid_for(n), BLOCK, 0, stream>>>(src, dst, n);
    return hipGetLastError();
}

template hipError_t convert_async<_Float16, float>(const _Float16*, float*, int64_t, hipStream_t);
template hipError_t convert_async<__bf16, float>(const __bf16*, float*, int64_t, hipStream_t);
template hipError_t convert_async<float, _Float16>(const float*, _Float16*, int64_t, hipStream_t);
template hipError_t convert_async<float, __bf16>(const float*, __bf16*, int64_t, hipStream_t);
template hipError_t noise_sample_async<float>(const float*, const float*, float, float*, int64_t, int64_t, hipStream_t);
template hipError_t noise_sample_async<double>(const double*, const double*, double, double*, int64_t, int64_t, hipStream_t);
template hipError_t round_async<float>(const double*, float*, int64_t, hipStream_t);
template hipError_t round_async<double>(const double*, double*, int64_t, hipStream_t);
template hipError_t accumulate_async<float>(double*, const float*, int64_t, bool, hipStream_t);
template hipError_t accumulate_async<double>(double*, const double*, int64_t, bool, hipStream_t);
template hipError_t round_async<_Float16>(const double*, _Float16*, int64_t, hipStream_t);
template hipError_t round_async<__bf16>(const double*, __bf16*, int64_t, hipStream_t);
template hipError_t fill_async<float>(float*, int64_t, float, hipStream_t);
template hipError_t fill_async<double>(double*, int64_t, double, hipStream_t);
template hipError_t fill_async<_Float16>(_Float16*, int64_t, _Float16, hipStream_t);
template hipError_t fill_async<__bf16>(__bf16*, int64_t, __bf16, hipStream_t);
template hipError_t fill_async<int32_t>(int32_t*, int64_t, int32_t, hipStream_t);
template size_t reduce_slots_scratch<float>(int, int64_t);
template size_t reduce_slots_scratch<double>(int, int64_t);
template hipError_t reduce_slots_async<float>(const float*, int, int64_t, float*, float*, hipStream_t);
template hipError_t reduce_slots_async<double>(const double*, int, int64_t, double*, double*, hipStream_t);

}  // namespace mca
