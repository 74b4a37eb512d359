// Host-side launchers of the HIP kernels (morpho_fwd.hip, morpho_bwd.hip, smorph.hip, util.hip),
// called by the C ABI (capi.cpp). Arguments are assumed validated by the caller; every launch is
// asynchronous on `stream`.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "common.hpp"

namespace mca
{

// Workspace bytes are rounded to this alignment for every sub-buffer.
constexpr size_t WS_ALIGN = 256;

inline size_t align_up(size_t v) { return (v + WS_ALIGN - 1) / WS_ALIGN * WS_ALIGN; }

// Rows of outputs each wave computes in the generic (runtime structuring element) kernels.
template <typename T>
constexpr int rows_per_wave()
{
    return sizeof(T) == 8 ? 4 : 8;
}

// LDS the tuned launch plans budget for one workgroup (bytes): what leaves room for two or more
// workgroups per CU. A plan exceeds it only for elements that fit nothing smaller.
constexpr size_t LDS_LIMIT = 64 * 1024;

// LDS one workgroup may allocate on the current device (bytes): the device's per-workgroup maximum
// (hipDeviceAttributeMaxSharedMemoryPerBlock, queried once per device). A launch needing more cannot
// run; the entry points reject such elements with an error.
size_t device_lds_limit();

// Saved winners of the forward pass ("indices"):
//   MAX / MIN merges: int32 (channel << 16) | tap per output pixel, [B, Cout, H, W];
//   ADD / AVERAGE / IDENTITY: the first extremal tap of every channel pair, [B, Cout, Cpair, H, W]
//   with Cpair = Cin (1 for IDENTITY), one byte per entry (two when KH * KW > 256).
inline bool packed_winners(int merge) { return merge == MERGE_MAX || merge == MERGE_MIN; }

inline size_t pair_tap_bytes(const Geom& g) { return g.taps() > 256 ? 2 : 1; }

inline size_t indices_bytes(int merge, const Geom& g)
{
    const size_t pix = (size_t)g.B * g.Cout * g.plane();
    if (packed_winners(merge)) return pix * sizeof(int32_t);
    const size_t cpair = merge == MERGE_IDENTITY ? 1 : (size_t)g.Cin;
    return pix * cpair * pair_tap_bytes(g);
}

// ST: the storage type of x, w and out (float, double, _Float16 or __bf16); the fill value is in its
// compute type (compute_t).
template <typename ST>
hipError_t morpho_forward(int op, int merge, bool replicate, compute_t<ST> fill, const ST* x, const ST* w, ST* out, void* indices,
                          const Geom& g, hipStream_t stream);

// Bytes of LDS the forward kernel needs; more than device_lds_limit() means the structuring element is
// too large.
template <typename ST>
size_t morpho_forward_lds(const Geom& g);

// ST: the storage type, as for morpho_forward. Float16 and bfloat16 gradients are routed by the
// float32 kernels (grad_output converted in, grad_input and grad_weight rounded out, in the workspace).
template <typename ST>
size_t morpho_backward_workspace(int merge, bool has_indices, const Geom& g);

template <typename ST>
size_t morpho_backward_lds(int merge, const Geom& g);

template <typename ST>
hipError_t morpho_backward(int op, int merge, bool replicate, compute_t<ST> fill, const ST* x, const ST* w, const void* indices,
                           const ST* grad_out, ST* grad_in, ST* grad_w, const Geom& g, void* workspace, size_t workspace_bytes,
                           hipStream_t stream);

// Values in each of the three arrays of saved smorph pair statistics (float32 static kernels only;
// 0 when the configuration has none).
int64_t smorph_stats_values(int merge, const Geom& g);
// Whether the configuration has the saved-statistics path (float32 static sizes), empty or not.
bool smorph_stats_supported(const Geom& g);

// `stats`: where to save the pair statistics (three arrays of smorph_stats_values values), or null.
template <typename T>
hipError_t smorph_forward(int merge, const T* x, const T* w, const T* alpha, T* out, const Geom& g, hipStream_t stream,
                          float* stats = nullptr);

template <typename T>
size_t smorph_lds(int merge, const Geom& g, bool backward);

template <typename T>
size_t smorph_backward_workspace(int merge, const Geom& g);

// `stats`: the pair statistics the forward saved, or null (recomputed).
template <typename T>
hipError_t smorph_backward(int merge, const T* x, const T* w, const T* alpha, const T* out, const T* grad_out, T* grad_in, T* grad_w,
                           T* grad_alpha, const Geom& g, void* workspace, size_t workspace_bytes, hipStream_t stream,
                           const float* stats = nullptr);

// Smorph with the SMOOTH channel merge (smorph_scm; generic kernels, float32 and float64).
// Forward workspace: every pair output, [B, Cout, Cin, H, W]. `sstats` (2 * B * Cout * H * W values:
// the soft merge's ref, then 1 / sum), written by the forward (may be null) and read by the backward.
// `pstats`: the pair statistics (as smorph_forward's `stats`, smorph_stats_count(MERGE_SMOOTH) values
// per array; float32 static configurations only), saved by the forward, whose pair outputs are then
// the W / S array (no workspace), and read by the backward; null: the backward recomputes them.
template <typename T>
size_t smorph_scm_forward_workspace(const Geom& g);
template <typename T>
size_t smorph_scm_backward_workspace(const Geom& g);
template <typename T>
size_t smorph_scm_lds(const Geom& g, bool backward);
template <typename T>
hipError_t smorph_scm_forward(const T* x, const T* w, const T* alpha, const T* beta, T* out, T* sstats, const Geom& g, void* workspace,
                              size_t workspace_bytes, hipStream_t stream, float* pstats = nullptr);
template <typename T>
hipError_t smorph_scm_backward(const T* x, const T* w, const T* alpha, const T* beta, const T* out, const T* sstats, const T* grad_out,
                               T* grad_in, T* grad_w, T* grad_alpha, T* grad_beta, const Geom& g, void* workspace, size_t workspace_bytes,
                               hipStream_t stream, const float* pstats = nullptr);

// Streaming kernels of the IDENTITY merge for 3x3 / 5x5 elements over bands of whole rows
// (morpho_ident.hip). ident_bands: R rows per band (0: the shape has no such kernels: planes whose
// width is not a multiple of 8, other elements, or bands too wide for the LDS), the bands per plane
// and one workgroup's LDS (elem_bytes: the gradients' storage type for the backward).
struct IdentBands
{
    int R, nbands;
    size_t lds;
};
IdentBands ident_bands(const Geom& g, size_t elem_bytes, bool backward);
// Forward (float / double): out and, when taps is not null, the first extremal tap of every pixel.
// Pointers 16-byte aligned (taps: 8-byte).
template <typename ST>
hipError_t ident_band_forward(int op, bool replicate, ST fill, const ST* x, const ST* w, ST* out, uint8_t* taps, const Geom& g,
                              hipStream_t stream);
// Backward from the saved taps: grad_input, and grad_weight's sums per (batch element, band) in
// part ([B * nbands][Cout][KH * KW], T: double for double storage, else float).
template <typename T, typename ST>
hipError_t ident_band_backward(int op, const uint8_t* taps, const ST* grad_out, ST* grad_in, T* part, const Geom& g, hipStream_t stream);

// Opening / closing with IDENTITY merges fused into one pass (morpho_fused.hip). g: Cin == Cout == C,
// Cw == 1; first_op: the first stage's op.
bool morpho_pair_supported(const Geom& g);
template <typename T>
hipError_t morpho_pair_forward(int first_op, bool replicate, T fill1, T fill2, const T* x, const T* w1, const T* w2, T* out, uint8_t* taps1,
                               uint8_t* taps2, const Geom& g, hipStream_t stream);
template <typename T>
size_t morpho_pair_backward_workspace(const Geom& g);
template <typename T>
hipError_t morpho_pair_backward(int first_op, const uint8_t* taps1, const uint8_t* taps2, const T* grad_out, T* grad_in, T* grad_w1,
                                T* grad_w2, const Geom& g, void* workspace, size_t workspace_bytes, hipStream_t stream);

// sigma_layer with the IDENTITY merge in one pass (morpho_fused.hip): out = erosion (1 - soft) + dilation
// soft per channel; we / wd as each operator receives its element (the erosion's flipped). fill: the
// border value both operations read. The backward writes grad_in, both elements' gradients and
// grad_terms [2][C] (sum of g * erosion, sum of g * dilation per channel).
template <typename T>
hipError_t morpho_sigma_forward(bool replicate, T fill, const T* x, const T* we, const T* wd, const T* soft, T* out, uint8_t* tapse,
                                uint8_t* tapsd, const Geom& g, hipStream_t stream);
template <typename T>
size_t morpho_sigma_backward_workspace(const Geom& g);
template <typename T>
hipError_t morpho_sigma_backward(bool replicate, T fill, const T* x, const T* we, const T* wd, const T* soft, const uint8_t* tapse,
                                 const uint8_t* tapsd, const T* grad_out, T* grad_in, T* grad_we, T* grad_wd, T* grad_terms, const Geom& g,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream);

// The smorph kernels' exponential applied elementwise (test probe).
template <typename T>
hipError_t exp_probe(const T* x, T* y, int64_t n, hipStream_t stream);

// Per-sample elements of weight noise from uniform draws u [batch, n]: w + (u * 2 - 1) * scale with the
// roundings of torch's four elementwise operations (util.hip).
template <typename T>
hipError_t noise_sample_async(const T* w, const T* u, T scale, T* out, int64_t n, int64_t batch, hipStream_t stream);

// dst = src converted between a 16-bit storage type and float32 (util.hip).
template <typename S, typename D>
hipError_t convert_async(const S* src, D* dst, int64_t n, hipStream_t stream);

// The output of a merge over no input channel (Cin == 0, a merge other than IDENTITY): the merge's
// start value, finalised, as the reference's merge over no channel (morpho_merge_policy.hpp:10-86):
// lowest() for MAX, max() for MIN, 0 for ADD and 0 / 0 (NaN) for AVERAGE. The kernels, which read the
// input channels, are not launched for it; every saved winner is then (channel 0, tap 0).
template <typename T>
inline T empty_merge_value(int merge)
{
    using C = compute_t<T>;
    if (merge == MERGE_MAX) return (T)std::numeric_limits<C>::lowest();
    if (merge == MERGE_MIN) return (T)std::numeric_limits<C>::max();
    if (merge == MERGE_AVERAGE) return (T)std::numeric_limits<C>::quiet_NaN();
    return T(0);
}

// Records `msg` as the calling thread's last error (mca_last_error) and returns MCA_ERR_INVALID
// (capi.cpp).
int api_fail(const char* msg);
// MCA_OK for hipSuccess; otherwise records the HIP error's text and returns MCA_ERR_HIP (capi.cpp).
int api_hip_status(hipError_t err);

// Shared helpers (util.hip).
template <typename T>
hipError_t fill_async(T* p, int64_t n, T v, hipStream_t stream);
template <typename T>
hipError_t round_async(const double* src, T* dst, int64_t n, hipStream_t stream);
// acc[j] = (first ? 0 : acc[j]) + part[j], in double.
template <typename T>
hipError_t accumulate_async(double* acc, const T* part, int64_t n, bool first, hipStream_t stream);

// Slots summed per group by the first stage of a long reduction.
constexpr int REDUCE_GROUP = 32;

// Scratch bytes reduce_slots_async needs for nslots partial slots of n values.
template <typename T>
size_t reduce_slots_scratch(int nslots, int64_t n);

// out[j] = sum of part[s * n + j] over the slots s, in a fixed order (deterministic).
template <typename T>
hipError_t reduce_slots_async(const T* part, int nslots, int64_t n, T* out, T* scratch, hipStream_t stream);

}  // namespace mca
