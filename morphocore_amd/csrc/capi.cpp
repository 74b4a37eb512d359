// C ABI of the morphocore_amd kernels: argument validation with the reference's messages, then the
// asynchronous launchers of morpho_fwd.hip / morpho_bwd.hip / smorph.hip. Declarations:
// include/morphocore_amd.h.
#include "../../include/morphocore_amd.h"

#include <limits>
#include <mutex>
#include <string>

#include "launch.hpp"

// Device scratch of mca_morpho_backward_noalloc_f32, the backward for callers that cannot allocate
// device memory. Each GPU holds its own copy (MCA_NOALLOC_SCRATCH_BYTES) from the first call on it
// until the process ends. In host code `scratch` only names the symbol: its device address on the
// current GPU comes from hipGetSymbolAddress (noalloc_scratch below), and only that address is
// handed to kernels and fills.
static __device__ __align__(256) unsigned char scratch[MCA_NOALLOC_SCRATCH_BYTES];

namespace
{

thread_local std::string g_last_error;

int fail(const std::string& msg)
{
    g_last_error = msg;
    return MCA_ERR_INVALID;
}

int hip_status(hipError_t err)
{
    if (err == hipSuccess) return MCA_OK;
    g_last_error = std::string("HIP error: ") + hipGetErrorString(err);
    return MCA_ERR_HIP;
}

bool fits_int(int64_t v) { return v >= 0 && v <= 0x7fffffff; }

// Geometry checks shared by every entry point; fills `g`. Returns MCA_OK or an error.
int make_geom(int merge, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, int64_t wbs,
              mca::Geom& g)
{
    if (merge < 0 || merge > mca::MERGE_IDENTITY) return fail("Unknown merge mode " + std::to_string(merge));
    if (merge == mca::MERGE_SMOOTH) return fail("Unsupported merge operation");
    if (!fits_int(B) || !fits_int(Cin) || !fits_int(Cout) || !fits_int(Cw) || !fits_int(H) || !fits_int(W) || !fits_int(KH) || !fits_int(KW))
        return fail("Tensor dimensions must be non negative and below 2^31");
    if (KH < 1 || KW < 1) return fail("The structuring element must have at least one tap");
    // The kernels address a pixel within its plane with 32-bit offsets.
    if (H * W > 0x7fffffff) return fail("Image planes of more than 2^31 - 1 pixels are not supported");
    if (merge == mca::MERGE_IDENTITY)
    {
        if (Cout != Cin) return fail("Identity mode requires weight.shape[0] == input.shape[1]");
        if (Cw != 1) return fail("Identity mode requires weight.shape[1] == 1");
    }
    else if (Cw != Cin)
    {
        return fail("Input channels must match weight input channels");
    }
    if (wbs < 0) return fail("weight_batch_stride must be non negative");
    // Workgroup counts of the launches: tiles x channels x batch must fit a 1-D grid.
    const int64_t tiles = ((W + mca::TILE_W - 1) / mca::TILE_W) * ((H + 15) / 16);
    if (B * tiles * (Cout > Cin ? Cout : Cin) > 0x7fffffff) return fail("Problem too large for one launch");
    g.B = (int)B;
    g.Cin = (int)Cin;
    g.Cout = (int)Cout;
    g.Cw = (int)Cw;
    g.H = (int)H;
    g.W = (int)W;
    g.KH = (int)KH;
    g.KW = (int)KW;
    g.wbs = wbs;
    return MCA_OK;
}

int check_lds(size_t bytes)
{
    if (bytes > mca::device_lds_limit()) return fail("Structuring element too large for the kernels' shared memory");
    return MCA_OK;
}

template <typename T>
int morpho_forward_impl(int op, int merge, int replicate, mca::compute_t<T> fill, const T* input, const T* weight, int64_t wbs, T* output,
                        void* indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW,
                        void* stream)
{
    mca::Geom g{};
    if (op != mca::DILATION && op != mca::EROSION) return fail("Unknown morphological operation " + std::to_string(op));
    int rc = make_geom(merge, B, Cin, Cout, Cw, H, W, KH, KW, wbs, g);
    if (rc != MCA_OK) return rc;
    if (indices && mca::packed_winners(merge) && !(KH * KW < (1 << 16) && Cin < (1 << 15)))
        return fail("Structuring element or channel count too large to save indices");
    if ((rc = check_lds(mca::morpho_forward_lds<T>(g))) != MCA_OK) return rc;
    return hip_status(mca::morpho_forward<T>(op, merge, replicate != 0, fill, input, weight, output, indices, g, (hipStream_t)stream));
}

template <typename T>
size_t morpho_workspace_impl(int merge, int has_indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W,
                             int64_t KH, int64_t KW)
{
    mca::Geom g{};
    if (make_geom(merge, B, Cin, Cout, Cw, H, W, KH, KW, 0, g) != MCA_OK) return 0;
    return mca::morpho_backward_workspace<T>(merge, has_indices != 0, g);
}

template <typename T>
int morpho_backward_impl(int op, int merge, int replicate, mca::compute_t<T> fill, const T* input, const T* weight, int64_t wbs, const void* indices,
                         const T* grad_output, T* grad_input, T* grad_weight, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H,
                         int64_t W, int64_t KH, int64_t KW, void* workspace, size_t workspace_bytes, void* stream)
{
    mca::Geom g{};
    if (op != mca::DILATION && op != mca::EROSION) return fail("Unknown morphological operation " + std::to_string(op));
    int rc = make_geom(merge, B, Cin, Cout, Cw, H, W, KH, KW, wbs, g);
    if (rc != MCA_OK) return rc;
    if (mca::packed_winners(merge) && !(KH * KW < (1 << 16) && Cin < (1 << 15)))
        return fail("Structuring element or channel count too large to save indices");
    if ((rc = check_lds(mca::morpho_backward_lds<T>(merge, g))) != MCA_OK) return rc;
    if (!indices && (rc = check_lds(mca::morpho_forward_lds<T>(g))) != MCA_OK) return rc;
    const size_t need = mca::morpho_backward_workspace<T>(merge, indices != nullptr, g);
    if (workspace_bytes < need || (need > 0 && !workspace))
        return fail("Workspace too small: " + std::to_string(workspace_bytes) + " bytes given, " + std::to_string(need) + " needed");
    return hip_status(mca::morpho_backward<T>(op, merge, replicate != 0, fill, input, weight, indices, grad_output, grad_input, grad_weight,
                                              g, workspace, workspace_bytes, (hipStream_t)stream));
}

template <typename T>
int smorph_forward_impl(int merge, const T* input, const T* weight, const T* alpha, T* output, int64_t B, int64_t Cin, int64_t Cout,
                        int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream, float* stats = nullptr)
{
    mca::Geom g{};
    int rc = make_geom(merge, B, Cin, Cout, Cw, H, W, KH, KW, 0, g);
    if (rc != MCA_OK) return rc;
    if ((rc = check_lds(mca::smorph_lds<T>(merge, g, false))) != MCA_OK) return rc;
    return hip_status(mca::smorph_forward<T>(merge, input, weight, alpha, output, g, (hipStream_t)stream, stats));
}

// Checks of the saved-statistics entry points: the configuration has them and a buffer is given.
int check_stats(int merge, const mca::Geom& g, const void* stats)
{
    if (!mca::smorph_stats_supported(g))
        return fail("No saved smorph statistics for this configuration (float32, square 3x3, 5x5, 7x7 or 11x11 elements only)");
    if (!stats && mca::smorph_stats_values(merge, g) > 0) return fail("stats must not be null");
    return MCA_OK;
}

template <typename T>
size_t smorph_workspace_impl(int merge, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    mca::Geom g{};
    if (make_geom(merge, B, Cin, Cout, Cw, H, W, KH, KW, 0, g) != MCA_OK) return 0;
    if (mca::smorph_lds<T>(merge, g, true) > mca::device_lds_limit()) return 0;  // no backward for this element
    return mca::smorph_backward_workspace<T>(merge, g);
}

template <typename T>
int smorph_backward_impl(int merge, const T* input, const T* weight, const T* alpha, const T* output, const T* grad_output, T* grad_input,
                         T* grad_weight, T* grad_alpha, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                         int64_t KW, void* workspace, size_t workspace_bytes, void* stream, const float* stats = nullptr)
{
    mca::Geom g{};
    int rc = make_geom(merge, B, Cin, Cout, Cw, H, W, KH, KW, 0, g);
    if (rc != MCA_OK) return rc;
    if ((rc = check_lds(mca::smorph_lds<T>(merge, g, true))) != MCA_OK) return rc;
    const size_t need = mca::smorph_backward_workspace<T>(merge, g);
    if (workspace_bytes < need || (need > 0 && !workspace))
        return fail("Workspace too small: " + std::to_string(workspace_bytes) + " bytes given, " + std::to_string(need) + " needed");
    return hip_status(mca::smorph_backward<T>(merge, input, weight, alpha, output, grad_output, grad_input, grad_weight, grad_alpha, g,
                                              workspace, workspace_bytes, (hipStream_t)stream, stats));
}

// Geometry of the SMOOTH merge entry points: the checks of every smorph entry point with a per-pair
// alpha (Cw == Cin), and at least one input channel to merge.
int make_scm_geom(int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, mca::Geom& g)
{
    const int rc = make_geom(mca::MERGE_ADD, B, Cin, Cout, Cw, H, W, KH, KW, 0, g);
    if (rc != MCA_OK) return rc;
    if (Cin < 1) return fail("smorph_scm needs at least one input channel");
    return MCA_OK;
}

template <typename T>
size_t scm_forward_workspace_impl(int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    mca::Geom g{};
    if (make_scm_geom(B, Cin, Cout, Cw, H, W, KH, KW, g) != MCA_OK) return 0;
    return mca::smorph_scm_forward_workspace<T>(g);
}

template <typename T>
size_t scm_backward_workspace_impl(int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    mca::Geom g{};
    if (make_scm_geom(B, Cin, Cout, Cw, H, W, KH, KW, g) != MCA_OK) return 0;
    if (mca::smorph_scm_lds<T>(g, true) > mca::device_lds_limit()) return 0;
    return mca::smorph_scm_backward_workspace<T>(g);
}

int check_workspace(size_t given, size_t need, const void* workspace)
{
    if (given < need || (need > 0 && !workspace))
        return fail("Workspace too small: " + std::to_string(given) + " bytes given, " + std::to_string(need) + " needed");
    return MCA_OK;
}

// `pair_stats` (float32 only, checked by the callers): the pair statistics saved by the forward (no
// workspace then) and read by the backward, or null.
template <typename T>
int scm_forward_impl(const T* input, const T* weight, const T* alpha, const T* beta, T* output, T* merge_stats, int64_t B, int64_t Cin,
                     int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* workspace, size_t workspace_bytes,
                     void* stream, float* pair_stats = nullptr)
{
    mca::Geom g{};
    int rc = make_scm_geom(B, Cin, Cout, Cw, H, W, KH, KW, g);
    if (rc != MCA_OK) return rc;
    if ((rc = check_lds(mca::smorph_scm_lds<T>(g, false))) != MCA_OK) return rc;
    if (!pair_stats && (rc = check_workspace(workspace_bytes, mca::smorph_scm_forward_workspace<T>(g), workspace)) != MCA_OK) return rc;
    return hip_status(mca::smorph_scm_forward<T>(input, weight, alpha, beta, output, merge_stats, g, workspace, workspace_bytes,
                                                 (hipStream_t)stream, pair_stats));
}

template <typename T>
int scm_backward_impl(const T* input, const T* weight, const T* alpha, const T* beta, const T* output, const T* merge_stats,
                      const T* grad_output, T* grad_input, T* grad_weight, T* grad_alpha, T* grad_beta, int64_t B, int64_t Cin, int64_t Cout,
                      int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* workspace, size_t workspace_bytes, void* stream,
                      const float* pair_stats = nullptr)
{
    mca::Geom g{};
    int rc = make_scm_geom(B, Cin, Cout, Cw, H, W, KH, KW, g);
    if (rc != MCA_OK) return rc;
    if ((rc = check_lds(mca::smorph_scm_lds<T>(g, true))) != MCA_OK) return rc;
    if (!merge_stats && (int64_t)g.B * g.Cout * g.plane() > 0) return fail("merge_stats must not be null");
    if ((rc = check_workspace(workspace_bytes, mca::smorph_scm_backward_workspace<T>(g), workspace)) != MCA_OK) return rc;
    return hip_status(mca::smorph_scm_backward<T>(input, weight, alpha, beta, output, merge_stats, grad_output, grad_input, grad_weight,
                                                  grad_alpha, grad_beta, g, workspace, workspace_bytes, (hipStream_t)stream, pair_stats));
}

// Device address of `scratch` on `device` (which must be the current device), looked up once per
// device and kept.
constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_noalloc_mutex;
void* g_noalloc_ptr[NOALLOC_MAX_DEVICES];

// Geometry of the fused opening / closing entry points: C channels, identity merges, a supported
// square element.
int make_pair_geom(int first_op, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW, int64_t wbs, mca::Geom& g)
{
    if (first_op != mca::DILATION && first_op != mca::EROSION) return fail("Unknown morphological operation " + std::to_string(first_op));
    int rc = make_geom(mca::MERGE_IDENTITY, B, C, C, 1, H, W, KH, KW, wbs, g);
    if (rc != MCA_OK) return rc;
    if (!mca::morpho_pair_supported(g)) return fail("The fused opening / closing takes square 3x3, 5x5 or 7x7 structuring elements");
    // Its tiles are 64 - (K - 1) columns by 16 rows.
    if (B * C * ((W + mca::TILE_W - KW) / (mca::TILE_W - KW + 1)) * ((H + 15) / 16) > 0x7fffffff) return fail("Problem too large for one launch");
    return MCA_OK;
}

template <typename T>
int pair_forward_impl(int first_op, int replicate, T fill1, T fill2, const T* input, const T* w1, const T* w2, int64_t wbs, T* output,
                      uint8_t* taps1, uint8_t* taps2, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream)
{
    mca::Geom g{};
    int rc = make_pair_geom(first_op, B, C, H, W, KH, KW, wbs, g);
    if (rc != MCA_OK) return rc;
    if ((taps1 == nullptr) != (taps2 == nullptr)) return fail("taps_first and taps_second must both be given or both be NULL");
    return hip_status(mca::morpho_pair_forward<T>(first_op, replicate != 0, fill1, fill2, input, w1, w2, output, taps1, taps2, g,
                                                  (hipStream_t)stream));
}

template <typename T>
size_t pair_workspace_impl(int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    mca::Geom g{};
    if (make_pair_geom(mca::EROSION, B, C, H, W, KH, KW, 0, g) != MCA_OK) return 0;
    return mca::morpho_pair_backward_workspace<T>(g);
}

template <typename T>
int pair_backward_impl(int first_op, const uint8_t* taps1, const uint8_t* taps2, const T* grad_output, T* grad_input, T* grad_w1,
                       T* grad_w2, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW, void* workspace,
                       size_t workspace_bytes, void* stream)
{
    mca::Geom g{};
    int rc = make_pair_geom(first_op, B, C, H, W, KH, KW, 0, g);
    if (rc != MCA_OK) return rc;
    if ((!taps1 || !taps2) && B * C * H * W > 0) return fail("The fused opening / closing backward needs both stages' saved taps");
    const size_t need = mca::morpho_pair_backward_workspace<T>(g);
    if ((rc = check_workspace(workspace_bytes, need, workspace)) != MCA_OK) return rc;
    return hip_status(mca::morpho_pair_backward<T>(first_op, taps1, taps2, grad_output, grad_input, grad_w1, grad_w2, g, workspace,
                                                   workspace_bytes, (hipStream_t)stream));
}

// The one border value both operations of the fused sigma_layer read: their common fill, or, for the
// geodesic pair (+inf for the erosion, -inf for the dilation), NaN, which neither operation ever
// picks, as it never picks its own geodesic fill.
template <typename T>
int sigma_fill(int replicate, T fill_e, T fill_d, T& fill)
{
    if (replicate || fill_e == fill_d)
    {
        fill = fill_e;
        return MCA_OK;
    }
    if (fill_e == std::numeric_limits<T>::infinity() && fill_d == -std::numeric_limits<T>::infinity())
    {
        fill = std::numeric_limits<T>::quiet_NaN();
        return MCA_OK;
    }
    return fail("The fused sigma_layer needs one border value for both operations (or the geodesic pair +inf / -inf)");
}

template <typename T>
int sigma_forward_impl(int replicate, T fill_e, T fill_d, const T* input, const T* we, const T* wd, int64_t wbs, const T* soft, T* output,
                       uint8_t* tapse, uint8_t* tapsd, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream)
{
    mca::Geom g{};
    int rc = make_pair_geom(mca::EROSION, B, C, H, W, KH, KW, wbs, g);
    if (rc != MCA_OK) return rc;
    if ((tapse == nullptr) != (tapsd == nullptr)) return fail("taps_erosion and taps_dilation must both be given or both be NULL");
    T fill{};
    if ((rc = sigma_fill<T>(replicate, fill_e, fill_d, fill)) != MCA_OK) return rc;
    return hip_status(mca::morpho_sigma_forward<T>(replicate != 0, fill, input, we, wd, soft, output, tapse, tapsd, g, (hipStream_t)stream));
}

template <typename T>
size_t sigma_workspace_impl(int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    mca::Geom g{};
    if (make_pair_geom(mca::EROSION, B, C, H, W, KH, KW, 0, g) != MCA_OK) return 0;
    return mca::morpho_sigma_backward_workspace<T>(g);
}

template <typename T>
int sigma_backward_impl(int replicate, T fill_e, T fill_d, const T* input, const T* we, const T* wd, int64_t wbs, const T* soft,
                        const uint8_t* tapse, const uint8_t* tapsd, const T* grad_output, T* grad_input, T* grad_we, T* grad_wd, T* grad_terms,
                        int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW, void* workspace, size_t workspace_bytes,
                        void* stream)
{
    mca::Geom g{};
    int rc = make_pair_geom(mca::EROSION, B, C, H, W, KH, KW, wbs, g);
    if (rc != MCA_OK) return rc;
    if ((!tapse || !tapsd) && B * C * H * W > 0) return fail("The fused sigma_layer backward needs both operations' saved taps");
    T fill{};
    if ((rc = sigma_fill<T>(replicate, fill_e, fill_d, fill)) != MCA_OK) return rc;
    if ((rc = check_workspace(workspace_bytes, mca::morpho_sigma_backward_workspace<T>(g), workspace)) != MCA_OK) return rc;
    return hip_status(mca::morpho_sigma_backward<T>(replicate != 0, fill, input, we, wd, soft, tapse, tapsd, grad_output, grad_input, grad_we,
                                                    grad_wd, grad_terms, g, workspace, workspace_bytes, (hipStream_t)stream));
}

int noalloc_scratch(int device, void** out)
{
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) return fail("Device index out of range for the no-allocation scratch");
    std::lock_guard<std::mutex> lock(g_noalloc_mutex);
    if (!g_noalloc_ptr[device])
    {
        void* p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return hip_status(err);
        if (!p) return fail("hipGetSymbolAddress returned a null address for the no-allocation scratch");
        g_noalloc_ptr[device] = p;
    }
    *out = g_noalloc_ptr[device];
    return MCA_OK;
}

}  // namespace

namespace mca
{
// Error reporting of the entry points, for the other translation units of the C ABI (stack.cpp).
int api_fail(const char* msg) { return fail(msg); }
int api_hip_status(hipError_t err) { return hip_status(err); }
}  // namespace mca

extern "C" {

const char* mca_version(void) { return "0.13.1-mi355x"; }

const char* mca_last_error(void) { return g_last_error.c_str(); }

size_t mca_morpho_indices_bytes(int merge, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    mca::Geom g{};
    if (make_geom(merge, B, Cin, Cout, Cw, H, W, KH, KW, 0, g) != MCA_OK) return 0;
    return mca::indices_bytes(merge, g);
}

int mca_morpho_forward_f32(int op, int merge, int replicate, float fill, const float* input, const float* weight,
                           int64_t weight_batch_stride, float* output, void* indices, int64_t B, int64_t Cin, int64_t Cout,
                           int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream)
{
    return morpho_forward_impl<float>(op, merge, replicate, fill, input, weight, weight_batch_stride, output, indices, B, Cin, Cout, Cw,
                                      H, W, KH, KW, stream);
}

int mca_morpho_forward_f64(int op, int merge, int replicate, double fill, const double* input, const double* weight,
                           int64_t weight_batch_stride, double* output, void* indices, int64_t B, int64_t Cin, int64_t Cout,
                           int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream)
{
    return morpho_forward_impl<double>(op, merge, replicate, fill, input, weight, weight_batch_stride, output, indices, B, Cin, Cout,
                                       Cw, H, W, KH, KW, stream);
}

size_t mca_morpho_backward_workspace_size_f32(int merge, int has_indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H,
                                              int64_t W, int64_t KH, int64_t KW)
{
    return morpho_workspace_impl<float>(merge, has_indices, B, Cin, Cout, Cw, H, W, KH, KW);
}

size_t mca_morpho_backward_workspace_size_f64(int merge, int has_indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H,
                                              int64_t W, int64_t KH, int64_t KW)
{
    return morpho_workspace_impl<double>(merge, has_indices, B, Cin, Cout, Cw, H, W, KH, KW);
}

int mca_morpho_backward_f32(int op, int merge, int replicate, float fill, const float* input, const float* weight,
                            int64_t weight_batch_stride, const void* indices, const float* grad_output, float* grad_input,
                            float* grad_weight, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                            int64_t KW, void* workspace, size_t workspace_bytes, void* stream)
{
    return morpho_backward_impl<float>(op, merge, replicate, fill, input, weight, weight_batch_stride, indices, grad_output, grad_input,
                                       grad_weight, B, Cin, Cout, Cw, H, W, KH, KW, workspace, workspace_bytes, stream);
}

int mca_morpho_backward_f64(int op, int merge, int replicate, double fill, const double* input, const double* weight,
                            int64_t weight_batch_stride, const void* indices, const double* grad_output, double* grad_input,
                            double* grad_weight, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                            int64_t KW, void* workspace, size_t workspace_bytes, void* stream)
{
    return morpho_backward_impl<double>(op, merge, replicate, fill, input, weight, weight_batch_stride, indices, grad_output, grad_input,
                                        grad_weight, B, Cin, Cout, Cw, H, W, KH, KW, workspace, workspace_bytes, stream);
}

int mca_morpho_forward_f16(int op, int merge, int replicate, float fill, const uint16_t* input, const uint16_t* weight,
                           int64_t weight_batch_stride, uint16_t* output, void* indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw,
                           int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream)
{
    return morpho_forward_impl<_Float16>(op, merge, replicate, fill, reinterpret_cast<const _Float16*>(input),
                                         reinterpret_cast<const _Float16*>(weight), weight_batch_stride, reinterpret_cast<_Float16*>(output),
                                         indices, B, Cin, Cout, Cw, H, W, KH, KW, stream);
}

int mca_morpho_forward_bf16(int op, int merge, int replicate, float fill, const uint16_t* input, const uint16_t* weight,
                            int64_t weight_batch_stride, uint16_t* output, void* indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw,
                            int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream)
{
    return morpho_forward_impl<__bf16>(op, merge, replicate, fill, reinterpret_cast<const __bf16*>(input),
                                       reinterpret_cast<const __bf16*>(weight), weight_batch_stride, reinterpret_cast<__bf16*>(output),
                                       indices, B, Cin, Cout, Cw, H, W, KH, KW, stream);
}

size_t mca_morpho_backward_workspace_size_f16(int merge, int has_indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H,
                                              int64_t W, int64_t KH, int64_t KW)
{
    return morpho_workspace_impl<_Float16>(merge, has_indices, B, Cin, Cout, Cw, H, W, KH, KW);
}

size_t mca_morpho_backward_workspace_size_bf16(int merge, int has_indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H,
                                               int64_t W, int64_t KH, int64_t KW)
{
    return morpho_workspace_impl<__bf16>(merge, has_indices, B, Cin, Cout, Cw, H, W, KH, KW);
}

int mca_morpho_backward_f16(int op, int merge, int replicate, float fill, const uint16_t* input, const uint16_t* weight,
                            int64_t weight_batch_stride, const void* indices, const uint16_t* grad_output, uint16_t* grad_input,
                            uint16_t* grad_weight, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                            int64_t KW, void* workspace, size_t workspace_bytes, void* stream)
{
    return morpho_backward_impl<_Float16>(op, merge, replicate, fill, reinterpret_cast<const _Float16*>(input),
                                          reinterpret_cast<const _Float16*>(weight), weight_batch_stride, indices,
                                          reinterpret_cast<const _Float16*>(grad_output), reinterpret_cast<_Float16*>(grad_input),
                                          reinterpret_cast<_Float16*>(grad_weight), B, Cin, Cout, Cw, H, W, KH, KW, workspace,
                                          workspace_bytes, stream);
}

int mca_morpho_backward_bf16(int op, int merge, int replicate, float fill, const uint16_t* input, const uint16_t* weight,
                             int64_t weight_batch_stride, const void* indices, const uint16_t* grad_output, uint16_t* grad_input,
                             uint16_t* grad_weight, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                             int64_t KW, void* workspace, size_t workspace_bytes, void* stream)
{
    return morpho_backward_impl<__bf16>(op, merge, replicate, fill, reinterpret_cast<const __bf16*>(input),
                                        reinterpret_cast<const __bf16*>(weight), weight_batch_stride, indices,
                                        reinterpret_cast<const __bf16*>(grad_output), reinterpret_cast<__bf16*>(grad_input),
                                        reinterpret_cast<__bf16*>(grad_weight), B, Cin, Cout, Cw, H, W, KH, KW, workspace, workspace_bytes,
                                        stream);
}

int mca_morpho_backward_noalloc_f32(int op, int merge, int replicate, float fill, const float* input, const float* weight,
                                    int64_t weight_batch_stride, const void* indices, const float* grad_output, float* grad_input,
                                    float* grad_weight, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W,
                                    int64_t KH, int64_t KW, void* stream)
{
    mca::Geom g{};
    if (op != mca::DILATION && op != mca::EROSION) return fail("Unknown morphological operation " + std::to_string(op));
    int rc = make_geom(merge, B, Cin, Cout, Cw, H, W, KH, KW, weight_batch_stride, g);
    if (rc != MCA_OK) return rc;
    if (mca::packed_winners(merge) && !(KH * KW < (1 << 16) && Cin < (1 << 15)))
        return fail("Structuring element or channel count too large to save indices");
    const size_t need = mca::morpho_backward_workspace<float>(merge, indices != nullptr, g);
    if (need > (size_t)MCA_NOALLOC_SCRATCH_BYTES)
        return fail("Problem too large for the no-allocation backward: it needs " + std::to_string(need) + " bytes of scratch, the limit is " +
                    std::to_string((size_t)MCA_NOALLOC_SCRATCH_BYTES) + " (use mca_morpho_backward_f32 with a workspace)");
    // The scratch belongs to the current device: the stream must run there.
    int device = -1;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) return hip_status(err);
    hipDevice_t stream_device = device;
    if ((err = hipStreamGetDevice((hipStream_t)stream, &stream_device)) != hipSuccess) return hip_status(err);
    if ((int)stream_device != device)
        return fail("The stream belongs to device " + std::to_string((int)stream_device) + " but device " + std::to_string(device) +
                    " is current");
    void* ptr = nullptr;
    if ((rc = noalloc_scratch(device, &ptr)) != MCA_OK) return rc;
    return morpho_backward_impl<float>(op, merge, replicate, fill, input, weight, weight_batch_stride, indices, grad_output, grad_input,
                                       grad_weight, B, Cin, Cout, Cw, H, W, KH, KW, ptr, (size_t)MCA_NOALLOC_SCRATCH_BYTES, stream);
}

int mca_smorph_forward_f32(int merge, const float* input, const float* weight, const float* alpha, float* output, int64_t B, int64_t Cin,
                           int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream)
{
    return smorph_forward_impl<float>(merge, input, weight, alpha, output, B, Cin, Cout, Cw, H, W, KH, KW, stream);
}

int mca_smorph_forward_f64(int merge, const double* input, const double* weight, const double* alpha, double* output, int64_t B,
                           int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream)
{
    return smorph_forward_impl<double>(merge, input, weight, alpha, output, B, Cin, Cout, Cw, H, W, KH, KW, stream);
}

size_t mca_smorph_backward_workspace_size_f32(int merge, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W,
                                              int64_t KH, int64_t KW)
{
    return smorph_workspace_impl<float>(merge, B, Cin, Cout, Cw, H, W, KH, KW);
}

size_t mca_smorph_backward_workspace_size_f64(int merge, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W,
                                              int64_t KH, int64_t KW)
{
    return smorph_workspace_impl<double>(merge, B, Cin, Cout, Cw, H, W, KH, KW);
}

int mca_smorph_backward_f32(int merge, const float* input, const float* weight, const float* alpha, const float* output,
                            const float* grad_output, float* grad_input, float* grad_weight, float* grad_alpha, int64_t B, int64_t Cin,
                            int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* workspace,
                            size_t workspace_bytes, void* stream)
{
    return smorph_backward_impl<float>(merge, input, weight, alpha, output, grad_output, grad_input, grad_weight, grad_alpha, B, Cin, Cout,
                                       Cw, H, W, KH, KW, workspace, workspace_bytes, stream);
}

int mca_smorph_backward_f64(int merge, const double* input, const double* weight, const double* alpha, const double* output,
                            const double* grad_output, double* grad_input, double* grad_weight, double* grad_alpha, int64_t B,
                            int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* workspace,
                            size_t workspace_bytes, void* stream)
{
    return smorph_backward_impl<double>(merge, input, weight, alpha, output, grad_output, grad_input, grad_weight, grad_alpha, B, Cin,
                                        Cout, Cw, H, W, KH, KW, workspace, workspace_bytes, stream);
}

size_t mca_smorph_stats_bytes_f32(int merge, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    mca::Geom g{};
    if (make_geom(merge, B, Cin, Cout, Cw, H, W, KH, KW, 0, g) != MCA_OK) return 0;
    return (size_t)mca::smorph_stats_values(merge, g) * 3 * sizeof(float);
}

int mca_smorph_forward_stats_f32(int merge, const float* input, const float* weight, const float* alpha, float* output, float* stats,
                                 int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW,
                                 void* stream)
{
    mca::Geom g{};
    int rc = make_geom(merge, B, Cin, Cout, Cw, H, W, KH, KW, 0, g);
    if (rc != MCA_OK) return rc;
    if ((rc = check_stats(merge, g, stats)) != MCA_OK) return rc;
    return smorph_forward_impl<float>(merge, input, weight, alpha, output, B, Cin, Cout, Cw, H, W, KH, KW, stream, stats);
}

int mca_smorph_backward_stats_f32(int merge, const float* input, const float* weight, const float* alpha, const float* output,
                                  const float* stats, const float* grad_output, float* grad_input, float* grad_weight, float* grad_alpha,
                                  int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW,
                                  void* workspace, size_t workspace_bytes, void* stream)
{
    mca::Geom g{};
    int rc = make_geom(merge, B, Cin, Cout, Cw, H, W, KH, KW, 0, g);
    if (rc != MCA_OK) return rc;
    if ((rc = check_stats(merge, g, stats)) != MCA_OK) return rc;
    return smorph_backward_impl<float>(merge, input, weight, alpha, output, grad_output, grad_input, grad_weight, grad_alpha, B, Cin, Cout,
                                       Cw, H, W, KH, KW, workspace, workspace_bytes, stream, stats);
}

size_t mca_smorph_scm_forward_workspace_size_f32(int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                                                 int64_t KW)
{
    return scm_forward_workspace_impl<float>(B, Cin, Cout, Cw, H, W, KH, KW);
}

size_t mca_smorph_scm_forward_workspace_size_f64(int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                                                 int64_t KW)
{
    return scm_forward_workspace_impl<double>(B, Cin, Cout, Cw, H, W, KH, KW);
}

int mca_smorph_scm_forward_f32(const float* input, const float* weight, const float* alpha, const float* beta, float* output,
                               float* merge_stats, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                               int64_t KW, void* workspace, size_t workspace_bytes, void* stream)
{
    return scm_forward_impl<float>(input, weight, alpha, beta, output, merge_stats, B, Cin, Cout, Cw, H, W, KH, KW, workspace,
                                   workspace_bytes, stream);
}

int mca_smorph_scm_forward_f64(const double* input, const double* weight, const double* alpha, const double* beta, double* output,
                               double* merge_stats, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                               int64_t KW, void* workspace, size_t workspace_bytes, void* stream)
{
    return scm_forward_impl<double>(input, weight, alpha, beta, output, merge_stats, B, Cin, Cout, Cw, H, W, KH, KW, workspace,
                                    workspace_bytes, stream);
}

size_t mca_smorph_scm_backward_workspace_size_f32(int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                                                  int64_t KW)
{
    return scm_backward_workspace_impl<float>(B, Cin, Cout, Cw, H, W, KH, KW);
}

size_t mca_smorph_scm_backward_workspace_size_f64(int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                                                  int64_t KW)
{
    return scm_backward_workspace_impl<double>(B, Cin, Cout, Cw, H, W, KH, KW);
}

int mca_smorph_scm_backward_f32(const float* input, const float* weight, const float* alpha, const float* beta, const float* output,
                                const float* merge_stats, const float* grad_output, float* grad_input, float* grad_weight, float* grad_alpha,
                                float* grad_beta, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                                int64_t KW, void* workspace, size_t workspace_bytes, void* stream)
{
    return scm_backward_impl<float>(input, weight, alpha, beta, output, merge_stats, grad_output, grad_input, grad_weight, grad_alpha,
                                    grad_beta, B, Cin, Cout, Cw, H, W, KH, KW, workspace, workspace_bytes, stream);
}

int mca_smorph_scm_backward_f64(const double* input, const double* weight, const double* alpha, const double* beta, const double* output,
                                const double* merge_stats, const double* grad_output, double* grad_input, double* grad_weight,
                                double* grad_alpha, double* grad_beta, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H,
                                int64_t W, int64_t KH, int64_t KW, void* workspace, size_t workspace_bytes, void* stream)
{
    return scm_backward_impl<double>(input, weight, alpha, beta, output, merge_stats, grad_output, grad_input, grad_weight, grad_alpha,
                                     grad_beta, B, Cin, Cout, Cw, H, W, KH, KW, workspace, workspace_bytes, stream);
}

size_t mca_smorph_scm_stats_bytes_f32(int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    mca::Geom g{};
    if (make_scm_geom(B, Cin, Cout, Cw, H, W, KH, KW, g) != MCA_OK) return 0;
    return (size_t)mca::smorph_stats_values(mca::MERGE_SMOOTH, g) * 3 * sizeof(float);
}

int mca_smorph_scm_forward_stats_f32(const float* input, const float* weight, const float* alpha, const float* beta, float* output,
                                     float* merge_stats, float* pair_stats, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H,
                                     int64_t W, int64_t KH, int64_t KW, void* stream)
{
    mca::Geom g{};
    int rc = make_scm_geom(B, Cin, Cout, Cw, H, W, KH, KW, g);
    if (rc != MCA_OK) return rc;
    if ((rc = check_stats(mca::MERGE_SMOOTH, g, pair_stats)) != MCA_OK) return rc;
    // An empty output has no statistics (a null pair_stats is allowed): nothing to compute.
    if (!pair_stats) return MCA_OK;
    return scm_forward_impl<float>(input, weight, alpha, beta, output, merge_stats, B, Cin, Cout, Cw, H, W, KH, KW, nullptr, 0, stream,
                                   pair_stats);
}

int mca_smorph_scm_backward_stats_f32(const float* input, const float* weight, const float* alpha, const float* beta, const float* output,
                                      const float* merge_stats, const float* pair_stats, const float* grad_output, float* grad_input,
                                      float* grad_weight, float* grad_alpha, float* grad_beta, int64_t B, int64_t Cin, int64_t Cout,
                                      int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* workspace, size_t workspace_bytes,
                                      void* stream)
{
    mca::Geom g{};
    int rc = make_scm_geom(B, Cin, Cout, Cw, H, W, KH, KW, g);
    if (rc != MCA_OK) return rc;
    if ((rc = check_stats(mca::MERGE_SMOOTH, g, pair_stats)) != MCA_OK) return rc;
    // An empty output (null pair_stats): the recomputing path, which only clears the gradients.
    return scm_backward_impl<float>(input, weight, alpha, beta, output, merge_stats, grad_output, grad_input, grad_weight, grad_alpha,
                                    grad_beta, B, Cin, Cout, Cw, H, W, KH, KW, workspace, workspace_bytes, stream, pair_stats);
}

int mca_noise_sample_weights_f32(const float* weight, const float* uniform, float scale, float* out, int64_t batch, int64_t n, void* stream)
{
    if (batch < 0 || n < 0) return fail("batch and n must be non negative");
    return hip_status(mca::noise_sample_async<float>(weight, uniform, scale, out, n, batch, (hipStream_t)stream));
}

int mca_noise_sample_weights_f64(const double* weight, const double* uniform, double scale, double* out, int64_t batch, int64_t n,
                                 void* stream)
{
    if (batch < 0 || n < 0) return fail("batch and n must be non negative");
    return hip_status(mca::noise_sample_async<double>(weight, uniform, scale, out, n, batch, (hipStream_t)stream));
}

int mca_morpho_pair_supported(int64_t KH, int64_t KW)
{
    mca::Geom g{};
    g.KH = (int)(KH > 0 && KH < 64 ? KH : 0);
    g.KW = (int)(KW > 0 && KW < 64 ? KW : 0);
    return mca::morpho_pair_supported(g) ? 1 : 0;
}

int mca_morpho_pair_forward_f32(int first_op, int replicate, float fill_first, float fill_second, const float* input, const float* w_first,
                                const float* w_second, int64_t weight_batch_stride, float* output, uint8_t* taps_first,
                                uint8_t* taps_second, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream)
{
    return pair_forward_impl<float>(first_op, replicate, fill_first, fill_second, input, w_first, w_second, weight_batch_stride, output,
                                    taps_first, taps_second, B, C, H, W, KH, KW, stream);
}

int mca_morpho_pair_forward_f64(int first_op, int replicate, double fill_first, double fill_second, const double* input,
                                const double* w_first, const double* w_second, int64_t weight_batch_stride, double* output,
                                uint8_t* taps_first, uint8_t* taps_second, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH,
                                int64_t KW, void* stream)
{
    return pair_forward_impl<double>(first_op, replicate, fill_first, fill_second, input, w_first, w_second, weight_batch_stride, output,
                                     taps_first, taps_second, B, C, H, W, KH, KW, stream);
}

size_t mca_morpho_pair_backward_workspace_size_f32(int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    return pair_workspace_impl<float>(B, C, H, W, KH, KW);
}

size_t mca_morpho_pair_backward_workspace_size_f64(int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    return pair_workspace_impl<double>(B, C, H, W, KH, KW);
}

int mca_morpho_pair_backward_f32(int first_op, const uint8_t* taps_first, const uint8_t* taps_second, const float* grad_output,
                                 float* grad_input, float* grad_w_first, float* grad_w_second, int64_t B, int64_t C, int64_t H, int64_t W,
                                 int64_t KH, int64_t KW, void* workspace, size_t workspace_bytes, void* stream)
{
    return pair_backward_impl<float>(first_op, taps_first, taps_second, grad_output, grad_input, grad_w_first, grad_w_second, B, C, H, W,
                                     KH, KW, workspace, workspace_bytes, stream);
}

int mca_morpho_pair_backward_f64(int first_op, const uint8_t* taps_first, const uint8_t* taps_second, const double* grad_output,
                                 double* grad_input, double* grad_w_first, double* grad_w_second, int64_t B, int64_t C, int64_t H,
                                 int64_t W, int64_t KH, int64_t KW, void* workspace, size_t workspace_bytes, void* stream)
{
    return pair_backward_impl<double>(first_op, taps_first, taps_second, grad_output, grad_input, grad_w_first, grad_w_second, B, C, H,
                                      W, KH, KW, workspace, workspace_bytes, stream);
}

int mca_morpho_sigma_forward_f32(int replicate, float fill_erosion, float fill_dilation, const float* input, const float* w_erosion,
                                 const float* w_dilation, int64_t weight_batch_stride, const float* soft, float* output,
                                 uint8_t* taps_erosion, uint8_t* taps_dilation, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH,
                                 int64_t KW, void* stream)
{
    return sigma_forward_impl<float>(replicate, fill_erosion, fill_dilation, input, w_erosion, w_dilation, weight_batch_stride, soft, output,
                                     taps_erosion, taps_dilation, B, C, H, W, KH, KW, stream);
}

int mca_morpho_sigma_forward_f64(int replicate, double fill_erosion, double fill_dilation, const double* input, const double* w_erosion,
                                 const double* w_dilation, int64_t weight_batch_stride, const double* soft, double* output,
                                 uint8_t* taps_erosion, uint8_t* taps_dilation, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH,
                                 int64_t KW, void* stream)
{
    return sigma_forward_impl<double>(replicate, fill_erosion, fill_dilation, input, w_erosion, w_dilation, weight_batch_stride, soft,
                                      output, taps_erosion, taps_dilation, B, C, H, W, KH, KW, stream);
}

size_t mca_morpho_sigma_backward_workspace_size_f32(int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    return sigma_workspace_impl<float>(B, C, H, W, KH, KW);
}

size_t mca_morpho_sigma_backward_workspace_size_f64(int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    return sigma_workspace_impl<double>(B, C, H, W, KH, KW);
}

int mca_morpho_sigma_backward_f32(int replicate, float fill_erosion, float fill_dilation, const float* input, const float* w_erosion,
                                  const float* w_dilation, int64_t weight_batch_stride, const float* soft, const uint8_t* taps_erosion,
                                  const uint8_t* taps_dilation, const float* grad_output, float* grad_input, float* grad_w_erosion,
                                  float* grad_w_dilation, float* grad_terms, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH,
                                  int64_t KW, void* workspace, size_t workspace_bytes, void* stream)
{
    return sigma_backward_impl<float>(replicate, fill_erosion, fill_dilation, input, w_erosion, w_dilation, weight_batch_stride, soft,
                                      taps_erosion, taps_dilation, grad_output, grad_input, grad_w_erosion, grad_w_dilation, grad_terms, B, C,
                                      H, W, KH, KW, workspace, workspace_bytes, stream);
}

int mca_morpho_sigma_backward_f64(int replicate, double fill_erosion, double fill_dilation, const double* input, const double* w_erosion,
                                  const double* w_dilation, int64_t weight_batch_stride, const double* soft, const uint8_t* taps_erosion,
                                  const uint8_t* taps_dilation, const double* grad_output, double* grad_input, double* grad_w_erosion,
                                  double* grad_w_dilation, double* grad_terms, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH,
                                  int64_t KW, void* workspace, size_t workspace_bytes, void* stream)
{
    return sigma_backward_impl<double>(replicate, fill_erosion, fill_dilation, input, w_erosion, w_dilation, weight_batch_stride, soft,
                                       taps_erosion, taps_dilation, grad_output, grad_input, grad_w_erosion, grad_w_dilation, grad_terms, B,
                                       C, H, W, KH, KW, workspace, workspace_bytes, stream);
}

int mca_probe_smorph_exp_f32(const float* x, float* y, int64_t n, void* stream)
{
    if (n < 0) return fail("n must be non negative");
    return hip_status(mca::exp_probe<float>(x, y, n, (hipStream_t)stream));
}

int mca_probe_smorph_exp_f64(const double* x, double* y, int64_t n, void* stream)
{
    if (n < 0) return fail("n must be non negative");
    return hip_status(mca::exp_probe<double>(x, y, n, (hipStream_t)stream));
}

}  // extern "C"
