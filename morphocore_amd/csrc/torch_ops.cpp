// PyTorch-ROCm extension morphocore_amd._C: registers torch.ops.morphocore.{dilation, erosion, smorph,
// smorph_scm} with the reference's schemas and dispatch key (plus opening_closing and sigma_identity,
// fused forms of the reference's Python opening / closing and sigma_layer), and implements them as C++ autograd
// Functions whose device work is the C ABI of libmorphocore_amd.so (include/morphocore_amd.h).
//
// This is the MI355X counterpart of the reference's host layer: bindings.cpp:15-156 (int checks,
// registration, empty Python module), morpho_op_wrap.hxx:24-211 (MorphoOperation forward / backward:
// rank handling, weight noise, the save-indices rule, saved state), smorph.cpp:20-111 and
// smorph_scm.cpp:13-96 (Smorph / SmorphSCM forward / backward, alpha pairs, the shared-alpha gradient
// sum), reshaper.cpp:3-151 (2-D / 3-D / 4-D ranks). Checks run in the reference's order with its
// messages. Tensors on another device than a HIP GPU are refused: there is no CPU path.
//
// Two extensions of the reference's saved state, neither of which changes a result:
//   * dilation / erosion with merge sum / mean / identity keep each channel pair's first extremal tap
//     (one byte per pair and output pixel) up to MORPHOCORE_AMD_SAVED_TAPS_LIMIT bytes per call
//     (default 8 GiB), so that the backward only routes;
//   * float32 smorph with a 3x3 / 5x5 / 7x7 / 11x11 element keeps each pair's window extremum, 1 / S
//     and W / S (12 bytes per pair and output pixel) under a budget shared by every live saved buffer
//     of the process (SavedStats below), so that the backward need not recompute them.
#include <Python.h>
#include <torch/all.h>
#include <torch/library.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPCachingAllocator.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>

#include <cstdlib>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/morphocore_amd.h"

namespace
{

using torch::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::tensor_list;

// Same integer values as the reference (morpho_op_enum.hpp:17-35, merge_enum.py:4-19).
enum Op : int64_t
{
    DILATION = 0,
    EROSION = 1
};
enum Merge : int64_t
{
    MAX = 0,
    MIN = 1,
    ADD = 2,
    AVERAGE = 3,
    SMOOTH = 4,
    IDENTITY = 5
};
enum Padding : int64_t
{
    ZERO = 0,
    GEODESIC = 1,
    CONSTANT = 2,
    REPLICATE = 3
};

// Max / min winners are saved only while the reference's CUDA grid could address every (batch,
// output channel) pair (morpho_op_wrap.hxx:65-66).
constexpr int64_t MAX_GRID_DIM = 65535;

int64_t env_bytes(const char* name, int64_t fallback)
{
    const char* v = std::getenv(name);
    if (!v || !*v) return fallback;
    return std::strtoll(v, nullptr, 10);
}

// bindings.cpp:16-20.
int64_t to_merge(int64_t merge)
{
    TORCH_CHECK(merge >= 0 && merge <= IDENTITY, "Unknown merge mode ", merge);
    return merge;
}

// bindings.cpp:23-27.
int64_t to_padding(int64_t padding)
{
    TORCH_CHECK(padding >= 0 && padding <= REPLICATE, "Unknown padding mode ", padding);
    return padding;
}

// Border value of the fill paddings (morpho_padding_policy.hpp:22-33): ZERO 0, CONSTANT the value,
// GEODESIC the identity element of the operation. REPLICATE reads the clamped edge pixel instead.
double fill_value(int64_t op, int64_t padding, double padding_value)
{
    switch (padding)
    {
        case CONSTANT: return padding_value;
        case GEODESIC: return op == DILATION ? -std::numeric_limits<double>::infinity() : std::numeric_limits<double>::infinity();
        default: return 0.0;
    }
}

// TensorInputDim::To4DTensor (reshaper.cpp:3-55): [H, W] and [C, H, W] gain leading unit axes.
Tensor input_to_4d(const Tensor& t)
{
    const int64_t d = t.dim();
    if (d == 4) return t;
    if (d == 3) return t.unsqueeze(0);
    if (d == 2) return t.unsqueeze(0).unsqueeze(0);
    TORCH_CHECK(false, "Invalid input tensor: please give a 2D, 3D or 4D input tensor, received: ", d, " dimensions !");
    return t;
}

// TensorInputDim::ToOriginalTensor (reshaper.cpp:57-81).
Tensor output_to_original(const Tensor& out, int64_t input_dims)
{
    if (input_dims == 3) return out.squeeze(0);
    if (input_dims == 2) return out.squeeze(0).squeeze(0);
    return out;
}

// TensorWeightDim::To4DTensor (reshaper.cpp:84-130): a [KH, KW] weight is one channel pair.
Tensor weight_to_4d(const Tensor& t)
{
    const int64_t d = t.dim();
    if (d == 4) return t;
    if (d == 2) return t.unsqueeze(0).unsqueeze(0);
    TORCH_CHECK(false, "Invalid weight tensor dimensions: expected 2D, 3D, 4D or 5D tensor, received ", d, "D tensor");
    return t;
}

void check_4d(const Tensor& x4, const Tensor& w4)
{
    TORCH_CHECK(x4.dim() == 4, "Input must be a 4d tensor (batch_size, in_channels, height, width)");
    TORCH_CHECK(w4.dim() == 4, "Weight must be a 4d tensor (out_channels, in_channels, kernel_height, kernel_width)");
}

void check_identity(const Tensor& x4, const Tensor& w4, bool smorph)
{
    TORCH_CHECK(w4.size(0) == x4.size(1), "Identity mode requires weight.shape[0] == input.shape[1]");
    if (smorph)
    {
        TORCH_CHECK(w4.size(1) == 1, "Identity mode requires weight.shape[1] == 1, got ", w4.size(1));
    }
    else
    {
        TORCH_CHECK(w4.size(1) == 1, "Identity mode requires weight.shape[1] == 1");
    }
}

const char* scalar_name(c10::ScalarType t)
{
    switch (t)
    {
        case c10::kFloat: return "Float";
        case c10::kDouble: return "Double";
        case c10::kHalf: return "Half";
        case c10::kBFloat16: return "BFloat16";
        default: return c10::toString(t);
    }
}

// The operators run only on a HIP device, in float32 or float64 (dilation and erosion also in
// float16 and bfloat16); everything else is an error, never a fallback.
void check_device(const char* name, const Tensor& x4, std::initializer_list<Tensor> others, bool allow_16bit = false)
{
    TORCH_CHECK(x4.is_cuda(), "morphocore_amd: ", name, " runs on AMD GPUs (HIP devices); got an input on ", x4.device());
    const auto st = x4.scalar_type();
    TORCH_CHECK(st == c10::kFloat || st == c10::kDouble || (allow_16bit && (st == c10::kHalf || st == c10::kBFloat16)), "\"", name,
                "\" not implemented for '", scalar_name(st), "'");
    for (const Tensor& t : others)
    {
        TORCH_CHECK(t.device() == x4.device(), "morphocore_amd: ", name, " expects every tensor on ", x4.device(), ", got one on ", t.device());
        TORCH_CHECK(t.scalar_type() == x4.scalar_type(), "expected scalar type ", scalar_name(x4.scalar_type()), " but found ",
                    scalar_name(t.scalar_type()));
    }
}

void check_rc(int rc)
{
    TORCH_CHECK(rc == MCA_OK, mca_last_error());
}

// torch's current HIP stream of the tensor's device: the C ABI only enqueues work on it.
void* stream_of(const Tensor& t) { return (void*)c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

struct Geom
{
    int64_t B, Cin, Cout, Cw, H, W, KH, KW;
};

Geom geom_of(const Tensor& x4, const Tensor& w4)
{
    return Geom{x4.size(0), x4.size(1), w4.size(0), w4.size(1), x4.size(2), x4.size(3), w4.size(2), w4.size(3)};
}

// The 16-bit payload of a float16 / bfloat16 tensor, as the C ABI takes it.
uint16_t* bits16(const Tensor& t) { return reinterpret_cast<uint16_t*>(t.data_ptr()); }

Tensor byte_buffer(int64_t nbytes, const Tensor& like) { return torch::empty({nbytes > 0 ? nbytes : 1}, like.options().dtype(torch::kUInt8)); }

// ------------------------------------------------------------------------------------------------
// Saved smorph statistics: one budget for every live buffer of the process.
// ------------------------------------------------------------------------------------------------

// A buffer is admitted when the per-call cap allows it (MORPHOCORE_AMD_SAVED_STATS_LIMIT bytes; 0
// disables saving), when the buffers still alive plus this one stay within the process budget
// (MORPHOCORE_AMD_SAVED_STATS_BUDGET bytes, default 40% of the device's memory), and when it takes at
// most half of the memory still available to torch (free plus cached but unused), which leaves the
// other half to the activations of the layers that follow.
bool stats_policy(int64_t nbytes, int64_t live, int64_t budget, int64_t avail, int64_t limit)
{
    if (nbytes <= 0) return false;
    if (limit >= 0 && nbytes > limit) return false;
    if (live + nbytes > budget) return false;
    return nbytes <= avail / 2;
}

class SavedStats
{
public:
    static SavedStats& get()
    {
        static SavedStats s;
        return s;
    }

    // Bytes of saved-statistics buffers still alive on `device`.
    int64_t live_bytes(c10::DeviceIndex device)
    {
        std::lock_guard<std::mutex> lock(m_);
        return prune_and_sum(device);
    }

    bool admit(int64_t nbytes, c10::DeviceIndex device)
    {
        std::lock_guard<std::mutex> lock(m_);
        return admit_locked(nbytes, device);
    }

    // A float32 buffer of nbytes for the statistics when the policy admits it, tracked from then on;
    // an undefined tensor otherwise (also when the allocation fails: the backward then recomputes).
    // The check, the allocation and the tracking are one critical section, so that forwards running
    // in several threads cannot together exceed the budget.
    Tensor allocate(int64_t nbytes, const c10::TensorOptions& options)
    {
        const c10::DeviceIndex device = options.device().index();
        std::lock_guard<std::mutex> lock(m_);
        if (!admit_locked(nbytes, device)) return Tensor();
        Tensor t;
        try
        {
            t = torch::empty({nbytes / 4}, options.dtype(torch::kFloat32));
        }
        catch (const c10::OutOfMemoryError&)
        {
            return Tensor();  // fragmented memory
        }
        live_.push_back(Entry{t.storage().getWeakStorageImpl(), static_cast<int64_t>(t.nbytes()), device});
        return t;
    }

private:
    struct Entry
    {
        c10::weak_intrusive_ptr<c10::StorageImpl> storage;
        int64_t nbytes;
        c10::DeviceIndex device;
    };

    bool admit_locked(int64_t nbytes, c10::DeviceIndex device)
    {
        if (nbytes <= 0) return false;
        size_t free_b = 0, total_b = 0;
        {
            const c10::DeviceGuard guard(c10::Device(c10::kCUDA, device));
            if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) return false;
        }
        const auto stats = c10::hip::HIPCachingAllocator::getDeviceStats(device);
        const int64_t agg = static_cast<int64_t>(c10::CachingAllocator::StatType::AGGREGATE);
        const int64_t cached_unused = stats.reserved_bytes[agg].current - stats.allocated_bytes[agg].current;
        const int64_t avail = static_cast<int64_t>(free_b) + (cached_unused > 0 ? cached_unused : 0);
        const int64_t budget = env_bytes("MORPHOCORE_AMD_SAVED_STATS_BUDGET", static_cast<int64_t>(total_b) / 10 * 4);
        const int64_t limit = env_bytes("MORPHOCORE_AMD_SAVED_STATS_LIMIT", -1);
        return stats_policy(nbytes, prune_and_sum(device), budget, avail, limit);
    }

    int64_t prune_and_sum(c10::DeviceIndex device)
    {
        int64_t sum = 0;
        std::vector<Entry> keep;
        keep.reserve(live_.size());
        for (Entry& e : live_)
        {
            if (e.storage.expired()) continue;
            if (e.device == device) sum += e.nbytes;
            keep.push_back(std::move(e));
        }
        live_.swap(keep);
        return sum;
    }

    std::mutex m_;
    std::vector<Entry> live_;
};

// Weight noise: one structuring element per batch element, [B, *w.shape], from torch::rand's draw on the
// weight's device (its generator, the reference's draw, morpho_op_wrap.hxx:55-64), formed by one
// kernel with the roundings of the reference's four elementwise operations.
Tensor sample_weights(const Tensor& w, int64_t B, double noise_scale)
{
    std::vector<int64_t> shape = w.sizes().vec();
    shape.insert(shape.begin(), B);
    const Tensor u = torch::rand(shape, w.options());
    // 16-bit elements: the same expression in torch's own elementwise operations.
    if (w.scalar_type() == c10::kHalf || w.scalar_type() == c10::kBFloat16) return (w.unsqueeze(0) + (u * 2.0 - 1.0) * noise_scale).contiguous();
    Tensor out = torch::empty(shape, w.options());
    const int64_t n = w.numel();
    if (w.scalar_type() == c10::kFloat)
        check_rc(mca_noise_sample_weights_f32(w.data_ptr<float>(), u.data_ptr<float>(), (float)noise_scale, out.data_ptr<float>(), B, n,
                                              stream_of(w)));
    else
        check_rc(mca_noise_sample_weights_f64(w.data_ptr<double>(), u.data_ptr<double>(), noise_scale, out.data_ptr<double>(), B, n,
                                              stream_of(w)));
    return out;
}

// ------------------------------------------------------------------------------------------------
// Dilation and erosion: MorphoOperation<op, merge, kind> (morpho_op_wrap.hxx:24-211).
// ------------------------------------------------------------------------------------------------

class MorphoFunction : public torch::autograd::Function<MorphoFunction>
{
public:
    static Tensor forward(AutogradContext* ctx, const Tensor& x4, const Tensor& w4, int64_t op, int64_t merge, int64_t padding,
                          double padding_value, bool save_indices, double noise_scale, bool needs_grad)
    {
        const c10::DeviceGuard guard(x4.device());
        const Tensor x = x4.contiguous();
        const Tensor w = w4.contiguous();
        const Geom g = geom_of(x, w);
        // Weight noise: one structuring element per batch element, drawn on the weight's device from
        // its generator as morpho_op_wrap.hxx:55-64 draws it.
        Tensor sample_weight;
        if (noise_scale > 0.0) sample_weight = sample_weights(w, g.B, noise_scale);
        const Tensor& kw = sample_weight.defined() ? sample_weight : w;
        const int64_t wbs = sample_weight.defined() ? g.Cout * g.Cw * g.KH * g.KW : 0;
        const int64_t nbytes = (int64_t)mca_morpho_indices_bytes((int)merge, g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW);
        bool save = save_indices && needs_grad;
        if (save)
            save = (merge == MAX || merge == MIN) ? g.Cout * g.B < MAX_GRID_DIM
                                                  : nbytes <= env_bytes("MORPHOCORE_AMD_SAVED_TAPS_LIMIT", int64_t(8) << 30);
        Tensor out = torch::empty({g.B, g.Cout, g.H, g.W}, x.options());
        // Layout per mca_morpho_indices_bytes: packed int32 winners (max / min) or per-pair taps.
        Tensor indices = save ? byte_buffer(nbytes, x) : Tensor();
        const bool replicate = padding == REPLICATE;
        const double fill = fill_value(op, padding, padding_value);
        void* idx = indices.defined() ? indices.data_ptr() : nullptr;
        if (x.scalar_type() == c10::kFloat)
            check_rc(mca_morpho_forward_f32((int)op, (int)merge, replicate, (float)fill, x.data_ptr<float>(), kw.data_ptr<float>(), wbs,
                                            out.data_ptr<float>(), idx, g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW, stream_of(x)));
        else if (x.scalar_type() == c10::kHalf || x.scalar_type() == c10::kBFloat16)
            check_rc((x.scalar_type() == c10::kHalf ? mca_morpho_forward_f16 : mca_morpho_forward_bf16)(
                (int)op, (int)merge, replicate, (float)fill, bits16(x), bits16(kw), wbs, bits16(out), idx, g.B, g.Cin, g.Cout, g.Cw, g.H, g.W,
                g.KH, g.KW, stream_of(x)));
        else
            check_rc(mca_morpho_forward_f64((int)op, (int)merge, replicate, fill, x.data_ptr<double>(), kw.data_ptr<double>(), wbs,
                                            out.data_ptr<double>(), idx, g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW, stream_of(x)));
        ctx->save_for_backward({x, w, indices, sample_weight});
        ctx->saved_data["op"] = op;
        ctx->saved_data["merge"] = merge;
        ctx->saved_data["padding"] = padding;
        ctx->saved_data["padding_value"] = padding_value;
        return out;
    }

    static tensor_list backward(AutogradContext* ctx, tensor_list grad_outputs)
    {
        const auto saved = ctx->get_saved_variables();
        const Tensor& x = saved[0];
        const Tensor& w = saved[1];
        const Tensor& indices = saved[2];
        const Tensor& sample_weight = saved[3];
        const int64_t op = ctx->saved_data["op"].toInt();
        const int64_t merge = ctx->saved_data["merge"].toInt();
        const int64_t padding = ctx->saved_data["padding"].toInt();
        const double padding_value = ctx->saved_data["padding_value"].toDouble();
        const Tensor grad_output = grad_outputs[0].contiguous();
        std::vector<int64_t> expected = x.sizes().vec();
        expected[1] = w.size(0);
        TORCH_CHECK(grad_output.sizes() == expected, "grad_output shape mismatch: expected [", expected, "] but got [", grad_output.sizes(),
                    "]");
        TORCH_CHECK(grad_output.device() == x.device(), "grad_output must be on the same device as input");
        TORCH_CHECK(grad_output.scalar_type() == x.scalar_type(), "grad_output must have the same dtype as input");
        const c10::DeviceGuard guard(x.device());
        const Geom g = geom_of(x, w);
        // The noisy weights chose the winning taps; the weight gradient keeps the shared weight's shape.
        const Tensor& kw = sample_weight.defined() ? sample_weight : w;
        const int64_t wbs = sample_weight.defined() ? g.Cout * g.Cw * g.KH * g.KW : 0;
        Tensor grad_input = torch::empty_like(x);
        Tensor grad_weight = torch::empty_like(w);
        const bool replicate = padding == REPLICATE;
        const double fill = fill_value(op, padding, padding_value);
        const void* idx = indices.defined() ? indices.data_ptr() : nullptr;
        const int has = idx != nullptr;
        if (x.scalar_type() == c10::kHalf || x.scalar_type() == c10::kBFloat16)
        {
            const bool h = x.scalar_type() == c10::kHalf;
            const size_t n = (h ? mca_morpho_backward_workspace_size_f16 : mca_morpho_backward_workspace_size_bf16)(
                (int)merge, has, g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW);
            Tensor ws = byte_buffer((int64_t)n, x);
            check_rc((h ? mca_morpho_backward_f16 : mca_morpho_backward_bf16)((int)op, (int)merge, replicate, (float)fill, bits16(x), bits16(kw),
                                                                              wbs, idx, bits16(grad_output), bits16(grad_input),
                                                                              bits16(grad_weight), g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH,
                                                                              g.KW, ws.data_ptr(), (size_t)ws.numel(), stream_of(x)));
        }
        else if (x.scalar_type() == c10::kFloat)
        {
            const size_t n = mca_morpho_backward_workspace_size_f32((int)merge, has, g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW);
            Tensor ws = byte_buffer((int64_t)n, x);
            check_rc(mca_morpho_backward_f32((int)op, (int)merge, replicate, (float)fill, x.data_ptr<float>(), kw.data_ptr<float>(), wbs, idx,
                                             grad_output.data_ptr<float>(), grad_input.data_ptr<float>(), grad_weight.data_ptr<float>(), g.B,
                                             g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW, ws.data_ptr(), (size_t)ws.numel(), stream_of(x)));
        }
        else
        {
            const size_t n = mca_morpho_backward_workspace_size_f64((int)merge, has, g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW);
            Tensor ws = byte_buffer((int64_t)n, x);
            check_rc(mca_morpho_backward_f64((int)op, (int)merge, replicate, fill, x.data_ptr<double>(), kw.data_ptr<double>(), wbs, idx,
                                             grad_output.data_ptr<double>(), grad_input.data_ptr<double>(), grad_weight.data_ptr<double>(),
                                             g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW, ws.data_ptr(), (size_t)ws.numel(),
                                             stream_of(x)));
        }
        return {grad_input, grad_weight, Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

// Body of the dilation / erosion operators: bindings.cpp:59-101, then MorphoOperation::forward's
// checks (morpho_op_wrap.hxx:24-77).
Tensor morpho_operation(int64_t op, const Tensor& input, const Tensor& weight, int64_t merge, int64_t padding, double padding_value,
                        bool save_indices, double noise_scale)
{
    padding = to_padding(padding);
    merge = to_merge(merge);
    TORCH_CHECK(merge != SMOOTH, "Unsupported merge operation");
    TORCH_CHECK(noise_scale >= 0.0, "noise_scale must be non negative");
    const int64_t input_dims = input.dim();
    const Tensor x4 = input_to_4d(input);
    const Tensor w4 = weight_to_4d(weight);
    check_4d(x4, w4);
    TORCH_CHECK(x4.size(1) == w4.size(1) || merge == IDENTITY, "Input channels must match weight input channels");
    if (merge == IDENTITY) check_identity(x4, w4, false);
    check_device(op == DILATION ? "morpho_dilation_forward_hip" : "morpho_erosion_forward_hip", x4, {w4}, true);
    const bool needs_grad = torch::GradMode::is_enabled() && (input.requires_grad() || weight.requires_grad());
    const Tensor out = MorphoFunction::apply(x4, w4, op, merge, padding, padding_value, save_indices, noise_scale, needs_grad);
    return output_to_original(out, input_dims);
}

Tensor morpho_dilation(const Tensor& input, const Tensor& weight, int64_t merge, int64_t padding, double padding_value, bool save_indices,
                       double noise_scale)
{
    return morpho_operation(DILATION, input, weight, merge, padding, padding_value, save_indices, noise_scale);
}

Tensor morpho_erosion(const Tensor& input, const Tensor& weight, int64_t merge, int64_t padding, double padding_value, bool save_indices,
                      double noise_scale)
{
    return morpho_operation(EROSION, input, weight, merge, padding, padding_value, save_indices, noise_scale);
}

// ------------------------------------------------------------------------------------------------
// Opening / closing with per-channel merges in one pass. The reference composes them in Python from
// two operator calls (functional/opening.py:96-101, functional/closing.py:96-101); this operator
// computes the same output from one kernel and keeps each stage's taps (one byte per pixel each) for
// a backward that only routes.
// ------------------------------------------------------------------------------------------------

class PairFunction : public torch::autograd::Function<PairFunction>
{
public:
    static Tensor forward(AutogradContext* ctx, const Tensor& x4, const Tensor& w1_4, const Tensor& w2_4, int64_t first_op, int64_t padding,
                          double padding_value, double noise_scale, bool needs_grad)
    {
        const c10::DeviceGuard guard(x4.device());
        const Tensor x = x4.contiguous();
        const Tensor w1 = w1_4.contiguous();
        const Tensor w2 = w2_4.contiguous();
        const int64_t B = x.size(0), C = x.size(1), H = x.size(2), W = x.size(3), K = w1.size(2);
        // Weight noise: each stage draws its own, the first stage first, as the two operator calls of
        // the composition do (MorphoFunction above, morpho_op_wrap.hxx:55-64).
        Tensor s1, s2;
        if (noise_scale > 0.0)
        {
            s1 = sample_weights(w1, B, noise_scale);
            s2 = sample_weights(w2, B, noise_scale);
        }
        const Tensor& k1 = s1.defined() ? s1 : w1;
        const Tensor& k2 = s2.defined() ? s2 : w2;
        const int64_t wbs = s1.defined() ? C * K * K : 0;
        Tensor out = torch::empty_like(x);
        Tensor taps = needs_grad ? torch::empty({2, B, C, H, W}, x.options().dtype(torch::kUInt8)) : Tensor();
        uint8_t* t1 = taps.defined() ? taps.data_ptr<uint8_t>() : nullptr;
        uint8_t* t2 = taps.defined() ? t1 + B * C * H * W : nullptr;
        const int64_t op2 = first_op == DILATION ? EROSION : DILATION;
        const double f1 = fill_value(first_op, padding, padding_value), f2 = fill_value(op2, padding, padding_value);
        const int replicate = padding == REPLICATE;
        if (x.scalar_type() == c10::kFloat)
            check_rc(mca_morpho_pair_forward_f32((int)first_op, replicate, (float)f1, (float)f2, x.data_ptr<float>(), k1.data_ptr<float>(),
                                                 k2.data_ptr<float>(), wbs, out.data_ptr<float>(), t1, t2, B, C, H, W, K, K, stream_of(x)));
        else
            check_rc(mca_morpho_pair_forward_f64((int)first_op, replicate, f1, f2, x.data_ptr<double>(), k1.data_ptr<double>(),
                                                 k2.data_ptr<double>(), wbs, out.data_ptr<double>(), t1, t2, B, C, H, W, K, K, stream_of(x)));
        ctx->save_for_backward({taps, w1});
        ctx->saved_data["first_op"] = first_op;
        return out;
    }

    static tensor_list backward(AutogradContext* ctx, tensor_list grad_outputs)
    {
        const auto saved = ctx->get_saved_variables();
        const Tensor& taps = saved[0];
        const Tensor& w1 = saved[1];
        const int64_t first_op = ctx->saved_data["first_op"].toInt();
        TORCH_CHECK(taps.defined(), "opening_closing: the forward ran without gradients and kept no taps");
        const Tensor grad_output = grad_outputs[0].contiguous();
        std::vector<int64_t> expected = taps.sizes().vec();
        expected.erase(expected.begin());
        TORCH_CHECK(grad_output.sizes() == expected, "grad_output shape mismatch: expected [", expected, "] but got [", grad_output.sizes(),
                    "]");
        TORCH_CHECK(grad_output.device() == taps.device(), "grad_output must be on the same device as input");
        TORCH_CHECK(grad_output.scalar_type() == w1.scalar_type(), "grad_output must have the same dtype as input");
        const c10::DeviceGuard guard(taps.device());
        const int64_t B = expected[0], C = expected[1], H = expected[2], W = expected[3], K = w1.size(2);
        Tensor grad_input = torch::empty_like(grad_output);
        Tensor gw1 = torch::empty_like(w1);
        Tensor gw2 = torch::empty_like(w1);
        const uint8_t* t1 = taps.data_ptr<uint8_t>();
        const uint8_t* t2 = t1 + B * C * H * W;
        if (grad_output.scalar_type() == c10::kFloat)
        {
            Tensor ws = byte_buffer((int64_t)mca_morpho_pair_backward_workspace_size_f32(B, C, H, W, K, K), grad_output);
            check_rc(mca_morpho_pair_backward_f32((int)first_op, t1, t2, grad_output.data_ptr<float>(), grad_input.data_ptr<float>(),
                                                  gw1.data_ptr<float>(), gw2.data_ptr<float>(), B, C, H, W, K, K, ws.data_ptr(),
                                                  (size_t)ws.numel(), stream_of(grad_output)));
        }
        else
        {
            Tensor ws = byte_buffer((int64_t)mca_morpho_pair_backward_workspace_size_f64(B, C, H, W, K, K), grad_output);
            check_rc(mca_morpho_pair_backward_f64((int)first_op, t1, t2, grad_output.data_ptr<double>(), grad_input.data_ptr<double>(),
                                                  gw1.data_ptr<double>(), gw2.data_ptr<double>(), B, C, H, W, K, K, ws.data_ptr(),
                                                  (size_t)ws.numel(), stream_of(grad_output)));
        }
        return {grad_input, gw1, gw2, Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

// Opening (first_op erosion) or closing (first_op dilation) with 'identity' merges on both stages; the
// weights as the two operators receive them (an erosion's element flipped, functional/erosion.py:89).
// Square 3x3 / 5x5 / 7x7 elements of equal size run fused; any other size, and a backward whose taps
// would exceed MORPHOCORE_AMD_SAVED_TAPS_LIMIT or that save_indices=False asks to recompute, run the
// two operators one after the other, exactly as the composition does.
Tensor opening_closing(const Tensor& input, const Tensor& w_first, const Tensor& w_second, int64_t first_op, int64_t padding,
                       double padding_value, bool save_indices, double noise_scale)
{
    padding = to_padding(padding);
    TORCH_CHECK(first_op == DILATION || first_op == EROSION, "Unknown morphological operation ", first_op);
    TORCH_CHECK(noise_scale >= 0.0, "noise_scale must be non negative");
    const int64_t input_dims = input.dim();
    const Tensor x4 = input_to_4d(input);
    const Tensor w1 = weight_to_4d(w_first);
    const Tensor w2 = weight_to_4d(w_second);
    check_4d(x4, w1);
    check_4d(x4, w2);
    check_identity(x4, w1, false);
    check_identity(x4, w2, false);
    check_device("morpho_pair_forward_hip", x4, {w1, w2}, true);
    const bool needs_grad = torch::GradMode::is_enabled() && (input.requires_grad() || w_first.requires_grad() || w_second.requires_grad());
    const bool same = w1.size(2) == w2.size(2) && w1.size(3) == w2.size(3);
    const int64_t tap_bytes = 2 * x4.numel();
    const bool wide = x4.scalar_type() == c10::kFloat || x4.scalar_type() == c10::kDouble;  // the fused kernels' types
    const bool fused = wide && same && mca_morpho_pair_supported(w1.size(2), w1.size(3)) &&
                       (!needs_grad || (save_indices && tap_bytes <= env_bytes("MORPHOCORE_AMD_SAVED_TAPS_LIMIT", int64_t(8) << 30)));
    if (!fused)
    {
        const int64_t op2 = first_op == DILATION ? EROSION : DILATION;
        const Tensor mid = morpho_operation(first_op, x4, w1, IDENTITY, padding, padding_value, save_indices, noise_scale);
        return output_to_original(morpho_operation(op2, mid, w2, IDENTITY, padding, padding_value, save_indices, noise_scale), input_dims);
    }
    return output_to_original(PairFunction::apply(x4, w1, w2, first_op, padding, padding_value, noise_scale, needs_grad), input_dims);
}

// ------------------------------------------------------------------------------------------------
// sigma_layer with the 'identity' merge in one pass. The reference composes it in Python from two
// operator calls and a blend (functional/sigma_layer.py:73-83); this operator computes the same output
// in one kernel and keeps each operation's taps for a backward that only routes.
// ------------------------------------------------------------------------------------------------

class SigmaFunction : public torch::autograd::Function<SigmaFunction>
{
public:
    static Tensor forward(AutogradContext* ctx, const Tensor& x4, const Tensor& we4, const Tensor& wd4, const Tensor& soft_in, int64_t padding,
                          double padding_value, double noise_scale, bool needs_grad)
    {
        const c10::DeviceGuard guard(x4.device());
        const Tensor x = x4.contiguous();
        const Tensor we = we4.contiguous();
        const Tensor wd = wd4.contiguous();
        const Tensor soft = soft_in.contiguous().reshape({-1});
        const int64_t B = x.size(0), C = x.size(1), H = x.size(2), W = x.size(3), K = we.size(2);
        // Weight noise: the erosion's draw, then the dilation's, as the composition's two operator
        // calls draw them (MorphoFunction above, morpho_op_wrap.hxx:55-64).
        Tensor se, sd;
        if (noise_scale > 0.0)
        {
            se = sample_weights(we, B, noise_scale);
            sd = sample_weights(wd, B, noise_scale);
        }
        const Tensor& ke = se.defined() ? se : we;
        const Tensor& kd = sd.defined() ? sd : wd;
        const int64_t wbs = se.defined() ? C * K * K : 0;
        Tensor out = torch::empty_like(x);
        Tensor taps = needs_grad ? torch::empty({2, B, C, H, W}, x.options().dtype(torch::kUInt8)) : Tensor();
        uint8_t* te = taps.defined() ? taps.data_ptr<uint8_t>() : nullptr;
        uint8_t* td = taps.defined() ? te + B * C * H * W : nullptr;
        const double fe = fill_value(EROSION, padding, padding_value), fd = fill_value(DILATION, padding, padding_value);
        const int replicate = padding == REPLICATE;
        if (x.scalar_type() == c10::kFloat)
            check_rc(mca_morpho_sigma_forward_f32(replicate, (float)fe, (float)fd, x.data_ptr<float>(), ke.data_ptr<float>(), kd.data_ptr<float>(),
                                                  wbs, soft.data_ptr<float>(), out.data_ptr<float>(), te, td, B, C, H, W, K, K, stream_of(x)));
        else
            check_rc(mca_morpho_sigma_forward_f64(replicate, fe, fd, x.data_ptr<double>(), ke.data_ptr<double>(), kd.data_ptr<double>(), wbs,
                                                  soft.data_ptr<double>(), out.data_ptr<double>(), te, td, B, C, H, W, K, K, stream_of(x)));
        ctx->save_for_backward({x, ke, kd, soft, taps, we});
        ctx->saved_data["padding"] = padding;
        ctx->saved_data["padding_value"] = padding_value;
        ctx->saved_data["wbs"] = wbs;
        ctx->saved_data["soft_sizes"] = soft_in.sizes().vec();
        return out;
    }

    static tensor_list backward(AutogradContext* ctx, tensor_list grad_outputs)
    {
        const auto saved = ctx->get_saved_variables();
        const Tensor& x = saved[0];
        const Tensor& ke = saved[1];
        const Tensor& kd = saved[2];
        const Tensor& soft = saved[3];
        const Tensor& taps = saved[4];
        const Tensor& we = saved[5];
        TORCH_CHECK(taps.defined(), "sigma_identity: the forward ran without gradients and kept no taps");
        const int64_t padding = ctx->saved_data["padding"].toInt();
        const double padding_value = ctx->saved_data["padding_value"].toDouble();
        const int64_t wbs = ctx->saved_data["wbs"].toInt();
        const Tensor grad_output = grad_outputs[0].contiguous();
        TORCH_CHECK(grad_output.sizes() == x.sizes(), "grad_output shape mismatch: expected [", x.sizes(), "] but got [", grad_output.sizes(),
                    "]");
        TORCH_CHECK(grad_output.device() == x.device(), "grad_output must be on the same device as input");
        TORCH_CHECK(grad_output.scalar_type() == x.scalar_type(), "grad_output must have the same dtype as input");
        const c10::DeviceGuard guard(x.device());
        const int64_t B = x.size(0), C = x.size(1), H = x.size(2), W = x.size(3), K = we.size(2);
        Tensor grad_input = torch::empty_like(x);
        Tensor gwe = torch::empty_like(we);
        Tensor gwd = torch::empty_like(we);
        Tensor terms = torch::empty({2, C}, x.options());
        const uint8_t* te = taps.data_ptr<uint8_t>();
        const uint8_t* td = te + B * C * H * W;
        const double fe = fill_value(EROSION, padding, padding_value), fd = fill_value(DILATION, padding, padding_value);
        const int replicate = padding == REPLICATE;
        if (x.scalar_type() == c10::kFloat)
        {
            Tensor ws = byte_buffer((int64_t)mca_morpho_sigma_backward_workspace_size_f32(B, C, H, W, K, K), x);
            check_rc(mca_morpho_sigma_backward_f32(replicate, (float)fe, (float)fd, x.data_ptr<float>(), ke.data_ptr<float>(), kd.data_ptr<float>(),
                                                   wbs, soft.data_ptr<float>(), te, td, grad_output.data_ptr<float>(), grad_input.data_ptr<float>(),
                                                   gwe.data_ptr<float>(), gwd.data_ptr<float>(), terms.data_ptr<float>(), B, C, H, W, K, K,
                                                   ws.data_ptr(), (size_t)ws.numel(), stream_of(x)));
        }
        else
        {
            Tensor ws = byte_buffer((int64_t)mca_morpho_sigma_backward_workspace_size_f64(B, C, H, W, K, K), x);
            check_rc(mca_morpho_sigma_backward_f64(replicate, fe, fd, x.data_ptr<double>(), ke.data_ptr<double>(), kd.data_ptr<double>(), wbs,
                                                   soft.data_ptr<double>(), te, td, grad_output.data_ptr<double>(),
                                                   grad_input.data_ptr<double>(), gwe.data_ptr<double>(), gwd.data_ptr<double>(),
                                                   terms.data_ptr<double>(), B, C, H, W, K, K, ws.data_ptr(), (size_t)ws.numel(), stream_of(x)));
        }
        // d out / d soft = sum g * dilation - sum g * erosion (the blend's two products).
        const Tensor grad_soft = (terms[1] - terms[0]).reshape(ctx->saved_data["soft_sizes"].toIntVector());
        return {grad_input, gwe, gwd, grad_soft, Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

// sigma_layer with the 'identity' merge; the elements as the two operators receive them (the
// erosion's flipped, functional/erosion.py:89) and soft = sigmoid(mean(alpha)) per channel. Square
// 3x3 / 5x5 / 7x7 elements of equal size run fused; other sizes, and a backward whose taps would exceed
// MORPHOCORE_AMD_SAVED_TAPS_LIMIT or that save_indices=False asks to recompute, run the two operators
// and the blend as the composition does.
Tensor sigma_identity(const Tensor& input, const Tensor& w_erosion, const Tensor& w_dilation, const Tensor& soft, int64_t padding,
                      double padding_value, bool save_indices, double noise_scale)
{
    padding = to_padding(padding);
    TORCH_CHECK(noise_scale >= 0.0, "noise_scale must be non negative");
    const int64_t input_dims = input.dim();
    const Tensor x4 = input_to_4d(input);
    const Tensor we = weight_to_4d(w_erosion);
    const Tensor wd = weight_to_4d(w_dilation);
    check_4d(x4, we);
    check_4d(x4, wd);
    check_identity(x4, we, false);
    check_identity(x4, wd, false);
    TORCH_CHECK(soft.numel() == x4.size(1), "soft must hold one value per channel");
    check_device("morpho_sigma_forward_hip", x4, {we, wd, soft}, true);
    const bool needs_grad = torch::GradMode::is_enabled() &&
                            (input.requires_grad() || w_erosion.requires_grad() || w_dilation.requires_grad() || soft.requires_grad());
    const bool same = we.size(2) == wd.size(2) && we.size(3) == wd.size(3);
    const int64_t tap_bytes = 2 * x4.numel();
    const bool wide = x4.scalar_type() == c10::kFloat || x4.scalar_type() == c10::kDouble;  // the fused kernels' types
    const bool fused = wide && same && mca_morpho_pair_supported(we.size(2), we.size(3)) &&
                       (!needs_grad || (save_indices && tap_bytes <= env_bytes("MORPHOCORE_AMD_SAVED_TAPS_LIMIT", int64_t(8) << 30)));
    if (!fused)
    {
        const Tensor e = morpho_operation(EROSION, x4, we, IDENTITY, padding, padding_value, save_indices, noise_scale);
        const Tensor d = morpho_operation(DILATION, x4, wd, IDENTITY, padding, padding_value, save_indices, noise_scale);
        const Tensor s = soft.reshape({1, -1, 1, 1});
        return output_to_original(e * (1.0 - s) + d * s, input_dims);
    }
    return output_to_original(SigmaFunction::apply(x4, we, wd, soft, padding, padding_value, noise_scale, needs_grad), input_dims);
}

// ------------------------------------------------------------------------------------------------
// Smorph: Smorph<merge> (smorph.cpp:20-111).
// ------------------------------------------------------------------------------------------------

// One alpha per channel pair, index o * Cin + i ([Cout] for IDENTITY), or one value shared by every
// pair (smorph_cpu_kernels.hxx:642-649).
Tensor pair_alphas(const Tensor& alpha, int64_t merge, int64_t Cin, int64_t Cout)
{
    const int64_t pairs = merge == IDENTITY ? Cout : Cout * Cin;
    TORCH_CHECK(alpha.numel() == pairs || alpha.numel() == 1, "Alpha must have one value, or shape ",
                merge == IDENTITY ? "[channels]" : "[out_channels, in_channels]");
    return alpha.numel() == pairs ? alpha.contiguous().reshape({pairs}) : alpha.reshape({1}).expand({pairs}).contiguous();
}

// A single alpha shared by every pair receives the gradient of all of them (smorph.cpp:96-98).
Tensor alpha_grad(const Tensor& alpha, const Tensor& grad_pairs)
{
    return alpha.numel() == grad_pairs.numel() ? grad_pairs.view_as(alpha) : grad_pairs.sum().view_as(alpha);
}

class SmorphFunction : public torch::autograd::Function<SmorphFunction>
{
public:
    static Tensor forward(AutogradContext* ctx, const Tensor& x4, const Tensor& w4, const Tensor& alpha, int64_t merge, bool needs_grad)
    {
        const c10::DeviceGuard guard(x4.device());
        const Tensor x = x4.contiguous();
        const Tensor w = w4.contiguous();
        const Geom g = geom_of(x, w);
        const Tensor ap = pair_alphas(alpha, merge, g.Cin, g.Cout);
        // (No channel pair or no output: nothing for the kernels to do, and no workspace.)
        if (needs_grad && g.B * g.Cout * g.Cin * g.H * g.W > 0)
        {
            const size_t ws = x.scalar_type() == c10::kFloat
                                  ? mca_smorph_backward_workspace_size_f32((int)merge, g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW)
                                  : mca_smorph_backward_workspace_size_f64((int)merge, g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW);
            TORCH_CHECK(ws > 0, "Structuring element too large for the smorph backward kernels' shared memory (", g.KH, "x", g.KW,
                        "); run it without gradients");
        }
        Tensor out = torch::empty({g.B, g.Cout, g.H, g.W}, x.options());
        Tensor stats;
        if (x.scalar_type() == c10::kFloat)
        {
            const int64_t nbytes = needs_grad ? (int64_t)mca_smorph_stats_bytes_f32((int)merge, g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW) : 0;
            if (nbytes > 0) stats = SavedStats::get().allocate(nbytes, x.options());
            if (stats.defined())
                check_rc(mca_smorph_forward_stats_f32((int)merge, x.data_ptr<float>(), w.data_ptr<float>(), ap.data_ptr<float>(),
                                                      out.data_ptr<float>(), stats.data_ptr<float>(), g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH,
                                                      g.KW, stream_of(x)));
            else
                check_rc(mca_smorph_forward_f32((int)merge, x.data_ptr<float>(), w.data_ptr<float>(), ap.data_ptr<float>(), out.data_ptr<float>(),
                                                g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW, stream_of(x)));
        }
        else
        {
            check_rc(mca_smorph_forward_f64((int)merge, x.data_ptr<double>(), w.data_ptr<double>(), ap.data_ptr<double>(), out.data_ptr<double>(),
                                            g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW, stream_of(x)));
        }
        // The backward reads the output: the merge target of MAX and MIN.
        ctx->save_for_backward({out, alpha, x, w, stats});
        ctx->saved_data["merge"] = merge;
        return out;
    }

    static tensor_list backward(AutogradContext* ctx, tensor_list grad_outputs)
    {
        const auto saved = ctx->get_saved_variables();
        const Tensor& out = saved[0];
        const Tensor& alpha = saved[1];
        const Tensor& x = saved[2];
        const Tensor& w = saved[3];
        const Tensor& stats = saved[4];
        const int64_t merge = ctx->saved_data["merge"].toInt();
        const Tensor grad_output = grad_outputs[0].contiguous();
        TORCH_CHECK(grad_output.scalar_type() == x.scalar_type(), "grad_output must have the same dtype as input");
        const c10::DeviceGuard guard(x.device());
        const Geom g = geom_of(x, w);
        const Tensor ap = pair_alphas(alpha, merge, g.Cin, g.Cout);
        Tensor grad_input = torch::empty_like(x);
        Tensor grad_weight = torch::empty_like(w);
        Tensor grad_pairs = torch::empty_like(ap);
        if (x.scalar_type() == c10::kFloat)
        {
            const size_t n = mca_smorph_backward_workspace_size_f32((int)merge, g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW);
            Tensor ws = byte_buffer((int64_t)n, x);
            if (stats.defined())
                check_rc(mca_smorph_backward_stats_f32((int)merge, x.data_ptr<float>(), w.data_ptr<float>(), ap.data_ptr<float>(),
                                                       out.data_ptr<float>(), stats.data_ptr<float>(), grad_output.data_ptr<float>(),
                                                       grad_input.data_ptr<float>(), grad_weight.data_ptr<float>(), grad_pairs.data_ptr<float>(),
                                                       g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW, ws.data_ptr(), (size_t)ws.numel(),
                                                       stream_of(x)));
            else
                check_rc(mca_smorph_backward_f32((int)merge, x.data_ptr<float>(), w.data_ptr<float>(), ap.data_ptr<float>(), out.data_ptr<float>(),
                                                 grad_output.data_ptr<float>(), grad_input.data_ptr<float>(), grad_weight.data_ptr<float>(),
                                                 grad_pairs.data_ptr<float>(), g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW, ws.data_ptr(),
                                                 (size_t)ws.numel(), stream_of(x)));
        }
        else
        {
            const size_t n = mca_smorph_backward_workspace_size_f64((int)merge, g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW);
            Tensor ws = byte_buffer((int64_t)n, x);
            check_rc(mca_smorph_backward_f64((int)merge, x.data_ptr<double>(), w.data_ptr<double>(), ap.data_ptr<double>(), out.data_ptr<double>(),
                                             grad_output.data_ptr<double>(), grad_input.data_ptr<double>(), grad_weight.data_ptr<double>(),
                                             grad_pairs.data_ptr<double>(), g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW, ws.data_ptr(),
                                             (size_t)ws.numel(), stream_of(x)));
        }
        return {grad_input, grad_weight, alpha_grad(alpha, grad_pairs), Tensor(), Tensor()};
    }
};

// Body of the smorph operator: bindings.cpp:109-120, then Smorph::forward's checks (smorph.cpp:20-47,
// smorph_cpu_kernels.hxx:642-649).
Tensor smorph(const Tensor& input, const Tensor& weight, const Tensor& alpha, int64_t merge)
{
    merge = to_merge(merge);
    TORCH_CHECK(merge != SMOOTH, "Unsupported merge operation for smorph");
    const int64_t input_dims = input.dim();
    const Tensor x4 = input_to_4d(input);
    const Tensor w4 = weight_to_4d(weight);
    check_4d(x4, w4);
    if (merge == IDENTITY)
    {
        check_identity(x4, w4, true);
    }
    else
    {
        TORCH_CHECK(x4.size(1) == w4.size(1), "Input channels must match weight input channels");
    }
    pair_alphas(alpha, merge, x4.size(1), w4.size(0));
    check_device("smorph_forward_hip", x4, {w4, alpha});
    // Inside the Function's forward autograd is off: whether a backward can follow is decided here.
    const bool needs_grad = torch::GradMode::is_enabled() && (input.requires_grad() || weight.requires_grad() || alpha.requires_grad());
    return output_to_original(SmorphFunction::apply(x4, w4, alpha, merge, needs_grad), input_dims);
}

// SmorphSCM (smorph_scm.cpp:13-96): smorph with the SMOOTH channel merge, one beta per output channel.
// The forward keeps the soft merge's ref and 1 / sum per output pixel for the backward, and in float32
// (when the saved-statistics budget admits them) each pair's ref, 1 / S and W / S, which spare the
// backward their recomputation.
class SmorphScmFunction : public torch::autograd::Function<SmorphScmFunction>
{
public:
    static Tensor forward(AutogradContext* ctx, const Tensor& x4, const Tensor& w4, const Tensor& alpha, const Tensor& beta, bool needs_grad)
    {
        const c10::DeviceGuard guard(x4.device());
        const Tensor x = x4.contiguous();
        const Tensor w = w4.contiguous();
        const Tensor bt = beta.contiguous().reshape({-1});
        const Geom g = geom_of(x, w);
        const Tensor ap = pair_alphas(alpha, SMOOTH, g.Cin, g.Cout);
        const bool f32 = x.scalar_type() == c10::kFloat;
        if (needs_grad && g.B * g.Cout * g.H * g.W > 0)
        {
            const size_t ws = f32 ? mca_smorph_scm_backward_workspace_size_f32(g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW)
                                  : mca_smorph_scm_backward_workspace_size_f64(g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW);
            TORCH_CHECK(ws > 0, "Structuring element too large for the smorph backward kernels' shared memory (", g.KH, "x", g.KW,
                        "); run it without gradients");
        }
        Tensor out = torch::empty({g.B, g.Cout, g.H, g.W}, x.options());
        Tensor mstats = needs_grad ? torch::empty({2, g.B, g.Cout, g.H, g.W}, x.options()) : Tensor();
        // float32 with a backward to follow: the pair statistics too, when the budget admits them
        // (they then also stand in for the pair-output workspace).
        Tensor pstats;
        if (f32 && needs_grad)
        {
            const int64_t nbytes = (int64_t)mca_smorph_scm_stats_bytes_f32(g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW);
            if (nbytes > 0) pstats = SavedStats::get().allocate(nbytes, x.options());
        }
        if (pstats.defined())
        {
            check_rc(mca_smorph_scm_forward_stats_f32(x.data_ptr<float>(), w.data_ptr<float>(), ap.data_ptr<float>(), bt.data_ptr<float>(),
                                                      out.data_ptr<float>(), mstats.data_ptr<float>(), pstats.data_ptr<float>(), g.B, g.Cin,
                                                      g.Cout, g.Cw, g.H, g.W, g.KH, g.KW, stream_of(x)));
        }
        else
        {
            const size_t n = f32 ? mca_smorph_scm_forward_workspace_size_f32(g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW)
                                 : mca_smorph_scm_forward_workspace_size_f64(g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW);
            Tensor ws = byte_buffer((int64_t)n, x);
            if (f32)
                check_rc(mca_smorph_scm_forward_f32(x.data_ptr<float>(), w.data_ptr<float>(), ap.data_ptr<float>(), bt.data_ptr<float>(),
                                                    out.data_ptr<float>(), mstats.defined() ? mstats.data_ptr<float>() : nullptr, g.B, g.Cin,
                                                    g.Cout, g.Cw, g.H, g.W, g.KH, g.KW, ws.data_ptr(), (size_t)ws.numel(), stream_of(x)));
            else
                check_rc(mca_smorph_scm_forward_f64(x.data_ptr<double>(), w.data_ptr<double>(), ap.data_ptr<double>(), bt.data_ptr<double>(),
                                                    out.data_ptr<double>(), mstats.defined() ? mstats.data_ptr<double>() : nullptr, g.B, g.Cin,
                                                    g.Cout, g.Cw, g.H, g.W, g.KH, g.KW, ws.data_ptr(), (size_t)ws.numel(), stream_of(x)));
        }
        ctx->save_for_backward({out, alpha, beta, x, w, mstats, pstats});
        return out;
    }

    static tensor_list backward(AutogradContext* ctx, tensor_list grad_outputs)
    {
        const auto saved = ctx->get_saved_variables();
        const Tensor& out = saved[0];
        const Tensor& alpha = saved[1];
        const Tensor& beta = saved[2];
        const Tensor& x = saved[3];
        const Tensor& w = saved[4];
        const Tensor& mstats = saved[5];
        const Tensor& pstats = saved[6];
        TORCH_CHECK(mstats.defined(), "smorph_scm: the forward ran without gradients and kept no merge statistics");
        const Tensor grad_output = grad_outputs[0].contiguous();
        TORCH_CHECK(grad_output.scalar_type() == x.scalar_type(), "grad_output must have the same dtype as input");
        const c10::DeviceGuard guard(x.device());
        const Geom g = geom_of(x, w);
        const Tensor ap = pair_alphas(alpha, SMOOTH, g.Cin, g.Cout);
        const Tensor bt = beta.contiguous().reshape({-1});
        Tensor grad_input = torch::empty_like(x);
        Tensor grad_weight = torch::empty_like(w);
        Tensor grad_pairs = torch::empty_like(ap);
        Tensor grad_beta = torch::empty_like(bt);
        if (x.scalar_type() == c10::kFloat)
        {
            const size_t n = mca_smorph_scm_backward_workspace_size_f32(g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW);
            Tensor ws = byte_buffer((int64_t)n, x);
            if (pstats.defined())
                check_rc(mca_smorph_scm_backward_stats_f32(x.data_ptr<float>(), w.data_ptr<float>(), ap.data_ptr<float>(), bt.data_ptr<float>(),
                                                           out.data_ptr<float>(), mstats.data_ptr<float>(), pstats.data_ptr<float>(),
                                                           grad_output.data_ptr<float>(), grad_input.data_ptr<float>(),
                                                           grad_weight.data_ptr<float>(), grad_pairs.data_ptr<float>(),
                                                           grad_beta.data_ptr<float>(), g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW,
                                                           ws.data_ptr(), (size_t)ws.numel(), stream_of(x)));
            else
                check_rc(mca_smorph_scm_backward_f32(x.data_ptr<float>(), w.data_ptr<float>(), ap.data_ptr<float>(), bt.data_ptr<float>(),
                                                     out.data_ptr<float>(), mstats.data_ptr<float>(), grad_output.data_ptr<float>(),
                                                     grad_input.data_ptr<float>(), grad_weight.data_ptr<float>(), grad_pairs.data_ptr<float>(),
                                                     grad_beta.data_ptr<float>(), g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW,
                                                     ws.data_ptr(), (size_t)ws.numel(), stream_of(x)));
        }
        else
        {
            const size_t n = mca_smorph_scm_backward_workspace_size_f64(g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW);
            Tensor ws = byte_buffer((int64_t)n, x);
            check_rc(mca_smorph_scm_backward_f64(x.data_ptr<double>(), w.data_ptr<double>(), ap.data_ptr<double>(), bt.data_ptr<double>(),
                                                 out.data_ptr<double>(), mstats.data_ptr<double>(), grad_output.data_ptr<double>(),
                                                 grad_input.data_ptr<double>(), grad_weight.data_ptr<double>(), grad_pairs.data_ptr<double>(),
                                                 grad_beta.data_ptr<double>(), g.B, g.Cin, g.Cout, g.Cw, g.H, g.W, g.KH, g.KW, ws.data_ptr(),
                                                 (size_t)ws.numel(), stream_of(x)));
        }
        return {grad_input, grad_weight, alpha_grad(alpha, grad_pairs), grad_beta.view_as(beta), Tensor()};
    }
};

// Body of the smorph_scm operator, smorph with the SMOOTH channel merge: bindings.cpp:122-125, then
// SmorphSCM::forward's checks (smorph_scm.cpp:13-34, smorph_cpu_kernels.hxx:642-649, 668-672).
Tensor smorph_scm(const Tensor& input, const Tensor& weight, const Tensor& alpha, const Tensor& beta)
{
    const int64_t input_dims = input.dim();
    const Tensor x4 = input_to_4d(input);
    const Tensor w4 = weight_to_4d(weight);
    check_4d(x4, w4);
    TORCH_CHECK(x4.size(1) == w4.size(1), "Input channels must match weight input channels");
    pair_alphas(alpha, SMOOTH, x4.size(1), w4.size(0));
    TORCH_CHECK(beta.numel() == w4.size(0), "Beta must have shape [out_channels]");
    check_device("smorph_scm_forward_hip", x4, {w4, alpha, beta});
    const bool needs_grad = torch::GradMode::is_enabled() &&
                            (input.requires_grad() || weight.requires_grad() || alpha.requires_grad() || beta.requires_grad());
    return output_to_original(SmorphScmFunction::apply(x4, w4, alpha, beta, needs_grad), input_dims);
}

// ------------------------------------------------------------------------------------------------
// Layer stacks: a chain of dilation / erosion / smorph layers as one operator and one autograd node,
// run by the C ABI's stack executor batch chunk by batch chunk (mca_stack_*). No reference counterpart:
// the reference chains one operator call and one autograd node per layer in Python
// (functional/dilation.py:89-91, functional/smorph.py:72-75, functional/erosion.py:89-91).
// ------------------------------------------------------------------------------------------------

constexpr int64_t STACK_SMORPH = MCA_STACK_SMORPH;

// The C ABI's layer descriptors: weights as each operator receives them, per-pair alphas (one tensor
// per smorph layer, in order), the save flag of each layer.
std::vector<mca_stack_layer> stack_layers(const std::vector<int64_t>& kinds, const std::vector<int64_t>& merges,
                                          const std::vector<int64_t>& paddings, const std::vector<double>& values,
                                          const std::vector<int64_t>& save, const std::vector<Tensor>& weights, const std::vector<Tensor>& aps)
{
    std::vector<mca_stack_layer> layers(kinds.size());
    size_t a = 0;
    for (size_t l = 0; l < kinds.size(); ++l)
    {
        mca_stack_layer& L = layers[l];
        const Tensor& w = weights[l];
        L.kind = (int)kinds[l];
        L.merge = (int)merges[l];
        L.replicate = kinds[l] != STACK_SMORPH && paddings[l] == REPLICATE;
        L.save = (int)save[l];
        L.fill = kinds[l] != STACK_SMORPH ? fill_value(kinds[l], paddings[l], values[l]) : 0.0;
        L.out_channels = w.size(0);
        L.weight_channels = w.size(1);
        L.kh = w.size(2);
        L.kw = w.size(3);
        L.weight = w.data_ptr();
        L.alpha = kinds[l] == STACK_SMORPH ? aps[a++].data_ptr() : nullptr;
        L.grad_weight = nullptr;
        L.grad_alpha = nullptr;
    }
    return layers;
}

int stack_plan(bool f32, const std::vector<mca_stack_layer>& layers, const Tensor& x, int64_t chunk, size_t* saved, size_t* backward)
{
    return (f32 ? mca_stack_plan_f32 : mca_stack_plan_f64)(layers.data(), (int)layers.size(), x.size(0), x.size(1), x.size(2), x.size(3), chunk,
                                                          saved, backward);
}

class StackFunction : public torch::autograd::Function<StackFunction>
{
public:
    // params: the n layers' weights, then the smorph layers' alphas.
    static Tensor forward(AutogradContext* ctx, const Tensor& x4, at::TensorList params, std::vector<int64_t> kinds, std::vector<int64_t> merges,
                          std::vector<int64_t> paddings, std::vector<double> values, bool save_indices, int64_t chunk, bool needs_grad,
                          bool input_grad)
    {
        const c10::DeviceGuard guard(x4.device());
        const Tensor x = x4.contiguous();
        const size_t n = kinds.size();
        const bool f32 = x.scalar_type() == c10::kFloat;
        std::vector<Tensor> weights, alphas, aps;
        int64_t cin = x.size(1);
        for (size_t l = 0, a = n; l < n; ++l)
        {
            weights.push_back(params[l].contiguous());
            if (kinds[l] == STACK_SMORPH)
            {
                alphas.push_back(params[a++]);
                aps.push_back(pair_alphas(alphas.back(), merges[l], cin, weights[l].size(0)));
            }
            cin = weights[l].size(0);
        }
        // What the backward may reuse: winners (per-pair taps within MORPHOCORE_AMD_SAVED_TAPS_LIMIT), and
        // float32 smorph statistics when the saved-statistics budget admits the whole saved state.
        std::vector<int64_t> save(n, 0);
        bool any_stats = false;
        cin = x.size(1);
        for (size_t l = 0; l < n; ++l)
        {
            const Tensor& w = weights[l];
            if (save_indices && needs_grad)
            {
                if (kinds[l] == STACK_SMORPH)
                {
                    save[l] = f32;
                    any_stats = any_stats || f32;
                }
                else
                {
                    const int64_t nbytes =
                        (int64_t)mca_morpho_indices_bytes((int)merges[l], x.size(0), cin, w.size(0), w.size(1), x.size(2), x.size(3), w.size(2), w.size(3));
                    save[l] = (merges[l] == MAX || merges[l] == MIN) || nbytes <= env_bytes("MORPHOCORE_AMD_SAVED_TAPS_LIMIT", int64_t(8) << 30);
                }
            }
            cin = w.size(0);
        }
        std::vector<mca_stack_layer> layers = stack_layers(kinds, merges, paddings, values, save, weights, aps);
        size_t saved_bytes = 0, backward_bytes = 0;
        check_rc(stack_plan(f32, layers, x, chunk, &saved_bytes, &backward_bytes));
        if (needs_grad && backward_bytes == 0 && x.numel() > 0)
            TORCH_CHECK(false, "Structuring element too large for the smorph backward kernels' shared memory; run the stack without gradients");
        Tensor saved;
        if (any_stats) saved = SavedStats::get().allocate((int64_t)saved_bytes, x.options());
        if (!saved.defined())
        {
            if (any_stats)
            {
                for (size_t l = 0; l < n; ++l)
                    if (kinds[l] == STACK_SMORPH) save[l] = 0;
                layers = stack_layers(kinds, merges, paddings, values, save, weights, aps);
                check_rc(stack_plan(f32, layers, x, chunk, &saved_bytes, &backward_bytes));
            }
            saved = byte_buffer((int64_t)saved_bytes, x);
        }
        Tensor out = torch::empty({x.size(0), weights.back().size(0), x.size(2), x.size(3)}, x.options());
        if (f32)
            check_rc(mca_stack_forward_f32(layers.data(), (int)n, x.data_ptr<float>(), out.data_ptr<float>(), x.size(0), x.size(1), x.size(2),
                                           x.size(3), chunk, saved.data_ptr(), (size_t)saved.nbytes(), stream_of(x)));
        else
            check_rc(mca_stack_forward_f64(layers.data(), (int)n, x.data_ptr<double>(), out.data_ptr<double>(), x.size(0), x.size(1), x.size(2),
                                           x.size(3), chunk, saved.data_ptr(), (size_t)saved.nbytes(), stream_of(x)));
        std::vector<Tensor> keep = {x, out, saved};
        keep.insert(keep.end(), weights.begin(), weights.end());
        keep.insert(keep.end(), alphas.begin(), alphas.end());
        keep.insert(keep.end(), aps.begin(), aps.end());
        ctx->save_for_backward(keep);
        ctx->saved_data["kinds"] = kinds;
        ctx->saved_data["merges"] = merges;
        ctx->saved_data["paddings"] = paddings;
        ctx->saved_data["values"] = values;
        ctx->saved_data["save"] = save;
        ctx->saved_data["chunk"] = chunk;
        ctx->saved_data["input_grad"] = input_grad;
        return out;
    }

    static tensor_list backward(AutogradContext* ctx, tensor_list grad_outputs)
    {
        const auto saved = ctx->get_saved_variables();
        const std::vector<int64_t> kinds = ctx->saved_data["kinds"].toIntVector();
        const std::vector<int64_t> merges = ctx->saved_data["merges"].toIntVector();
        const std::vector<int64_t> paddings = ctx->saved_data["paddings"].toIntVector();
        const std::vector<double> values = ctx->saved_data["values"].toDoubleVector();
        const std::vector<int64_t> save = ctx->saved_data["save"].toIntVector();
        const int64_t chunk = ctx->saved_data["chunk"].toInt();
        const bool input_grad = ctx->saved_data["input_grad"].toBool();
        const size_t n = kinds.size();
        const size_t m = (saved.size() - 3 - n) / 2;
        const Tensor& x = saved[0];
        const Tensor& out = saved[1];
        const Tensor& state = saved[2];
        const std::vector<Tensor> weights(saved.begin() + 3, saved.begin() + 3 + n);
        const std::vector<Tensor> alphas(saved.begin() + 3 + n, saved.begin() + 3 + n + m);
        const std::vector<Tensor> aps(saved.begin() + 3 + n + m, saved.end());
        const Tensor grad_output = grad_outputs[0].contiguous();
        TORCH_CHECK(grad_output.sizes() == out.sizes(), "grad_output shape mismatch: expected [", out.sizes(), "] but got [", grad_output.sizes(),
                    "]");
        TORCH_CHECK(grad_output.device() == x.device(), "grad_output must be on the same device as input");
        TORCH_CHECK(grad_output.scalar_type() == x.scalar_type(), "grad_output must have the same dtype as input");
        const c10::DeviceGuard guard(x.device());
        const bool f32 = x.scalar_type() == c10::kFloat;
        std::vector<mca_stack_layer> layers = stack_layers(kinds, merges, paddings, values, save, weights, aps);
        std::vector<Tensor> grad_w, grad_pairs;
        for (size_t l = 0, a = 0; l < n; ++l)
        {
            grad_w.push_back(torch::empty_like(weights[l]));
            layers[l].grad_weight = grad_w.back().data_ptr();
            if (kinds[l] == STACK_SMORPH)
            {
                grad_pairs.push_back(torch::empty_like(aps[a++]));
                layers[l].grad_alpha = grad_pairs.back().data_ptr();
            }
        }
        size_t saved_bytes = 0, backward_bytes = 0;
        check_rc(stack_plan(f32, layers, x, chunk, &saved_bytes, &backward_bytes));
        Tensor ws = byte_buffer((int64_t)backward_bytes, x);
        Tensor grad_input = input_grad ? torch::empty_like(x) : Tensor();
        if (f32)
            check_rc(mca_stack_backward_f32(layers.data(), (int)n, x.data_ptr<float>(), out.data_ptr<float>(), grad_output.data_ptr<float>(),
                                            input_grad ? grad_input.data_ptr<float>() : nullptr, x.size(0), x.size(1), x.size(2), x.size(3),
                                            chunk, state.data_ptr(), (size_t)state.nbytes(), ws.data_ptr(), (size_t)ws.numel(), stream_of(x)));
        else
            check_rc(mca_stack_backward_f64(layers.data(), (int)n, x.data_ptr<double>(), out.data_ptr<double>(), grad_output.data_ptr<double>(),
                                            input_grad ? grad_input.data_ptr<double>() : nullptr, x.size(0), x.size(1), x.size(2), x.size(3),
                                            chunk, state.data_ptr(), (size_t)state.nbytes(), ws.data_ptr(), (size_t)ws.numel(), stream_of(x)));
        tensor_list grads = {grad_input};
        grads.insert(grads.end(), grad_w.begin(), grad_w.end());
        for (size_t a = 0; a < m; ++a) grads.push_back(alpha_grad(alphas[a], grad_pairs[a]));
        for (int k = 0; k < 8; ++k) grads.push_back(Tensor());  // kinds .. input_grad
        return grads;
    }
};

// morpho_stack(input, weights, alphas, kinds, merges, paddings, padding_values, save_indices, chunk):
// layer l is kinds[l] (0 dilation, 1 erosion, 2 smorph) with weights[l] as that operator receives it
// (an erosion's element flipped, a smorph's blended w~), merges[l], and for dilation / erosion the
// padding paddings[l] / padding_values[l]; alphas holds one alpha per smorph layer, in order (any shape
// the smorph operator takes). Each layer's checks are the single operator's.
Tensor morpho_stack(const Tensor& input, at::TensorList weights, at::TensorList alphas, at::IntArrayRef kinds, at::IntArrayRef merges,
                    at::IntArrayRef paddings, at::ArrayRef<double> padding_values, bool save_indices, int64_t chunk)
{
    const size_t n = kinds.size();
    TORCH_CHECK(n >= 1, "morpho_stack needs at least one layer");
    TORCH_CHECK(weights.size() == n && merges.size() == n && paddings.size() == n && padding_values.size() == n,
                "morpho_stack: weights, kinds, merges, paddings and padding_values must have one entry per layer");
    TORCH_CHECK(chunk >= 0, "chunk must be non negative");
    const int64_t input_dims = input.dim();
    const Tensor x4 = input_to_4d(input);
    TORCH_CHECK(x4.dim() == 4, "Input must be a 4d tensor (batch_size, in_channels, height, width)");
    std::vector<Tensor> params;
    std::vector<int64_t> kv(kinds.begin(), kinds.end()), mv, pv(n, 0);
    bool needs_grad = input.requires_grad();
    size_t a = 0;
    int64_t cin = x4.size(1);
    for (size_t l = 0; l < n; ++l)
    {
        TORCH_CHECK(kinds[l] == DILATION || kinds[l] == EROSION || kinds[l] == STACK_SMORPH, "Unknown layer kind ", kinds[l], " at layer ", l);
        const int64_t merge = to_merge(merges[l]);
        TORCH_CHECK(merge != SMOOTH, "Unsupported merge operation");
        mv.push_back(merge);
        if (kinds[l] != STACK_SMORPH) pv[l] = to_padding(paddings[l]);
        const Tensor w4 = weight_to_4d(weights[l]);
        TORCH_CHECK(w4.dim() == 4, "Weight must be a 4d tensor (out_channels, in_channels, kernel_height, kernel_width)");
        if (merge == IDENTITY)
        {
            TORCH_CHECK(w4.size(0) == cin, "Identity mode requires weight.shape[0] == input.shape[1]");
            TORCH_CHECK(w4.size(1) == 1, "Identity mode requires weight.shape[1] == 1");
        }
        else
        {
            TORCH_CHECK(w4.size(1) == cin, "Input channels must match weight input channels");
        }
        check_device("morpho_stack_forward_hip", x4, {w4});
        params.push_back(w4);
        needs_grad = needs_grad || weights[l].requires_grad();
        if (kinds[l] == STACK_SMORPH)
        {
            TORCH_CHECK(a < alphas.size(), "morpho_stack: one alpha per smorph layer");
            pair_alphas(alphas[a], merge, cin, w4.size(0));
            check_device("morpho_stack_forward_hip", x4, {alphas[a]});
            needs_grad = needs_grad || alphas[a].requires_grad();
            ++a;
        }
        cin = w4.size(0);
    }
    TORCH_CHECK(a == alphas.size(), "morpho_stack: one alpha per smorph layer");
    params.insert(params.end(), alphas.begin(), alphas.end());
    needs_grad = needs_grad && torch::GradMode::is_enabled();
    std::vector<double> vv(padding_values.begin(), padding_values.end());
    const Tensor out = StackFunction::apply(x4, at::TensorList(params), kv, mv, pv, vv, save_indices, chunk, needs_grad,
                                            needs_grad && input.requires_grad());
    return output_to_original(out, input_dims);
}

// Module-level helpers for tests and the benchmark (no reference counterpart).
PyObject* py_saved_stats_live_bytes(PyObject*, PyObject* args)
{
    int device = 0;
    if (!PyArg_ParseTuple(args, "i", &device)) return nullptr;
    return PyLong_FromLongLong(SavedStats::get().live_bytes((c10::DeviceIndex)device));
}

PyObject* py_saved_stats_admit(PyObject*, PyObject* args)
{
    long long nbytes = 0;
    int device = 0;
    if (!PyArg_ParseTuple(args, "Li", &nbytes, &device)) return nullptr;
    bool ok = false;
    try
    {
        ok = SavedStats::get().admit(nbytes, (c10::DeviceIndex)device);
    }
    catch (const std::exception& e)
    {
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    return PyBool_FromLong(ok);
}

PyObject* py_saved_stats_policy(PyObject*, PyObject* args)
{
    long long nbytes = 0, live = 0, budget = 0, avail = 0, limit = -1;
    if (!PyArg_ParseTuple(args, "LLLL|L", &nbytes, &live, &budget, &avail, &limit)) return nullptr;
    return PyBool_FromLong(stats_policy(nbytes, live, budget, avail, limit));
}

PyMethodDef g_methods[] = {
    {"saved_stats_live_bytes", py_saved_stats_live_bytes, METH_VARARGS,
     "saved_stats_live_bytes(device) -> bytes of saved smorph statistics still alive on the device"},
    {"saved_stats_admit", py_saved_stats_admit, METH_VARARGS,
     "saved_stats_admit(nbytes, device) -> whether a smorph forward would save nbytes of statistics now"},
    {"saved_stats_policy", py_saved_stats_policy, METH_VARARGS,
     "saved_stats_policy(nbytes, live, budget, avail[, limit]) -> the admission rule on given numbers"},
    {nullptr, nullptr, 0, nullptr},
};

}  // namespace

// Same namespace, names and schemas as the reference (bindings.cpp:130-138).
TORCH_LIBRARY(morphocore, m)
{
    m.def("dilation(Tensor input, Tensor weight, int merge, int padding, float padding_value=0., bool save_indices=True, "
          "float noise_scale=0.) -> Tensor");
    m.def("erosion(Tensor input, Tensor weight, int merge, int padding, float padding_value=0., bool save_indices=True, "
          "float noise_scale=0.) -> Tensor");
    m.def("smorph(Tensor input, Tensor weight, Tensor alpha, int merge) -> Tensor");
    m.def("smorph_scm(Tensor input, Tensor weight, Tensor alpha, Tensor beta) -> Tensor");
    // No reference counterpart: the fused form of the reference's Python opening / closing.
    m.def("opening_closing(Tensor input, Tensor w_first, Tensor w_second, int first_op, int padding, float padding_value=0., "
          "bool save_indices=True, float noise_scale=0.) -> Tensor");
    // No reference counterpart: the fused form of the reference's Python sigma_layer, 'identity' merge.
    m.def("sigma_identity(Tensor input, Tensor w_erosion, Tensor w_dilation, Tensor soft, int padding, float padding_value=0., "
          "bool save_indices=True, float noise_scale=0.) -> Tensor");
    // No reference counterpart: a chain of dilation / erosion / smorph layers as one operator.
    m.def("morpho_stack(Tensor input, Tensor[] weights, Tensor[] alphas, int[] kinds, int[] merges, int[] paddings, "
          "float[] padding_values, bool save_indices=True, int chunk=0) -> Tensor");
}

// CompositeImplicitAutograd, as the reference (bindings.cpp:142-148): the kernels run above autograd
// and the autograd Functions above record the backward themselves.
TORCH_LIBRARY_IMPL(morphocore, CompositeImplicitAutograd, m)
{
    m.impl("dilation", &morpho_dilation);
    m.impl("erosion", &morpho_erosion);
    m.impl("smorph", &smorph);
    m.impl("smorph_scm", &smorph_scm);
    m.impl("opening_closing", &opening_closing);
    m.impl("sigma_identity", &sigma_identity);
    m.impl("morpho_stack", &morpho_stack);
}

// Importing morphocore_amd._C loads this library, which runs the registrations above.
PyMODINIT_FUNC PyInit__C(void)
{
    static struct PyModuleDef module_def = {PyModuleDef_HEAD_INIT, "_C", "morphocore_amd operators (torch.ops.morphocore.*)", -1, g_methods};
    return PyModule_Create(&module_def);
}
