// Layer stacks (mca_stack_*): a chain of dilation / erosion / smorph layers run forward and backward
// by one call each, batch chunk by batch chunk, through the single-layer entry points. The reference
// composes such chains layer by layer in Python (functional/dilation.py:89-91 ->
// functional/smorph.py:72-75 -> functional/erosion.py:89-91), one autograd node and one whole-batch
// launch per layer. Here each chunk of batch elements passes through every layer before the next chunk
// starts: a layer reads its input activation right after the previous layer wrote it, and the backward
// keeps one chunk of each intermediate gradient, in two ping-pong buffers, instead of whole-batch
// gradient tensors. The default chunk is the whole batch: the layers of such stacks are bound by their
// instruction issue, not by HBM, so smaller chunks save no measurable time by reading activations from
// the last-level cache and lose some to each launch's tail (chunks of 1, 2, 4 of 8 batch elements of an
// 8 x 64 x 512 x 512, 11 x 11 dilation -> smorph -> erosion step: 2.0, 1.5, 0.9% slower); they bound
// the backward's intermediate gradient memory to one chunk.
//
// Buffers (offsets aligned to 256 bytes):
//   saved (forward -> backward): the activation after every layer but the last, [B, C_{l+1}, H, W];
//     per saving layer and chunk, the winners (mca_morpho_indices_bytes of the chunk) or the smorph
//     pair statistics (mca_smorph_stats_bytes_f32 of the chunk), each chunk in its own region;
//   backward workspace: the two chunk gradient buffers, the largest layer backward's workspace, one
//     partial weight / alpha gradient of one chunk and, when there are several chunks, a double
//     accumulator per wanted gradient (partials added in chunk order, rounded once at the end).
#include "../../include/morphocore_amd.h"

#include <algorithm>
#include <string>
#include <vector>

#include "launch.hpp"

namespace
{

template <typename T>
struct Api;

template <>
struct Api<float>
{
    static constexpr auto fwd = mca_morpho_forward_f32;
    static constexpr auto bwd = mca_morpho_backward_f32;
    static constexpr auto bwd_ws = mca_morpho_backward_workspace_size_f32;
    static constexpr auto sfwd = mca_smorph_forward_f32;
    static constexpr auto sbwd = mca_smorph_backward_f32;
    static constexpr auto sbwd_ws = mca_smorph_backward_workspace_size_f32;
};

template <>
struct Api<double>
{
    static constexpr auto fwd = mca_morpho_forward_f64;
    static constexpr auto bwd = mca_morpho_backward_f64;
    static constexpr auto bwd_ws = mca_morpho_backward_workspace_size_f64;
    static constexpr auto sfwd = mca_smorph_forward_f64;
    static constexpr auto sbwd = mca_smorph_backward_f64;
    static constexpr auto sbwd_ws = mca_smorph_backward_workspace_size_f64;
};

struct LayerPlan
{
    int64_t cin = 0, wnumel = 0, npairs = 0;
    size_t act = 0;                       // offset of the layer's output activation in `saved` (not the last layer)
    size_t idx = 0, idx_chunk = 0;        // saved winners: offset and bytes per chunk (idx_chunk 0: none)
    size_t stats = 0, stats_chunk = 0;    // saved smorph statistics: offset and bytes per chunk (0: none)
    size_t acc_w = 0, acc_a = 0;          // double accumulators of the wanted gradients (several chunks)
};

struct Plan
{
    int n = 0;
    int64_t B = 0, H = 0, W = 0, plane = 0, chunk = 1, nchunks = 0;
    std::vector<int64_t> ch;  // C_0 .. C_n
    std::vector<LayerPlan> layers;
    size_t saved = 0;
    size_t gbuf[2] = {0, 0}, lws = 0, lws_bytes = 0, part_w = 0, part_a = 0, backward = 0;
    bool backward_ok = true;
};

size_t take(size_t& end, size_t bytes)
{
    const size_t at = end;
    end += mca::align_up(bytes);
    return at;
}

int64_t chunk_at(const Plan& p, int64_t c) { return std::min(p.chunk, p.B - c * p.chunk); }

template <typename T>
int make_plan(const mca_stack_layer* layers, int n, int64_t B, int64_t C, int64_t H, int64_t W, int64_t chunk, Plan& p)
{
    if (n < 1 || !layers) return mca::api_fail("A layer stack needs at least one layer");
    if (B < 0 || C < 0 || H < 0 || W < 0) return mca::api_fail("Tensor dimensions must be non negative and below 2^31");
    if (chunk < 0) return mca::api_fail("chunk must be non negative");
    p.n = n;
    p.B = B;
    p.H = H;
    p.W = W;
    p.plane = H * W;
    p.ch.assign(1, C);
    for (int l = 0; l < n; ++l)
    {
        const mca_stack_layer& L = layers[l];
        const int64_t cin = p.ch.back();
        if (L.kind != MCA_STACK_DILATION && L.kind != MCA_STACK_EROSION && L.kind != MCA_STACK_SMORPH)
            return mca::api_fail(("Unknown layer kind " + std::to_string(L.kind) + " at layer " + std::to_string(l)).c_str());
        if (L.merge < 0 || L.merge > mca::MERGE_IDENTITY) return mca::api_fail(("Unknown merge mode " + std::to_string(L.merge)).c_str());
        if (L.merge == mca::MERGE_SMOOTH) return mca::api_fail("Unsupported merge operation");
        if (L.out_channels < 0 || L.weight_channels < 0 || L.kh < 1 || L.kw < 1)
            return mca::api_fail(("Invalid structuring element shape at layer " + std::to_string(l)).c_str());
        if (L.merge == mca::MERGE_IDENTITY ? (L.out_channels != cin || L.weight_channels != 1) : L.weight_channels != cin)
            return mca::api_fail(("Layer " + std::to_string(l) + ": the structuring element does not match the " + std::to_string(cin) +
                                  " channels it reads")
                                     .c_str());
        const int64_t wnumel = L.out_channels * L.weight_channels * L.kh * L.kw;
        if (wnumel > 0 && !L.weight) return mca::api_fail(("Layer " + std::to_string(l) + ": weight must not be null").c_str());
        LayerPlan lp;
        lp.cin = cin;
        lp.wnumel = wnumel;
        if (L.kind == MCA_STACK_SMORPH)
        {
            lp.npairs = L.merge == mca::MERGE_IDENTITY ? L.out_channels : L.out_channels * cin;
            if (lp.npairs > 0 && !L.alpha) return mca::api_fail(("Layer " + std::to_string(l) + ": alpha must not be null").c_str());
        }
        p.layers.push_back(lp);
        p.ch.push_back(L.out_channels);
    }
    p.chunk = std::max<int64_t>(1, std::min(chunk > 0 ? chunk : B, std::max<int64_t>(B, 1)));
    p.nchunks = (B + p.chunk - 1) / p.chunk;
    const int64_t last = B - (p.nchunks - 1) * p.chunk;  // batch elements of the last chunk (B > 0)

    size_t end = 0;
    for (int l = 0; l + 1 < n; ++l) p.layers[l].act = take(end, (size_t)(B * p.ch[l + 1] * p.plane) * sizeof(T));
    for (int l = 0; l < n && B > 0; ++l)
    {
        const mca_stack_layer& L = layers[l];
        LayerPlan& lp = p.layers[l];
        if (!L.save) continue;
        if (L.kind != MCA_STACK_SMORPH)
        {
            if (mca::packed_winners(L.merge) && !(L.kh * L.kw < (1 << 16) && lp.cin < (1 << 15))) continue;
            lp.idx_chunk = mca::align_up(mca_morpho_indices_bytes(L.merge, p.chunk, lp.cin, L.out_channels, L.weight_channels, H, W, L.kh, L.kw));
            lp.idx = take(end, lp.idx_chunk * p.nchunks);
        }
        else if (sizeof(T) == 4)
        {
            lp.stats_chunk =
                mca::align_up(mca_smorph_stats_bytes_f32(L.merge, p.chunk, lp.cin, L.out_channels, L.weight_channels, H, W, L.kh, L.kw));
            lp.stats = take(end, lp.stats_chunk * p.nchunks);
        }
    }
    p.saved = end;

    end = 0;
    int64_t gch = 0;
    for (int l = 0; l < n; ++l) gch = std::max(gch, p.ch[l]);
    const size_t gbytes = (size_t)(p.chunk * gch * p.plane) * sizeof(T);
    p.gbuf[0] = take(end, gbytes);
    p.gbuf[1] = take(end, gbytes);
    int64_t maxw = 0, maxa = 0;
    for (int l = 0; l < n && B > 0; ++l)
    {
        const mca_stack_layer& L = layers[l];
        const LayerPlan& lp = p.layers[l];
        maxw = std::max(maxw, lp.wnumel);
        maxa = std::max(maxa, lp.npairs);
        for (const int64_t bc : {p.chunk, last})
        {
            size_t ws;
            if (L.kind == MCA_STACK_SMORPH)
            {
                ws = Api<T>::sbwd_ws(L.merge, bc, lp.cin, L.out_channels, L.weight_channels, H, W, L.kh, L.kw);
                if (ws == 0 && bc * L.out_channels * lp.cin * p.plane > 0) p.backward_ok = false;
            }
            else
            {
                ws = Api<T>::bwd_ws(L.merge, lp.idx_chunk > 0, bc, lp.cin, L.out_channels, L.weight_channels, H, W, L.kh, L.kw);
            }
            p.lws_bytes = std::max(p.lws_bytes, ws);
        }
    }
    p.lws = take(end, p.lws_bytes);
    p.part_w = take(end, (size_t)maxw * sizeof(T));
    p.part_a = take(end, (size_t)maxa * sizeof(T));
    for (int l = 0; l < n && p.nchunks > 1; ++l)
    {
        LayerPlan& lp = p.layers[l];
        if (layers[l].grad_weight) lp.acc_w = take(end, (size_t)lp.wnumel * sizeof(double));
        if (layers[l].kind == MCA_STACK_SMORPH && layers[l].grad_alpha) lp.acc_a = take(end, (size_t)lp.npairs * sizeof(double));
    }
    p.backward = end;
    return MCA_OK;
}

template <typename T>
int stack_plan(const mca_stack_layer* layers, int n, int64_t B, int64_t C, int64_t H, int64_t W, int64_t chunk, size_t* saved_bytes,
               size_t* backward_bytes)
{
    Plan p;
    const int rc = make_plan<T>(layers, n, B, C, H, W, chunk, p);
    if (rc != MCA_OK) return rc;
    if (saved_bytes) *saved_bytes = p.saved;
    if (backward_bytes) *backward_bytes = p.backward_ok ? p.backward : 0;
    return MCA_OK;
}

template <typename T>
const T* layer_input(const Plan& p, const T* input, const unsigned char* saved, int l, int64_t b0)
{
    const T* base = l == 0 ? input : reinterpret_cast<const T*>(saved + p.layers[l - 1].act);
    return base + b0 * p.ch[l] * p.plane;
}

template <typename T>
int stack_forward(const mca_stack_layer* layers, int n, const T* input, T* output, int64_t B, int64_t C, int64_t H, int64_t W, int64_t chunk,
                  void* saved, size_t saved_bytes, void* stream)
{
    Plan p;
    int rc = make_plan<T>(layers, n, B, C, H, W, chunk, p);
    if (rc != MCA_OK) return rc;
    if (saved_bytes < p.saved || (p.saved > 0 && !saved))
        return mca::api_fail(("Saved-state buffer too small: " + std::to_string(saved_bytes) + " bytes given, " + std::to_string(p.saved) +
                              " needed")
                                 .c_str());
    unsigned char* sv = static_cast<unsigned char*>(saved);
    for (int64_t c = 0; c < p.nchunks; ++c)
    {
        const int64_t b0 = c * p.chunk, bc = chunk_at(p, c);
        for (int l = 0; l < n; ++l)
        {
            const mca_stack_layer& L = layers[l];
            const LayerPlan& lp = p.layers[l];
            const T* in = layer_input<T>(p, input, sv, l, b0);
            T* out = (l + 1 == n ? output : reinterpret_cast<T*>(sv + lp.act)) + b0 * p.ch[l + 1] * p.plane;
            const T* w = static_cast<const T*>(L.weight);
            if (L.kind == MCA_STACK_SMORPH)
            {
                const T* a = static_cast<const T*>(L.alpha);
                if constexpr (sizeof(T) == 4)
                {
                    if (lp.stats_chunk > 0)
                    {
                        float* st = reinterpret_cast<float*>(sv + lp.stats + c * lp.stats_chunk);
                        rc = mca_smorph_forward_stats_f32(L.merge, in, w, a, out, st, bc, lp.cin, L.out_channels, L.weight_channels, H, W, L.kh,
                                                          L.kw, stream);
                        if (rc != MCA_OK) return rc;
                        continue;
                    }
                }
                rc = Api<T>::sfwd(L.merge, in, w, a, out, bc, lp.cin, L.out_channels, L.weight_channels, H, W, L.kh, L.kw, stream);
            }
            else
            {
                void* idx = lp.idx_chunk > 0 ? sv + lp.idx + c * lp.idx_chunk : nullptr;
                rc = Api<T>::fwd(L.kind == MCA_STACK_DILATION ? mca::DILATION : mca::EROSION, L.merge, L.replicate, (T)L.fill, in, w, 0, out, idx,
                                 bc, lp.cin, L.out_channels, L.weight_channels, H, W, L.kh, L.kw, stream);
            }
            if (rc != MCA_OK) return rc;
        }
    }
    return MCA_OK;
}

template <typename T>
int stack_backward(const mca_stack_layer* layers, int n, const T* input, const T* output, const T* grad_output, T* grad_input, int64_t B,
                   int64_t C, int64_t H, int64_t W, int64_t chunk, const void* saved, size_t saved_bytes, void* workspace,
                   size_t workspace_bytes, void* stream)
{
    Plan p;
    int rc = make_plan<T>(layers, n, B, C, H, W, chunk, p);
    if (rc != MCA_OK) return rc;
    if (!p.backward_ok) return mca::api_fail("Structuring element too large for the smorph backward kernels' shared memory");
    if (saved_bytes < p.saved || (p.saved > 0 && !saved))
        return mca::api_fail(("Saved-state buffer too small: " + std::to_string(saved_bytes) + " bytes given, " + std::to_string(p.saved) +
                              " needed")
                                 .c_str());
    if (workspace_bytes < p.backward || (p.backward > 0 && !workspace))
        return mca::api_fail(("Workspace too small: " + std::to_string(workspace_bytes) + " bytes given, " + std::to_string(p.backward) +
                              " needed")
                                 .c_str());
    const hipStream_t st = (hipStream_t)stream;
    if (p.nchunks == 0)
    {
        // An empty batch: every wanted gradient is zero (the input's is empty).
        for (int l = 0; l < n; ++l)
        {
            if (layers[l].grad_weight && (rc = mca::api_hip_status(mca::fill_async<T>(static_cast<T*>(layers[l].grad_weight),
                                                                                       p.layers[l].wnumel, T(0), st))) != MCA_OK)
                return rc;
            if (layers[l].kind == MCA_STACK_SMORPH && layers[l].grad_alpha &&
                (rc = mca::api_hip_status(mca::fill_async<T>(static_cast<T*>(layers[l].grad_alpha), p.layers[l].npairs, T(0), st))) != MCA_OK)
                return rc;
        }
        return MCA_OK;
    }
    const unsigned char* sv = static_cast<const unsigned char*>(saved);
    unsigned char* ws = static_cast<unsigned char*>(workspace);
    T* gbuf[2] = {reinterpret_cast<T*>(ws + p.gbuf[0]), reinterpret_cast<T*>(ws + p.gbuf[1])};
    void* lws = ws + p.lws;
    T* part_w = reinterpret_cast<T*>(ws + p.part_w);
    T* part_a = reinterpret_cast<T*>(ws + p.part_a);
    const bool several = p.nchunks > 1;
    for (int64_t c = 0; c < p.nchunks; ++c)
    {
        const int64_t b0 = c * p.chunk, bc = chunk_at(p, c);
        for (int l = n - 1; l >= 0; --l)
        {
            const mca_stack_layer& L = layers[l];
            const LayerPlan& lp = p.layers[l];
            const T* in = layer_input<T>(p, input, sv, l, b0);
            const T* out = (l + 1 == n ? output : reinterpret_cast<const T*>(sv + lp.act)) + b0 * p.ch[l + 1] * p.plane;
            // The gradient of layer l's output, and where the gradient of its input goes: the chunk
            // buffers alternate by layer, the first layer writes grad_input (or a discarded buffer).
            const T* gout = l + 1 == n ? grad_output + b0 * p.ch[n] * p.plane : gbuf[l & 1];
            T* gin = l == 0 ? (grad_input ? grad_input + b0 * p.ch[0] * p.plane : gbuf[1]) : gbuf[(l - 1) & 1];
            T* gw = L.grad_weight && !several ? static_cast<T*>(L.grad_weight) : part_w;
            T* ga = L.grad_alpha && !several ? static_cast<T*>(L.grad_alpha) : part_a;
            const T* w = static_cast<const T*>(L.weight);
            if (L.kind == MCA_STACK_SMORPH)
            {
                const T* a = static_cast<const T*>(L.alpha);
                bool done = false;
                if constexpr (sizeof(T) == 4)
                {
                    if (lp.stats_chunk > 0)
                    {
                        const float* sst = reinterpret_cast<const float*>(sv + lp.stats + c * lp.stats_chunk);
                        rc = mca_smorph_backward_stats_f32(L.merge, in, w, a, out, sst, gout, gin, gw, ga, bc, lp.cin, L.out_channels,
                                                           L.weight_channels, H, W, L.kh, L.kw, lws, p.lws_bytes, stream);
                        done = true;
                    }
                }
                if (!done)
                    rc = Api<T>::sbwd(L.merge, in, w, a, out, gout, gin, gw, ga, bc, lp.cin, L.out_channels, L.weight_channels, H, W, L.kh,
                                      L.kw, lws, p.lws_bytes, stream);
            }
            else
            {
                const void* idx = lp.idx_chunk > 0 ? sv + lp.idx + c * lp.idx_chunk : nullptr;
                rc = Api<T>::bwd(L.kind == MCA_STACK_DILATION ? mca::DILATION : mca::EROSION, L.merge, L.replicate, (T)L.fill, in, w, 0, idx, gout,
                                 gin, gw, bc, lp.cin, L.out_channels, L.weight_channels, H, W, L.kh, L.kw, lws, p.lws_bytes, stream);
            }
            if (rc != MCA_OK) return rc;
            if (several && L.grad_weight &&
                (rc = mca::api_hip_status(mca::accumulate_async<T>(reinterpret_cast<double*>(ws + lp.acc_w), part_w, lp.wnumel, c == 0, st))) !=
                    MCA_OK)
                return rc;
            if (several && L.kind == MCA_STACK_SMORPH && L.grad_alpha &&
                (rc = mca::api_hip_status(mca::accumulate_async<T>(reinterpret_cast<double*>(ws + lp.acc_a), part_a, lp.npairs, c == 0, st))) !=
                    MCA_OK)
                return rc;
        }
    }
    for (int l = 0; l < n && several; ++l)
    {
        const mca_stack_layer& L = layers[l];
        const LayerPlan& lp = p.layers[l];
        if (L.grad_weight &&
            (rc = mca::api_hip_status(mca::round_async<T>(reinterpret_cast<const double*>(ws + lp.acc_w), static_cast<T*>(L.grad_weight),
                                                           lp.wnumel, st))) != MCA_OK)
            return rc;
        if (L.kind == MCA_STACK_SMORPH && L.grad_alpha &&
            (rc = mca::api_hip_status(mca::round_async<T>(reinterpret_cast<const double*>(ws + lp.acc_a), static_cast<T*>(L.grad_alpha),
                                                           lp.npairs, st))) != MCA_OK)
            return rc;
    }
    return MCA_OK;
}

}  // namespace

extern "C" {

int mca_stack_plan_f32(const mca_stack_layer* layers, int n, int64_t B, int64_t C, int64_t H, int64_t W, int64_t chunk, size_t* saved_bytes,
                       size_t* backward_bytes)
{
    return stack_plan<float>(layers, n, B, C, H, W, chunk, saved_bytes, backward_bytes);
}

int mca_stack_plan_f64(const mca_stack_layer* layers, int n, int64_t B, int64_t C, int64_t H, int64_t W, int64_t chunk, size_t* saved_bytes,
                       size_t* backward_bytes)
{
    return stack_plan<double>(layers, n, B, C, H, W, chunk, saved_bytes, backward_bytes);
}

int mca_stack_forward_f32(const mca_stack_layer* layers, int n, const float* input, float* output, int64_t B, int64_t C, int64_t H,
                          int64_t W, int64_t chunk, void* saved, size_t saved_bytes, void* stream)
{
    return stack_forward<float>(layers, n, input, output, B, C, H, W, chunk, saved, saved_bytes, stream);
}

int mca_stack_forward_f64(const mca_stack_layer* layers, int n, const double* input, double* output, int64_t B, int64_t C, int64_t H,
                          int64_t W, int64_t chunk, void* saved, size_t saved_bytes, void* stream)
{
    return stack_forward<double>(layers, n, input, output, B, C, H, W, chunk, saved, saved_bytes, stream);
}

int mca_stack_backward_f32(const mca_stack_layer* layers, int n, const float* input, const float* output, const float* grad_output,
                           float* grad_input, int64_t B, int64_t C, int64_t H, int64_t W, int64_t chunk, const void* saved,
                           size_t saved_bytes, void* workspace, size_t workspace_bytes, void* stream)
{
    return stack_backward<float>(layers, n, input, output, grad_output, grad_input, B, C, H, W, chunk, saved, saved_bytes, workspace,
                                 workspace_bytes, stream);
}

int mca_stack_backward_f64(const mca_stack_layer* layers, int n, const double* input, const double* output, const double* grad_output,
                           double* grad_input, int64_t B, int64_t C, int64_t H, int64_t W, int64_t chunk, const void* saved,
                           size_t saved_bytes, void* workspace, size_t workspace_bytes, void* stream)
{
    return stack_backward<double>(layers, n, input, output, grad_output, grad_input, B, C, H, W, chunk, saved, saved_bytes, workspace,
                                  workspace_bytes, stream);
}

}  // extern "C"
