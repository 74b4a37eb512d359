/*
 * morphocore_amd — C ABI of the MI355X (gfx950) morphology kernels.
 *
 * This is the drop-in boundary for morphocore's csrc hot path. Each entry point replaces one
 * device-level launcher of the reference extension (cited per function below; paths relative to the
 * reference repository root) and keeps its argument meaning:
 *   - tensors are dense row-major device pointers (NCHW), already contiguous;
 *   - x is [B, Cin, H, W]; the structuring element is [Cout, Cw, KH, KW] with Cw == Cin, or Cw == 1
 *     for the IDENTITY merge; with weight noise it is [B, Cout, Cw, KH, KW] and
 *     weight_batch_stride = Cout * Cw * KH * KW (0 for a shared structuring element);
 *   - outputs are [B, Cout, H, W]; packed indices are int32 (channel << 16) | (kh * KW + kw);
 *   - op: 0 dilation, 1 erosion; merge: 0 MAX, 1 MIN, 2 ADD ("sum"), 3 AVERAGE ("mean"),
 *     5 IDENTITY (4, SMOOTH, is not provided by this library); padding is resolved by the caller into
 *     `replicate` (clamped edge pixel) or a `fill` value (ZERO: 0, CONSTANT: the value, GEODESIC:
 *     -inf for dilation, +inf for erosion), as morpho_fill_value does
 *     (morphocore/functional/csrc/cpp/morpho_padding_policy.hpp:22-33);
 *   - `stream` is a hipStream_t (NULL: the null stream). Every call only enqueues work on it.
 *
 * Return value: 0 on success, MCA_ERR_INVALID for a rejected argument (the message mirrors the
 * reference's TORCH_CHECK text), MCA_ERR_HIP for a HIP runtime error. mca_last_error() returns the
 * calling thread's last message.
 *
 * Backward entry points take a caller-owned device workspace of at least the size the matching
 * *_workspace_size function returns; its contents on entry are irrelevant.
 */
#ifndef MORPHOCORE_AMD_H
#define MORPHOCORE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MCA_OK 0
#define MCA_ERR_INVALID 1
#define MCA_ERR_HIP 2

/* Library version string ("0.13.1-mi355x"). No reference counterpart (morphocore/__init__.py:1
 * holds the reference package's version). */
const char* mca_version(void);

/* Message of the calling thread's last failed call, "" if none. Stands in for the text of the
 * c10::Error the reference's TORCH_CHECKs raise. */
const char* mca_last_error(void);

/* Bytes of the winners ("indices") the forward can save for the backward, by merge:
 *   MAX / MIN: int32 (channel << 16) | tap per output pixel, [B, Cout, H, W], as the reference saves
 *     them (morphocore/functional/csrc/cpp/morpho_op_cpu_kernels.hxx:36-41; requires
 *     KH * KW < 65536 and Cin < 32768, morpho_op.cu:40-41);
 *   ADD / AVERAGE / IDENTITY: the first extremal tap kh * KW + kw of every channel pair,
 *     [B, Cout, Cpair, H, W] with Cpair = Cin (1 for IDENTITY), uint8 (uint16 when KH * KW > 256).
 *     The reference recomputes these in its backward (morpho_op_cpu_backward.hxx:90-156); saving
 *     them is this library's extension of the reference's save_indices flag.
 * No reference counterpart (the reference sizes its index tensor inline, morpho_op_wrap.hxx:85-88). */
size_t mca_morpho_indices_bytes(int merge, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW);

/* Dilation / erosion forward, every merge.
 * Replaces morpho_forward_cuda<op, T> (morphocore/functional/csrc/cuda/morpho_op.cuh:16-17,
 * morpho_op.cu:30-74). `indices` may be NULL, else it receives the winners described by
 * mca_morpho_indices_bytes. */
int mca_morpho_forward_f32(int op, int merge, int replicate, float fill, const float* input, const float* weight,
                           int64_t weight_batch_stride, float* output, void* indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw,
                           int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream);
int mca_morpho_forward_f64(int op, int merge, int replicate, double fill, const double* input, const double* weight,
                           int64_t weight_batch_stride, double* output, void* indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw,
                           int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream);

/* Workspace bytes mca_morpho_backward_* needs for this merge and geometry; has_indices says
 * whether saved indices will be passed. No reference counterpart: the reference allocates its
 * temporaries inside morpho_backward_cuda (morpho_op.cu:102-177) from torch's allocator. */
size_t mca_morpho_backward_workspace_size_f32(int merge, int has_indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H,
                                              int64_t W, int64_t KH, int64_t KW);
size_t mca_morpho_backward_workspace_size_f64(int merge, int has_indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H,
                                              int64_t W, int64_t KH, int64_t KW);

/* Dilation / erosion backward: overwrites grad_input [B, Cin, H, W] and grad_weight [Cout, Cw, KH, KW]
 * (summed over the batch when the structuring element is per batch element).
 * Replaces morpho_backward_cuda<op, T> (morphocore/functional/csrc/cuda/morpho_op.cuh:21-24,
 * morpho_op.cu:102-177). `indices` holds the forward's winners (see mca_morpho_indices_bytes) or is
 * NULL, in which case they are recomputed into the workspace. */
int mca_morpho_backward_f32(int op, int merge, int replicate, float fill, const float* input, const float* weight,
                            int64_t weight_batch_stride, const void* indices, const float* grad_output, float* grad_input,
                            float* grad_weight, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                            int64_t KW, void* workspace, size_t workspace_bytes, void* stream);
int mca_morpho_backward_f64(int op, int merge, int replicate, double fill, const double* input, const double* weight,
                            int64_t weight_batch_stride, const void* indices, const double* grad_output, double* grad_input,
                            double* grad_weight, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                            int64_t KW, void* workspace, size_t workspace_bytes, void* stream);

/* Dilation / erosion in float16 and bfloat16 (no reference counterpart: the reference's
 * "TODO: Add float16 support", morphocore/functional/csrc/cpp/morpho_op.cpp:7). Buffers hold IEEE
 * binary16 / bfloat16 bits; the arithmetic is float32 (every 16-bit value converts exactly) and each
 * stored result is rounded once to nearest even, so an output equals the float32 operator's on the
 * same values, rounded. `fill` is a float32. The forward reads and writes 16-bit data directly; the
 * backward converts grad_output to float32 in its workspace, routes it with the float32 kernels and
 * rounds grad_input and grad_weight once. Arguments otherwise as the f32 entry points. */
int mca_morpho_forward_f16(int op, int merge, int replicate, float fill, const uint16_t* input, const uint16_t* weight,
                           int64_t weight_batch_stride, uint16_t* output, void* indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw,
                           int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream);
int mca_morpho_forward_bf16(int op, int merge, int replicate, float fill, const uint16_t* input, const uint16_t* weight,
                            int64_t weight_batch_stride, uint16_t* output, void* indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw,
                            int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream);
size_t mca_morpho_backward_workspace_size_f16(int merge, int has_indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H,
                                              int64_t W, int64_t KH, int64_t KW);
size_t mca_morpho_backward_workspace_size_bf16(int merge, int has_indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H,
                                               int64_t W, int64_t KH, int64_t KW);
int mca_morpho_backward_f16(int op, int merge, int replicate, float fill, const uint16_t* input, const uint16_t* weight,
                            int64_t weight_batch_stride, const void* indices, const uint16_t* grad_output, uint16_t* grad_input,
                            uint16_t* grad_weight, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                            int64_t KW, void* workspace, size_t workspace_bytes, void* stream);
int mca_morpho_backward_bf16(int op, int merge, int replicate, float fill, const uint16_t* input, const uint16_t* weight,
                             int64_t weight_batch_stride, const void* indices, const uint16_t* grad_output, uint16_t* grad_input,
                             uint16_t* grad_weight, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                             int64_t KW, void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of device scratch each GPU holds for mca_morpho_backward_noalloc_f32 (64 MiB). */
#define MCA_NOALLOC_SCRATCH_BYTES (64u << 20)

/* Dilation / erosion backward (float32) that allocates nothing: mca_morpho_backward_f32 without the
 * workspace arguments. No counterpart in the reference; it is for callers that cannot allocate device
 * memory (code under stream capture, tight serving loops, harnesses that forbid hipMalloc). The
 * workspace is a file-scope device array of MCA_NOALLOC_SCRATCH_BYTES that each GPU holds from the
 * first call on it until the process ends; a problem whose workspace
 * (mca_morpho_backward_workspace_size_f32) exceeds it is rejected with MCA_ERR_INVALID. The stream
 * must belong to the current device. Every call on one GPU shares that GPU's scratch: calls that
 * overlap on one GPU (other streams, other host threads) race and must be serialised by the caller.
 * Outputs and argument meaning are those of mca_morpho_backward_f32. */
int mca_morpho_backward_noalloc_f32(int op, int merge, int replicate, float fill, const float* input, const float* weight,
                                    int64_t weight_batch_stride, const void* indices, const float* grad_output, float* grad_input,
                                    float* grad_weight, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W,
                                    int64_t KH, int64_t KW, void* stream);

/* Smorph forward. `weight` is the blended structuring element w~ the Python layer builds
 * (morphocore/functional/smorph.py:56-70); `alpha` holds one value per channel pair, index
 * o * Cin + i ([Cout] for IDENTITY), as smorph_pair_alphas expands it
 * (morphocore/functional/csrc/cpp/smorph_cpu_kernels.hxx:642-649).
 * Replaces smorph_forward_cuda<T> (morphocore/functional/csrc/cuda/smorph.cuh:15-16, smorph.cu:32-61). */
int mca_smorph_forward_f32(int merge, const float* input, const float* weight, const float* alpha, float* output, int64_t B, int64_t Cin,
                           int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream);
int mca_smorph_forward_f64(int merge, const double* input, const double* weight, const double* alpha, double* output, int64_t B,
                           int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream);

/* Workspace bytes mca_smorph_backward_* needs; 0 for an invalid geometry or a structuring element
 * too large for the backward kernels' shared memory (a caller that trains can check this before the
 * forward). No reference counterpart (the reference allocates inside smorph_backward_cuda,
 * smorph.cu:63-103). */
size_t mca_smorph_backward_workspace_size_f32(int merge, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W,
                                              int64_t KH, int64_t KW);
size_t mca_smorph_backward_workspace_size_f64(int merge, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W,
                                              int64_t KH, int64_t KW);

/* Smorph backward: overwrites grad_input, grad_weight (gradient of w~) and grad_alpha (one value per
 * channel pair, like `alpha`). `output` is the forward's output (the MAX / MIN merge target).
 * Replaces smorph_backward_cuda<T> (morphocore/functional/csrc/cuda/smorph.cuh:21-25, smorph.cu:63-103). */
int mca_smorph_backward_f32(int merge, const float* input, const float* weight, const float* alpha, const float* output,
                            const float* grad_output, float* grad_input, float* grad_weight, float* grad_alpha, int64_t B, int64_t Cin,
                            int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* workspace,
                            size_t workspace_bytes, void* stream);
int mca_smorph_backward_f64(int merge, const double* input, const double* weight, const double* alpha, const double* output,
                            const double* grad_output, double* grad_input, double* grad_weight, double* grad_alpha, int64_t B,
                            int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* workspace,
                            size_t workspace_bytes, void* stream);

/* Smorph with saved pair statistics (float32; square 3x3, 5x5, 7x7 and 11x11 elements). No reference
 * counterpart: the reference's backward recomputes each pair's softmax statistics from the saved
 * input (smorph.cu:63-103, smorph_cpu_kernels.hxx:387-638). The forward below also stores, for every
 * channel pair at every output pixel, the window's extremum, 1 / S and W / S (three float32 arrays of
 * B * Cout * P * H * W values, P = Cin, or 1 for IDENTITY; mca_smorph_stats_bytes_f32 bytes, 0 when
 * the configuration has no such path); the backward below reads them instead of recomputing them
 * (the same workspace as mca_smorph_backward_f32). The forward's output is bit for bit that of
 * mca_smorph_forward_f32; the gradients agree with mca_smorph_backward_f32's within the float32
 * tolerance (the two kernels add the same terms in different orders). */
size_t mca_smorph_stats_bytes_f32(int merge, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW);
int mca_smorph_forward_stats_f32(int merge, const float* input, const float* weight, const float* alpha, float* output, float* stats,
                                 int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW,
                                 void* stream);
int mca_smorph_backward_stats_f32(int merge, const float* input, const float* weight, const float* alpha, const float* output,
                                  const float* stats, const float* grad_output, float* grad_input, float* grad_weight, float* grad_alpha,
                                  int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* Smorph with the SMOOTH channel merge (the smorph_scm operator, selected by a `beta` in
 * morphocore/functional/smorph.py:72-73), float32 and float64, any structuring-element size.
 * Replaces smorph_forward_cuda / smorph_backward_cuda with merge SMOOTH and a beta
 * (morphocore/functional/csrc/cuda/smorph.cuh:15-25, smorph_kernels.cuh:247-298,512-523; the host
 * side is smorph_scm.cpp:13-96). For every output channel o and pixel, the pair outputs c_i of the
 * input channels (each as mca_smorph_forward computes it) are merged softly with beta[o]:
 * ref = the extremum of the c_i (max for beta >= 0, min otherwise), q_i = exp(beta[o] (c_i - ref)),
 * out = sum q_i c_i / sum q_i. alpha holds one value per pair (index o * Cin + i); Cw == Cin >= 1.
 * `merge_stats` receives (forward) and provides (backward) 2 * B * Cout * H * W values: ref, then
 * 1 / sum q_i, per output pixel; the forward may pass NULL when no backward follows. Both directions
 * take a caller-owned workspace of the size the matching function returns (0: invalid geometry, or,
 * for the backward, an element too large for the kernels' shared memory). The backward overwrites
 * grad_input, grad_weight (of w~), grad_alpha (per pair) and grad_beta [Cout]. */
size_t mca_smorph_scm_forward_workspace_size_f32(int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                                                 int64_t KW);
size_t mca_smorph_scm_forward_workspace_size_f64(int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                                                 int64_t KW);
int mca_smorph_scm_forward_f32(const float* input, const float* weight, const float* alpha, const float* beta, float* output,
                               float* merge_stats, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                               int64_t KW, void* workspace, size_t workspace_bytes, void* stream);
int mca_smorph_scm_forward_f64(const double* input, const double* weight, const double* alpha, const double* beta, double* output,
                               double* merge_stats, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                               int64_t KW, void* workspace, size_t workspace_bytes, void* stream);
size_t mca_smorph_scm_backward_workspace_size_f32(int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                                                  int64_t KW);
size_t mca_smorph_scm_backward_workspace_size_f64(int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                                                  int64_t KW);
int mca_smorph_scm_backward_f32(const float* input, const float* weight, const float* alpha, const float* beta, const float* output,
                                const float* merge_stats, const float* grad_output, float* grad_input, float* grad_weight, float* grad_alpha,
                                float* grad_beta, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                                int64_t KW, void* workspace, size_t workspace_bytes, void* stream);
int mca_smorph_scm_backward_f64(const double* input, const double* weight, const double* alpha, const double* beta, const double* output,
                                const double* merge_stats, const double* grad_output, double* grad_input, double* grad_weight,
                                double* grad_alpha, double* grad_beta, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H,
                                int64_t W, int64_t KH, int64_t KW, void* workspace, size_t workspace_bytes, void* stream);

/* Smorph with the SMOOTH channel merge and saved pair statistics (float32; square 3x3, 5x5, 7x7 and
 * 11x11 elements). No reference counterpart: the reference's backward recomputes each pair's softmax
 * statistics (smorph_kernels.cuh:512-523 with smorph_scm.cpp:36-96). The forward stores, for every
 * channel pair at every output pixel, the window's extremum, 1 / S and W / S (three float32 arrays of
 * B * Cout * Cin * H * W values, mca_smorph_scm_stats_bytes_f32 bytes, 0 when the configuration has no
 * such path), the last being the pair outputs the soft merge reads (no workspace); it also writes
 * merge_stats as mca_smorph_scm_forward_f32 does. The backward reads both instead of recomputing (the
 * workspace of mca_smorph_scm_backward_f32). Output bit for bit that of mca_smorph_scm_forward_f32;
 * gradients within the float32 tolerance of mca_smorph_scm_backward_f32's (the same terms added in
 * another order). */
size_t mca_smorph_scm_stats_bytes_f32(int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW);
int mca_smorph_scm_forward_stats_f32(const float* input, const float* weight, const float* alpha, const float* beta, float* output,
                                     float* merge_stats, float* pair_stats, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H,
                                     int64_t W, int64_t KH, int64_t KW, void* stream);
int mca_smorph_scm_backward_stats_f32(const float* input, const float* weight, const float* alpha, const float* beta, const float* output,
                                      const float* merge_stats, const float* pair_stats, const float* grad_output, float* grad_input,
                                      float* grad_weight, float* grad_alpha, float* grad_beta, int64_t B, int64_t Cin, int64_t Cout,
                                      int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW, void* workspace, size_t workspace_bytes,
                                      void* stream);

/* Per-sample structuring elements of weight noise in one pass: out[b][j] = weight[j] + (uniform[b][j] * 2
 * - 1) * scale for b < batch, j < n, with the roundings of the four elementwise operations the
 * reference composes it from (morphocore/functional/csrc/cpp/morpho_op_wrap.hxx:55-64: torch::rand's
 * draw, times 2, minus 1, times noise_scale, plus the shared weight), so the elements are bit for bit
 * those; `uniform` holds the caller's draw ([batch, n], in [0, 1)). For the forward launchers'
 * weight_batch_stride = n. */
int mca_noise_sample_weights_f32(const float* weight, const float* uniform, float scale, float* out, int64_t batch, int64_t n, void* stream);
int mca_noise_sample_weights_f64(const double* weight, const double* uniform, double scale, double* out, int64_t batch, int64_t n,
                                 void* stream);

/* Opening / closing with 'identity' merges in one pass (x to the final output per tile; the
 * intermediate image stays in on-chip memory). Replaces the two operator calls of
 * morphocore/functional/opening.py:96-101 (erosion, then dilation) and closing.py:96-101 (dilation,
 * then erosion) when both stages merge per channel, the form nn/opening.py:104-180 and
 * nn/closing.py build by default (one shared structuring element). first_op: MCA-level op of the first
 * stage (1 = erosion: opening; 0 = dilation: closing). w_first / w_second: [C, 1, K, K] as each
 * operator receives it (an erosion's element already flipped, as functional/erosion.py passes it), or
 * one per batch element, weight_batch_stride apart. fill_first / fill_second: the border value each
 * stage reads (its op's fill for the padding; unused with replicate). Output, tap by tap and value by
 * value, that of the two separate IDENTITY launches; taps_first / taps_second receive each stage's
 * first extremal tap per pixel ([B, C, H, W] bytes; both NULL when no backward follows). Square odd
 * elements 3x3, 5x5, 7x7 only (mca_morpho_pair_supported); others: run the two separate launches. */
int mca_morpho_pair_supported(int64_t KH, int64_t KW);
int mca_morpho_pair_forward_f32(int first_op, int replicate, float fill_first, float fill_second, const float* input, const float* w_first,
                                const float* w_second, int64_t weight_batch_stride, float* output, uint8_t* taps_first,
                                uint8_t* taps_second, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW, void* stream);
int mca_morpho_pair_forward_f64(int first_op, int replicate, double fill_first, double fill_second, const double* input,
                                const double* w_first, const double* w_second, int64_t weight_batch_stride, double* output,
                                uint8_t* taps_first, uint8_t* taps_second, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH,
                                int64_t KW, void* stream);

/* Backward of mca_morpho_pair_forward from its saved taps: grad_input [B, C, H, W] and the gradient of
 * each stage's element [C, 1, K, K] (in the frame the operator received it), all overwritten; the same
 * routing as the two separate IDENTITY backwards (a tap that read outside the image sends nothing to
 * its input; an element tap receives +g for a dilation, -g for an erosion). Workspace: the bytes
 * mca_morpho_pair_backward_workspace_size_* returns (0: unsupported). */
size_t mca_morpho_pair_backward_workspace_size_f32(int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW);
size_t mca_morpho_pair_backward_workspace_size_f64(int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW);
int mca_morpho_pair_backward_f32(int first_op, const uint8_t* taps_first, const uint8_t* taps_second, const float* grad_output,
                                 float* grad_input, float* grad_w_first, float* grad_w_second, int64_t B, int64_t C, int64_t H, int64_t W,
                                 int64_t KH, int64_t KW, void* workspace, size_t workspace_bytes, void* stream);
int mca_morpho_pair_backward_f64(int first_op, const uint8_t* taps_first, const uint8_t* taps_second, const double* grad_output,
                                 double* grad_input, double* grad_w_first, double* grad_w_second, int64_t B, int64_t C, int64_t H,
                                 int64_t W, int64_t KH, int64_t KW, void* workspace, size_t workspace_bytes, void* stream);

/* sigma_layer with the 'identity' merge in one pass: out = erosion(x) (1 - soft) + dilation(x) soft per
 * channel, with torch's roundings of that expression. Replaces the two operator calls and the blend of
 * morphocore/functional/sigma_layer.py:73-83 when the merge is 'identity' (soft = sigmoid(mean(alpha)),
 * [C], computed by the caller). w_erosion / w_dilation: [C, 1, K, K] as each operator receives its
 * element (the erosion's flipped, as functional/erosion.py passes it), or one per batch element,
 * weight_batch_stride apart. fill_erosion / fill_dilation: each operation's border value; they must
 * be equal, or the geodesic pair (+inf, -inf). taps_erosion / taps_dilation receive each operation's
 * first extremal tap ([B, C, H, W] bytes; both NULL when no backward follows). Square odd elements 3x3,
 * 5x5, 7x7 (mca_morpho_pair_supported). */
int mca_morpho_sigma_forward_f32(int replicate, float fill_erosion, float fill_dilation, const float* input, const float* w_erosion,
                                 const float* w_dilation, int64_t weight_batch_stride, const float* soft, float* output,
                                 uint8_t* taps_erosion, uint8_t* taps_dilation, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH,
                                 int64_t KW, void* stream);
int mca_morpho_sigma_forward_f64(int replicate, double fill_erosion, double fill_dilation, const double* input, const double* w_erosion,
                                 const double* w_dilation, int64_t weight_batch_stride, const double* soft, double* output,
                                 uint8_t* taps_erosion, uint8_t* taps_dilation, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH,
                                 int64_t KW, void* stream);

/* Backward of mca_morpho_sigma_forward from its saved taps: grad_input, the gradients of both
 * elements (in the frame each operator received) and grad_terms [2, C]: per channel the sum of
 * grad_output * erosion and of grad_output * dilation, from which the caller forms the gradient of soft
 * (their difference, dilation minus erosion). The routing is that of the two IDENTITY backwards with
 * grad_output (1 - soft) and grad_output soft; grad_input is their sum. Workspace:
 * mca_morpho_sigma_backward_workspace_size_* bytes (0: unsupported). */
size_t mca_morpho_sigma_backward_workspace_size_f32(int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW);
size_t mca_morpho_sigma_backward_workspace_size_f64(int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH, int64_t KW);
int mca_morpho_sigma_backward_f32(int replicate, float fill_erosion, float fill_dilation, const float* input, const float* w_erosion,
                                  const float* w_dilation, int64_t weight_batch_stride, const float* soft, const uint8_t* taps_erosion,
                                  const uint8_t* taps_dilation, const float* grad_output, float* grad_input, float* grad_w_erosion,
                                  float* grad_w_dilation, float* grad_terms, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH,
                                  int64_t KW, void* workspace, size_t workspace_bytes, void* stream);
int mca_morpho_sigma_backward_f64(int replicate, double fill_erosion, double fill_dilation, const double* input, const double* w_erosion,
                                  const double* w_dilation, int64_t weight_batch_stride, const double* soft, const uint8_t* taps_erosion,
                                  const uint8_t* taps_dilation, const double* grad_output, double* grad_input, double* grad_w_erosion,
                                  double* grad_w_dilation, double* grad_terms, int64_t B, int64_t C, int64_t H, int64_t W, int64_t KH,
                                  int64_t KW, void* workspace, size_t workspace_bytes, void* stream);

/* Layer stacks: a chain of dilation / erosion / smorph layers (configs such as dilation -> smorph ->
 * erosion) run forward and backward by one call each, batch chunk by batch chunk. Replaces the
 * reference's layer-by-layer composition of operator calls (morphocore/functional/dilation.py:89-91,
 * smorph.py:72-75, erosion.py:89-91, each a separate MorphoOperation / Smorph autograd node,
 * morpho_op_wrap.hxx:24-211, smorph.cpp:13-104). Each chunk of `chunk` batch elements goes through every
 * layer before the next chunk starts, and the backward keeps only one chunk of each intermediate
 * gradient (two chunk-sized buffers for the whole chain) instead of whole-batch tensors. Values and winners are
 * those of the separate entry points for the same layers; weight and alpha gradients are the chunks'
 * partial gradients summed in chunk order (in double, rounded once), within the tolerance of the
 * separate backward's.
 *
 * Layer l reads C_l channels (C_0 = the input's C) and writes out_channels = C_{l+1}; weight is
 * [out_channels, weight_channels, kh, kw] as the single-layer entry points take it (an erosion's
 * element already flipped, as functional/erosion.py passes it; a smorph's the blended w~), alpha one
 * value per pair (index o * C_l + i; [C_l] for IDENTITY). merge: MAX, MIN, ADD, AVERAGE, IDENTITY.
 * replicate / fill: the dilation's / erosion's border, as in mca_morpho_forward. save: keep what the
 * backward can reuse — a dilation's / erosion's winners (packed for MAX / MIN, per pair otherwise;
 * not kept when mca_morpho_forward could not save them), a float32 smorph's pair statistics (when
 * mca_smorph_stats_bytes_f32 has them for the layer); otherwise the backward recomputes. grad_weight
 * and grad_alpha are the backward's outputs for the layer (NULL: not wanted). */
#define MCA_STACK_DILATION 0
#define MCA_STACK_EROSION 1
#define MCA_STACK_SMORPH 2

typedef struct mca_stack_layer
{
    int kind;  /* MCA_STACK_DILATION, MCA_STACK_EROSION or MCA_STACK_SMORPH */
    int merge;
    int replicate;
    int save;
    double fill;
    int64_t out_channels, weight_channels, kh, kw;
    const void* weight;
    const void* alpha; /* smorph only */
    void* grad_weight;
    void* grad_alpha; /* smorph only */
} mca_stack_layer;

/* Validates the chain and sizes its buffers: *saved_bytes for what the forward keeps for the
 * backward (the activations between layers, the saved winners and statistics), *backward_bytes for the
 * backward's own workspace. chunk: batch elements per chunk, 0 = the whole batch (the fastest for
 * instruction-bound layers; smaller chunks bound the backward's intermediate gradient memory). The same
 * (layers, n, shape, chunk) must be passed to the forward and the backward. */
int mca_stack_plan_f32(const mca_stack_layer* layers, int n, int64_t B, int64_t C, int64_t H, int64_t W, int64_t chunk, size_t* saved_bytes,
                       size_t* backward_bytes);
int mca_stack_plan_f64(const mca_stack_layer* layers, int n, int64_t B, int64_t C, int64_t H, int64_t W, int64_t chunk, size_t* saved_bytes,
                       size_t* backward_bytes);
/* Forward of the chain: input [B, C, H, W] to output [B, C_n, H, W]; `saved` (saved_bytes) receives
 * the state the backward reads. */
int mca_stack_forward_f32(const mca_stack_layer* layers, int n, const float* input, float* output, int64_t B, int64_t C, int64_t H,
                          int64_t W, int64_t chunk, void* saved, size_t saved_bytes, void* stream);
int mca_stack_forward_f64(const mca_stack_layer* layers, int n, const double* input, double* output, int64_t B, int64_t C, int64_t H,
                          int64_t W, int64_t chunk, void* saved, size_t saved_bytes, void* stream);
/* Backward of the chain from the forward's input, output and saved state: grad_input [B, C, H, W]
 * (NULL: not wanted) and every layer's grad_weight / grad_alpha, all overwritten. */
int mca_stack_backward_f32(const mca_stack_layer* layers, int n, const float* input, const float* output, const float* grad_output,
                           float* grad_input, int64_t B, int64_t C, int64_t H, int64_t W, int64_t chunk, const void* saved,
                           size_t saved_bytes, void* workspace, size_t workspace_bytes, void* stream);
int mca_stack_backward_f64(const mca_stack_layer* layers, int n, const double* input, const double* output, const double* grad_output,
                           double* grad_input, int64_t B, int64_t C, int64_t H, int64_t W, int64_t chunk, const void* saved,
                           size_t saved_bytes, void* workspace, size_t workspace_bytes, void* stream);

/* Test probe, no reference counterpart: y[j] = the exponential every smorph kernel evaluates, applied
 * to x[j] (n values, device pointers). It restates the reference's vector exponential
 * (morphocore/functional/csrc/cpp/morpho_cpu_simd.hpp:127-169) for the arguments the kernels pass,
 * alpha (v - ref) <= 0 or NaN; the tests compare its bits with the oracle's. */
int mca_probe_smorph_exp_f32(const float* x, float* y, int64_t n, void* stream);
int mca_probe_smorph_exp_f64(const double* x, double* y, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MORPHOCORE_AMD_H */
