/*
 * Body of the CPU oracle, included once per element type by morpho_oracle.c with
 *   T       the element type (float or double),
 *   ACC     the accumulation type of gradient sums (double for float, long double for double),
 *   SFX     the symbol suffix (f32 or f64),
 *   T_LOWEST / T_MAX / T_INF  the numeric limits of T,
 *   EXP_T   the vector exponential restated from the reference (oracle_exp_f32 / oracle_exp_f64),
 *   FMA_T   the fused multiply-add of T (fmaf / fma), where the reference's AVX2 build fuses.
 *
 * TEST INFRASTRUCTURE ONLY. Scalar loops that restate, in the reference's own order of operations,
 * what the reference CPU extension computes. Forward values are computed in T with the reference's
 * operation order, so that max / min / identity outputs and indices are bit exact and sum / mean
 * outputs follow the same channel order. Gradient sums are accumulated in ACC: the reference's own
 * order of gradient accumulation depends on its thread count and scheduling
 * (morpho_op_cpu_kernels.hxx:132-142, morpho_op_cpu_backward.hxx:281-289), so the oracle uses a
 * near exact sum of the same per-term values instead.
 */

#define CAT_(a, b) a##_##b
#define CAT(a, b) CAT_(a, b)
#define FN(name) CAT(name, SFX)

/* Value read by tap (kh, kw) of output (h, w): the in-image pixel, the clamped edge pixel for
 * REPLICATE, the fill value otherwise. Restates morpho_pad_rows
 * (morpho_padding_policy.hpp:45-74) and the tap read rule of morpho_row_origin
 * (morpho_op_cpu_kernels.hxx:254-263): tap (kh, kw) reads input (h + pad_h - kh, w + pad_w - kw). */
static inline T FN(tap_read)(const T* plane, int64_t H, int64_t W, int64_t y, int64_t x, int replicate, T fill)
{
    if (y >= 0 && y < H && x >= 0 && x < W) return plane[y * W + x];
    if (!replicate) return fill;
    y = y < 0 ? 0 : (y >= H ? H - 1 : y);
    x = x < 0 ? 0 : (x >= W ? W - 1 : x);
    return plane[y * W + x];
}

/* Extremum of one (output, input) channel pair at one pixel, with the flat index of the first tap
 * reaching it. Restates morpho_block_extremum (morpho_op_cpu_kernels.hxx:211-252) and
 * MorphoPolicyCPU (morpho_op_policy.hpp:10-64): start at -inf (dilation) / +inf (erosion), visit taps
 * kh then kw, replace on a strict improvement only, so ties keep the first tap, NaN never wins and
 * the index stays 0 when no tap improves on the start value. */
static inline T FN(pair_extremum)(const T* plane, const T* wpair, const oracle_geom* g, int64_t h, int64_t w, int op, int replicate, T fill,
                                  int32_t* arg)
{
    const int64_t pad_h = g->kh / 2, pad_w = g->kw / 2;
    T best = op == ORACLE_DILATION ? -T_INF : T_INF;
    int32_t best_k = 0;
    int32_t k = 0;
    for (int64_t kh = 0; kh < g->kh; kh++)
    {
        for (int64_t kw = 0; kw < g->kw; kw++, k++)
        {
            const T xv = FN(tap_read)(plane, g->h, g->w, h + pad_h - kh, w + pad_w - kw, replicate, fill);
            const T v = op == ORACLE_DILATION ? xv + wpair[k] : xv - wpair[k];
            const int better = op == ORACLE_DILATION ? (v > best) : (v < best);
            if (better)
            {
                best = v;
                best_k = k;
            }
        }
    }
    *arg = best_k;
    return best;
}

/* Forward of dilation / erosion for every merge.
 * Restates MorphoForwardBands::run (morpho_op_cpu_forward.hxx:33-93), morpho_row_merge
 * (morpho_op_cpu_kernels.hxx:364-395) and MorphoMergePolicy (morpho_merge_policy.hpp:7-87):
 *   ADD / AVERAGE: m = 0, m = m + best_i in channel order, AVERAGE then m / Cin;
 *   MAX: m = lowest, m = std::max(m, best_i); MIN: m = max, m = std::min(m, best_i);
 *   IDENTITY: output channel o reads input channel o alone and writes its extremum;
 *   winner (MAX / MIN, when indices are requested): channel 0 first, then a channel that is
 *   strictly better than the running merge; the packed index is (channel << 16) | tap
 *   (morpho_op_cpu_kernels.hxx:36-41).
 * weight_batch_stride is 0 for a shared weight, Cout * Cw * KH * KW for one weight per batch element
 * (morpho_op_cpu_forward.hxx:123-148). */
int FN(oracle_morpho_forward)(int op, int merge, int replicate, T fill, const T* x, const T* wt, int64_t weight_batch_stride, T* out,
                              int32_t* indices, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH,
                              int64_t KW)
{
    oracle_geom g = {B, Cin, Cout, Cw, H, W, KH, KW};
    const int64_t taps = KH * KW;
    const int identity = merge == ORACLE_IDENTITY;
    if (identity && (Cout != Cin || Cw != 1)) return 1;
    if (!identity && Cw != Cin) return 1;
    if (indices && !(merge == ORACLE_MAX || merge == ORACLE_MIN)) return 1;
    if (indices && !(taps < (1 << 16) && Cin < (1 << 15))) return 1;

#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int64_t b = 0; b < B; b++)
    {
        for (int64_t o = 0; o < Cout; o++)
        {
            const T* wout = wt + b * weight_batch_stride + o * Cw * taps;
            for (int64_t h = 0; h < H; h++)
            {
                for (int64_t w = 0; w < W; w++)
                {
                    const int64_t oi = ((b * Cout + o) * H + h) * W + w;
                    int32_t arg;
                    if (identity)
                    {
                        out[oi] = FN(pair_extremum)(x + (b * Cin + o) * H * W, wout, &g, h, w, op, replicate, fill, &arg);
                        continue;
                    }
                    T m = merge == ORACLE_MAX ? T_LOWEST : (merge == ORACLE_MIN ? T_MAX : (T)0);
                    int32_t winner = 0;
                    for (int64_t i = 0; i < Cin; i++)
                    {
                        const T best = FN(pair_extremum)(x + (b * Cin + i) * H * W, wout + i * taps, &g, h, w, op, replicate, fill, &arg);
                        if (merge == ORACLE_MAX)
                        {
                            if (i == 0 || best > m) winner = (int32_t)((i << 16) | arg);
                            m = (m < best) ? best : m; /* std::max(m, best) */
                        }
                        else if (merge == ORACLE_MIN)
                        {
                            if (i == 0 || best < m) winner = (int32_t)((i << 16) | arg);
                            m = (best < m) ? best : m; /* std::min(m, best) */
                        }
                        else
                        {
                            m = m + best;
                        }
                    }
                    out[oi] = merge == ORACLE_AVERAGE ? m / (T)Cin : m;
                    if (indices) indices[oi] = winner;
                }
            }
        }
    }
    return 0;
}

/* Backward of dilation / erosion.
 * MAX / MIN restate MorphoBackwardBands::run_single_winner (morpho_op_cpu_backward.hxx:42-88): the
 * whole output gradient goes to the winning (channel, tap), to grad_input when the tap read an
 * in-image pixel (never to the copied edge pixel of REPLICATE) and to grad_weight with sign +1
 * (dilation) or -1 (erosion); zero gradients are skipped. The winners come from `indices` when given,
 * else they are recomputed as the forward does.
 * ADD / AVERAGE / IDENTITY restate run_per_pair (morpho_op_cpu_backward.hxx:94-156): every pair routes
 * grad * scale to its own first extremal tap, scale = (T)1 / Cin for AVERAGE
 * (morpho_op_cpu_backward.hxx:268), 1 otherwise. grad_weight has the shared [Cout, Cw, KH, KW] shape
 * and sums over the batch when the weight is per batch element.
 * grad_input and grad_weight are overwritten. */
int FN(oracle_morpho_backward)(int op, int merge, int replicate, T fill, const T* x, const T* wt, int64_t weight_batch_stride,
                               const int32_t* indices, const T* grad_out, T* grad_in, T* grad_w, int64_t B, int64_t Cin, int64_t Cout,
                               int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    oracle_geom g = {B, Cin, Cout, Cw, H, W, KH, KW};
    const int64_t taps = KH * KW, pad_h = KH / 2, pad_w = KW / 2, plane = H * W;
    const int identity = merge == ORACLE_IDENTITY;
    const int single_winner = merge == ORACLE_MAX || merge == ORACLE_MIN;
    const T sign = op == ORACLE_DILATION ? (T)1 : (T)-1;
    const T scale = merge == ORACLE_AVERAGE ? (T)1.0 / (T)Cin : (T)1.0;
    if (identity && (Cout != Cin || Cw != 1)) return 1;
    if (!identity && Cw != Cin) return 1;
    const int64_t wnumel = Cout * Cw * taps;

    ACC* gx_acc = (ACC*)calloc((size_t)(B * Cin * plane), sizeof(ACC));
    ACC* gw_part = (ACC*)calloc((size_t)(B * wnumel), sizeof(ACC));
    int32_t* winners = NULL;
    if (!gx_acc || !gw_part) return 2;
    if (single_winner && !indices)
    {
        winners = (int32_t*)malloc((size_t)(B * Cout * plane) * sizeof(int32_t));
        T* scratch = (T*)malloc((size_t)(B * Cout * plane) * sizeof(T));
        if (!winners || !scratch) return 2;
        FN(oracle_morpho_forward)(op, merge, replicate, fill, x, wt, weight_batch_stride, scratch, winners, B, Cin, Cout, Cw, H, W, KH, KW);
        free(scratch);
        indices = winners;
    }

    /* Batch elements own disjoint grad_input planes and their own grad_weight partial. */
#pragma omp parallel for schedule(dynamic)
    for (int64_t b = 0; b < B; b++)
    {
        ACC* gw = gw_part + b * wnumel;
        for (int64_t o = 0; o < Cout; o++)
        {
            const T* wout = wt + b * weight_batch_stride + o * Cw * taps;
            for (int64_t h = 0; h < H; h++)
            {
                for (int64_t w = 0; w < W; w++)
                {
                    const int64_t oi = ((b * Cout + o) * H + h) * W + w;
                    if (single_winner)
                    {
                        const T grad = grad_out[oi];
                        if (grad == (T)0) continue;
                        const int64_t c = indices[oi] >> 16, k = indices[oi] & 0xFFFF;
                        const int64_t ih = h + pad_h - k / KW, iw = w + pad_w - k % KW;
                        if (ih >= 0 && ih < H && iw >= 0 && iw < W) gx_acc[(b * Cin + c) * plane + ih * W + iw] += (ACC)grad;
                        gw[(o * Cw + c) * taps + k] += (ACC)(sign * grad);
                        continue;
                    }
                    const T grad = grad_out[oi] * scale;
                    const int64_t i_begin = identity ? o : 0, i_end = identity ? o + 1 : Cin;
                    for (int64_t i = i_begin; i < i_end; i++)
                    {
                        const int64_t wi = identity ? 0 : i;
                        int32_t k;
                        FN(pair_extremum)(x + (b * Cin + i) * plane, wout + wi * taps, &g, h, w, op, replicate, fill, &k);
                        const int64_t ih = h + pad_h - k / KW, iw = w + pad_w - k % KW;
                        if (ih >= 0 && ih < H && iw >= 0 && iw < W) gx_acc[(b * Cin + i) * plane + ih * W + iw] += (ACC)grad;
                        gw[(o * Cw + wi) * taps + k] += (ACC)(sign * grad);
                    }
                }
            }
        }
    }

    for (int64_t j = 0; j < B * Cin * plane; j++) grad_in[j] = (T)gx_acc[j];
    for (int64_t j = 0; j < wnumel; j++)
    {
        ACC s = 0;
        for (int64_t b = 0; b < B; b++) s += gw_part[b * wnumel + j];
        grad_w[j] = (T)s;
    }
    free(gx_acc);
    free(gw_part);
    free(winners);
    return 0;
}

/* Soft extremum of one channel pair at one pixel, over the taps that read an in-image pixel.
 * Restates smorph_block_forward (smorph_cpu_kernels.hxx:75-147) with smorph_valid_rows (:62-66) and
 * SmorphBlockMask (:32-59): ref = max v (alpha >= 0) or min v, strict replacement from -inf / +inf;
 * e = exp((v - ref) * alpha) with the reference's vector exponential; S = sum e, W = sum e * v in tap
 * order (fused); out = W * (1 / S). When `exps` is given it receives e per tap, 0 for excluded taps.
 * *weighted_out receives W, which the ADD / AVERAGE merges fuse into the running sum. */
static inline T FN(smorph_pair)(const T* plane, const T* wpair, T alpha, const oracle_geom* g, int64_t h, int64_t w, T* ref_out, T* inv_out,
                                T* exps, T* weighted_out)
{
    const int64_t pad_h = g->kh / 2, pad_w = g->kw / 2;
    int64_t kh_begin = h + pad_h - (g->h - 1);
    if (kh_begin < 0) kh_begin = 0;
    int64_t kh_end = h + pad_h + 1;
    if (kh_end > g->kh) kh_end = g->kh;
    const int dilation_like = alpha >= (T)0;

    T ref = dilation_like ? -T_INF : T_INF;
    for (int64_t kh = kh_begin; kh < kh_end; kh++)
    {
        const T* row = plane + (h + pad_h - kh) * g->w;
        for (int64_t kw = 0; kw < g->kw; kw++)
        {
            const int64_t col = w + pad_w - kw;
            if (col < 0 || col >= g->w) continue;
            const T v = row[col] + wpair[kh * g->kw + kw];
            if (dilation_like ? (v > ref) : (v < ref)) ref = v;
        }
    }
    if (exps)
        for (int64_t k = 0; k < g->kh * g->kw; k++) exps[k] = (T)0;
    T sum = (T)0, weighted = (T)0;
    for (int64_t kh = kh_begin; kh < kh_end; kh++)
    {
        const T* row = plane + (h + pad_h - kh) * g->w;
        for (int64_t kw = 0; kw < g->kw; kw++)
        {
            const int64_t col = w + pad_w - kw;
            if (col < 0 || col >= g->w) continue;
            const T v = row[col] + wpair[kh * g->kw + kw];
            const T e = EXP_T((v - ref) * alpha);
            sum = sum + e;
            weighted = FMA_T(e, v, weighted);
            if (exps) exps[kh * g->kw + kw] = e;
        }
    }
    const T inv = (T)1 / sum;
    *ref_out = ref;
    *inv_out = inv;
    if (weighted_out) *weighted_out = weighted;
    return weighted * inv;
}

/* Forward of smorph: SmorphForwardBands::run (smorph_cpu_kernels.hxx:308-380) with the merges of
 * smorph_merge (:210-229) and the AVERAGE finalisation m / Cin. alpha holds one value per pair,
 * index o * Cin + i, or o for IDENTITY (smorph_alpha_index, :283-287). */
int FN(oracle_smorph_forward)(int merge, const T* x, const T* wt, const T* alpha, T* out, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw,
                              int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    oracle_geom g = {B, Cin, Cout, Cw, H, W, KH, KW};
    const int64_t taps = KH * KW, plane = H * W;
    const int identity = merge == ORACLE_IDENTITY;
    if (identity && (Cout != Cin || Cw != 1)) return 1;
    if (!identity && Cw != Cin) return 1;

#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int64_t b = 0; b < B; b++)
    {
        for (int64_t o = 0; o < Cout; o++)
        {
            for (int64_t h = 0; h < H; h++)
            {
                for (int64_t w = 0; w < W; w++)
                {
                    T ref, inv, weighted;
                    const int64_t oi = ((b * Cout + o) * H + h) * W + w;
                    if (identity)
                    {
                        out[oi] = FN(smorph_pair)(x + (b * Cin + o) * plane, wt + o * taps, alpha[o], &g, h, w, &ref, &inv, NULL, NULL);
                        continue;
                    }
                    T m = merge == ORACLE_MAX ? T_LOWEST : (merge == ORACLE_MIN ? T_MAX : (T)0);
                    for (int64_t i = 0; i < Cin; i++)
                    {
                        const T c = FN(smorph_pair)(x + (b * Cin + i) * plane, wt + (o * Cin + i) * taps, alpha[o * Cin + i], &g, h, w, &ref, &inv,
                                                    NULL, &weighted);
                        if (merge == ORACLE_MAX)
                            m = m < c ? c : m;
                        else if (merge == ORACLE_MIN)
                            m = c < m ? c : m;
                        else
                            m = FMA_T(weighted, inv, m); /* merged + W * (1 / S), fused */
                    }
                    out[oi] = merge == ORACLE_AVERAGE ? m / (T)Cin : m;
                }
            }
        }
    }
    return 0;
}

/* Backward of smorph: SmorphBackwardBands::run (smorph_cpu_kernels.hxx:420-603) with
 * smorph_block_backward (:157-206). For each pixel, g = grad * scale (scale = (T)1 / Cin for
 * AVERAGE). MAX / MIN first recompute every channel output, take the hard extremum of the channels
 * (channel 0, then strictly better ones) and split g equally between the channels within 1e-6 of it
 * (is_winner, :622-627). Each routed pair recomputes its forward with exps, then per tap, kw outer and
 * kh inner over the valid rows:
 *   pg = e * (g * inv_sum), centered = v - out, c = pg + alpha * pg * centered,
 *   grad_input[read pixel] += c, grad_weight[k] += c,
 *   grad_alpha += pg * (v - ref) * centered on in-image taps.
 * grad_alpha has one value per pair (index as in oracle_smorph_forward). All outputs overwritten. */
int FN(oracle_smorph_backward)(int merge, const T* x, const T* wt, const T* alpha, const T* grad_out, T* grad_in, T* grad_w, T* grad_alpha,
                               int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    oracle_geom g = {B, Cin, Cout, Cw, H, W, KH, KW};
    const int64_t taps = KH * KW, plane = H * W, pad_h = KH / 2, pad_w = KW / 2;
    const int identity = merge == ORACLE_IDENTITY;
    const int winner_takes_all = merge == ORACLE_MAX || merge == ORACLE_MIN;
    const T scale = merge == ORACLE_AVERAGE ? (T)1.0 / (T)Cin : (T)1.0;
    const T tol = (T)1e-6;
    if (identity && (Cout != Cin || Cw != 1)) return 1;
    if (!identity && Cw != Cin) return 1;
    const int64_t wnumel = Cout * Cw * taps;
    const int64_t anumel = identity ? Cout : Cout * Cin;

    const int nthreads = omp_get_max_threads();
    const int64_t gx_numel = B * Cin * plane;
    /* One grad_input accumulator per thread: the (b, o) units of different threads add to the same
     * input pixels. Summed in thread order at the end. */
    ACC* gx_thr = (ACC*)calloc((size_t)(nthreads * gx_numel), sizeof(ACC));
    ACC* gw_part = (ACC*)calloc((size_t)(B * wnumel), sizeof(ACC));
    ACC* ga_part = (ACC*)calloc((size_t)(B * anumel), sizeof(ACC));
    if (!gx_thr || !gw_part || !ga_part) return 2;

#pragma omp parallel
    {
        T* exps = (T*)malloc((size_t)taps * sizeof(T));
        T* outs = (T*)malloc((size_t)Cin * sizeof(T));
        ACC* gx_acc = gx_thr + (int64_t)omp_get_thread_num() * gx_numel;
#pragma omp for collapse(2) schedule(dynamic)
        for (int64_t b = 0; b < B; b++)
        {
          for (int64_t o_unit = 0; o_unit < Cout; o_unit++)
          {
            /* grad_weight and grad_alpha of the pairs of output channel o_unit belong to this unit alone. */
            ACC* gw = gw_part + b * wnumel;
            ACC* ga = ga_part + b * anumel;
            {
                const int64_t o = o_unit;
                for (int64_t h = 0; h < H; h++)
                {
                    int64_t kh_begin = h + pad_h - (H - 1);
                    if (kh_begin < 0) kh_begin = 0;
                    int64_t kh_end = h + pad_h + 1;
                    if (kh_end > KH) kh_end = KH;
                    for (int64_t w = 0; w < W; w++)
                    {
                        T grad = grad_out[((b * Cout + o) * H + h) * W + w] * scale;
                        T target = 0;
                        if (winner_takes_all)
                        {
                            for (int64_t i = 0; i < Cin; i++)
                            {
                                T ref, inv;
                                outs[i] = FN(smorph_pair)(x + (b * Cin + i) * plane, wt + (o * Cin + i) * taps, alpha[o * Cin + i], &g, h, w, &ref,
                                                          &inv, NULL, NULL);
                                if (i == 0)
                                    target = outs[i];
                                else if (merge == ORACLE_MAX)
                                    target = outs[i] > target ? outs[i] : target;
                                else
                                    target = outs[i] < target ? outs[i] : target;
                            }
                            T winners = 0;
                            for (int64_t i = 0; i < Cin; i++)
                            {
                                const T d = outs[i] - target;
                                if (d < tol && d > -tol) winners = winners + (T)1;
                            }
                            grad = grad / (winners > (T)0 ? winners : (T)1);
                        }
                        const int64_t i_begin = identity ? o : 0, i_end = identity ? o + 1 : Cin;
                        for (int64_t i = i_begin; i < i_end; i++)
                        {
                            T pair_grad = grad;
                            if (winner_takes_all)
                            {
                                const T d = outs[i] - target;
                                pair_grad = (d < tol && d > -tol) ? grad : (T)0;
                            }
                            const int64_t wi = identity ? 0 : i;
                            const int64_t ai = identity ? o : o * Cin + i;
                            const T a = alpha[ai];
                            const T* pl = x + (b * Cin + i) * plane;
                            const T* wp = wt + (o * Cw + wi) * taps;
                            T ref, inv;
                            const T out = FN(smorph_pair)(pl, wp, a, &g, h, w, &ref, &inv, exps, NULL);
                            const T scaled = pair_grad * inv;
                            ACC alpha_sum = 0;
                            for (int64_t kw = 0; kw < KW; kw++)
                            {
                                for (int64_t kh = kh_begin; kh < kh_end; kh++)
                                {
                                    const int64_t k = kh * KW + kw;
                                    const int64_t ih = h + pad_h - kh, iw = w + pad_w - kw;
                                    if (iw < 0 || iw >= W) continue; /* e = 0 there: c = 0 */
                                    const T v = pl[ih * W + iw] + wp[k];
                                    const T pg = exps[k] * scaled;
                                    const T centered = v - out;
                                    const T c = FMA_T(a * pg, centered, pg); /* pg + alpha * pg * centered, fused */
                                    gx_acc[(b * Cin + i) * plane + ih * W + iw] += (ACC)c;
                                    gw[(o * Cw + wi) * taps + k] += (ACC)TERM(c);
                                    alpha_sum += (ACC)TERM(pg * (v - ref) * centered);
                                }
                            }
                            ga[ai] += alpha_sum;
                        }
                    }
                }
            }
          }
        }
        free(exps);
        free(outs);
    }

    for (int64_t j = 0; j < gx_numel; j++)
    {
        ACC sx = 0;
        for (int t = 0; t < nthreads; t++) sx += gx_thr[(int64_t)t * gx_numel + j];
        grad_in[j] = (T)sx;
    }
    for (int64_t j = 0; j < wnumel; j++)
    {
        ACC s = 0;
        for (int64_t b = 0; b < B; b++) s += gw_part[b * wnumel + j];
        grad_w[j] = (T)s;
    }
    for (int64_t j = 0; j < anumel; j++)
    {
        ACC s = 0;
        for (int64_t b = 0; b < B; b++) s += ga_part[b * anumel + j];
        grad_alpha[j] = (T)s;
    }
    free(gx_thr);
    free(gw_part);
    free(ga_part);
    return 0;
}

/* Soft extremum over the channels of one pixel, the SMOOTH merge: smorph_soft_merge
 * (smorph_cpu_kernels.hxx:231-266). ref starts at channel 0 and takes each later channel that is
 * strictly greater (beta >= 0) or smaller (beta < 0); q_i = exp((c_i - ref) * beta) with the
 * reference's vector exponential; sum = sum q_i and weighted = sum q_i c_i (fused) in channel order;
 * merged = weighted * (1 / sum). */
static inline T FN(soft_merge)(const T* c, int64_t n, T beta, T* ref_out, T* inv_out)
{
    const int max_like = beta >= (T)0;
    T ref = c[0];
    for (int64_t i = 1; i < n; i++)
        if (max_like ? (c[i] > ref) : (c[i] < ref)) ref = c[i];
    T sum = (T)0, weighted = (T)0;
    for (int64_t i = 0; i < n; i++)
    {
        const T q = EXP_T((c[i] - ref) * beta);
        sum = sum + q;
        weighted = FMA_T(q, c[i], weighted);
    }
    const T inv = (T)1 / sum;
    *ref_out = ref;
    *inv_out = inv;
    return weighted * inv;
}

/* Forward of smorph with the SMOOTH channel merge (the smorph_scm operator): SmorphForwardBands::run
 * (smorph_cpu_kernels.hxx:308-380) stores the pair output c_i of every input channel, then
 * smorph_soft_merge merges them with the output channel's beta (no AVERAGE division). alpha holds one
 * value per pair, index o * Cin + i (smorph_pair_alphas<SMOOTH>, :642-649); beta one per output
 * channel. */
int FN(oracle_smorph_scm_forward)(const T* x, const T* wt, const T* alpha, const T* beta, T* out, int64_t B, int64_t Cin, int64_t Cout,
                                  int64_t Cw, int64_t H, int64_t W, int64_t KH, int64_t KW)
{
    oracle_geom g = {B, Cin, Cout, Cw, H, W, KH, KW};
    const int64_t taps = KH * KW, plane = H * W;
    if (Cw != Cin || Cin < 1) return 1;

#pragma omp parallel
    {
        T* outs = (T*)malloc((size_t)Cin * sizeof(T));
#pragma omp for collapse(2) schedule(dynamic)
        for (int64_t b = 0; b < B; b++)
        {
            for (int64_t o = 0; o < Cout; o++)
            {
                for (int64_t h = 0; h < H; h++)
                {
                    for (int64_t w = 0; w < W; w++)
                    {
                        T ref, inv;
                        for (int64_t i = 0; i < Cin; i++)
                            outs[i] = FN(smorph_pair)(x + (b * Cin + i) * plane, wt + (o * Cin + i) * taps, alpha[o * Cin + i], &g, h, w, &ref, &inv,
                                                      NULL, NULL);
                        out[((b * Cout + o) * H + h) * W + w] = FN(soft_merge)(outs, Cin, beta[o], &ref, &inv);
                    }
                }
            }
        }
        free(outs);
    }
    return 0;
}

/* Backward of smorph_scm: SmorphBackwardBands::run with soft_merge (smorph_cpu_kernels.hxx:420-603).
 * For each pixel (g = grad, no scaling): recompute every channel's pair output c_i and the soft merge
 * (ref, 1 / sum, final); channel i receives
 *   p_i = exp((c_i - ref) * beta) * (1 / sum),  g_i = g * (p_i + beta * p_i * (c_i - final)) (fused),
 * and routes g_i through its pair exactly as the ADD merge routes g (oracle_smorph_backward), while
 *   grad_beta[o] += p_i * (c_i - ref) * (c_i - final) * g.
 * grad_alpha has one value per pair, grad_beta one per output channel. All outputs overwritten. */
int FN(oracle_smorph_scm_backward)(const T* x, const T* wt, const T* alpha, const T* beta, const T* grad_out, T* grad_in, T* grad_w,
                                   T* grad_alpha, T* grad_beta, int64_t B, int64_t Cin, int64_t Cout, int64_t Cw, int64_t H, int64_t W,
                                   int64_t KH, int64_t KW)
{
    oracle_geom g = {B, Cin, Cout, Cw, H, W, KH, KW};
    const int64_t taps = KH * KW, plane = H * W, pad_h = KH / 2, pad_w = KW / 2;
    if (Cw != Cin || Cin < 1) return 1;
    const int64_t wnumel = Cout * Cw * taps;
    const int64_t anumel = Cout * Cin;

    const int nthreads = omp_get_max_threads();
    const int64_t gx_numel = B * Cin * plane;
    /* One grad_input accumulator per thread: the (b, o) units of different threads add to the same
     * input pixels. Summed in thread order at the end. */
    ACC* gx_thr = (ACC*)calloc((size_t)(nthreads * gx_numel), sizeof(ACC));
    ACC* gw_part = (ACC*)calloc((size_t)(B * wnumel), sizeof(ACC));
    ACC* ga_part = (ACC*)calloc((size_t)(B * anumel), sizeof(ACC));
    ACC* gb_part = (ACC*)calloc((size_t)(B * Cout), sizeof(ACC));
    if (!gx_thr || !gw_part || !ga_part || !gb_part) return 2;

#pragma omp parallel
    {
        T* exps = (T*)malloc((size_t)taps * sizeof(T));
        T* outs = (T*)malloc((size_t)Cin * sizeof(T));
        ACC* gx_acc = gx_thr + (int64_t)omp_get_thread_num() * gx_numel;
#pragma omp for collapse(2) schedule(dynamic)
        for (int64_t b = 0; b < B; b++)
        {
          for (int64_t o_unit = 0; o_unit < Cout; o_unit++)
          {
            /* grad_weight and grad_alpha of the pairs of output channel o_unit belong to this unit alone. */
            ACC* gw = gw_part + b * wnumel;
            ACC* ga = ga_part + b * anumel;
            ACC* gb = gb_part + b * Cout;
            {
                const int64_t o = o_unit;
                const T bt = beta[o];
                for (int64_t h = 0; h < H; h++)
                {
                    int64_t kh_begin = h + pad_h - (H - 1);
                    if (kh_begin < 0) kh_begin = 0;
                    int64_t kh_end = h + pad_h + 1;
                    if (kh_end > KH) kh_end = KH;
                    for (int64_t w = 0; w < W; w++)
                    {
                        const T grad = grad_out[((b * Cout + o) * H + h) * W + w];
                        for (int64_t i = 0; i < Cin; i++)
                        {
                            T ref, inv;
                            outs[i] = FN(smorph_pair)(x + (b * Cin + i) * plane, wt + (o * Cin + i) * taps, alpha[o * Cin + i], &g, h, w, &ref, &inv,
                                                      NULL, NULL);
                        }
                        T sref, sinv;
                        const T fin = FN(soft_merge)(outs, Cin, bt, &sref, &sinv);
                        for (int64_t i = 0; i < Cin; i++)
                        {
                            const T c = outs[i];
                            const T p = EXP_T((c - sref) * bt) * sinv;
                            gb[o] += (ACC)TERM(p * (c - sref) * (c - fin) * grad);
                        }
                        for (int64_t i = 0; i < Cin; i++)
                        {
                            const T c = outs[i];
                            const T p = EXP_T((c - sref) * bt) * sinv;
                            const T pair_grad = grad * FMA_T(bt * p, c - fin, p); /* g * (p + beta * p * (c - final)), fused */
                            const int64_t ai = o * Cin + i;
                            const T a = alpha[ai];
                            const T* pl = x + (b * Cin + i) * plane;
                            const T* wp = wt + (o * Cw + i) * taps;
                            T ref, pinv;
                            const T out = FN(smorph_pair)(pl, wp, a, &g, h, w, &ref, &pinv, exps, NULL);
                            const T scaled = pair_grad * pinv;
                            ACC alpha_sum = 0;
                            for (int64_t kw = 0; kw < KW; kw++)
                            {
                                for (int64_t kh = kh_begin; kh < kh_end; kh++)
                                {
                                    const int64_t k = kh * KW + kw;
                                    const int64_t ih = h + pad_h - kh, iw = w + pad_w - kw;
                                    if (iw < 0 || iw >= W) continue;
                                    const T v = pl[ih * W + iw] + wp[k];
                                    const T pg = exps[k] * scaled;
                                    const T centered = v - out;
                                    const T cc = FMA_T(a * pg, centered, pg);
                                    gx_acc[(b * Cin + i) * plane + ih * W + iw] += (ACC)cc;
                                    gw[(o * Cw + i) * taps + k] += (ACC)TERM(cc);
                                    alpha_sum += (ACC)TERM(pg * (v - ref) * centered);
                                }
                            }
                            ga[ai] += alpha_sum;
                        }
                    }
                }
            }
          }
        }
        free(exps);
        free(outs);
    }

    for (int64_t j = 0; j < gx_numel; j++)
    {
        ACC sx = 0;
        for (int t = 0; t < nthreads; t++) sx += gx_thr[(int64_t)t * gx_numel + j];
        grad_in[j] = (T)sx;
    }
    for (int64_t j = 0; j < wnumel; j++)
    {
        ACC s = 0;
        for (int64_t b = 0; b < B; b++) s += gw_part[b * wnumel + j];
        grad_w[j] = (T)s;
    }
    for (int64_t j = 0; j < anumel; j++)
    {
        ACC s = 0;
        for (int64_t b = 0; b < B; b++) s += ga_part[b * anumel + j];
        grad_alpha[j] = (T)s;
    }
    for (int64_t o = 0; o < Cout; o++)
    {
        ACC s = 0;
        for (int64_t b = 0; b < B; b++) s += gb_part[b * Cout + o];
        grad_beta[o] = (T)s;
    }
    free(gx_thr);
    free(gw_part);
    free(ga_part);
    free(gb_part);
    return 0;
}

#undef FN
#undef CAT
#undef CAT_
