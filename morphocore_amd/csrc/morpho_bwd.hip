// Dilation / erosion backward for gfx950: gradient routing from the winners of the forward pass.
//
// MAX / MIN (morpho_bwd_packed_kernel): one workgroup per (output channel, pixel chunk) scatters each
// output gradient to its packed (channel, tap): grad_input by global double atomics (one per output
// pixel; a pixel can collect up to Cout * KH * KW of them, which float32 sums would round past the
// 1e-6 tolerance), rounded once to float32 afterwards, grad_weight into LDS bins that become this
// workgroup's partial slot. Small problems (whose time is launches) gather grad_input instead, in
// further workgroups of the same launch: each input pixel sums, in double and in (output channel,
// tap) order, the gradients of the output pixels whose winner it is, written once (no zero fill, no
// atomics, no rounding pass), and keep at most 32 slots (one reduction launch).
// Reference semantics: morpho_op_cpu_backward.hxx:39-88 (run_single_winner).
//
// ADD / AVERAGE / IDENTITY: every channel pair routes g * scale to its own first extremal tap
// (morpho_op_cpu_backward.hxx:90-156, scale = 1 / Cin for AVERAGE). One workgroup per (batch
// element, tile, input channels) walks the output channels, reads each pair's saved tap (one byte),
// accumulates grad_input in LDS over the tile plus halo (flushed once: plain stores where only this
// tile's outputs land, atomics on the halo shared with neighbouring tiles) and grad_weight in
// lane-striped LDS bins, written once per chunk of output channels into the workgroup's partial
// slot. Partial slots are then summed in a fixed order (reduce_slots_async). LDS accumulators are
// double (see Acc). Two kernels:
//   morpho_bwd_planes_kernel  ADD / AVERAGE whose KW planes of the tile fit in LDS: one input
//                             channel per workgroup, grad_input split into one plane per
//                             structuring-element column, which makes the atomic adds bank-conflict
//                             free (measured: the scattered adds of one shared tile spend ~3x their
//                             conflict-free time in bank and address conflicts);
//   morpho_bwd_ident_gather_kernel  IDENTITY 3x3 / 5x5: grad_input gathered per input pixel from
//                             the taps of its window, written once (no fill, no atomics);
//   morpho_bwd_taps_kernel    other IDENTITY and larger structuring elements: one shared tile per
//                             channel.
//
// A tap that read outside the image (including REPLICATE's clamped edge pixel) sends nothing to
// grad_input; grad_weight always receives sign * g (sign -1 for erosion).
// When the forward pass did not save its winners, the forward kernel recomputes them into the
// workspace first.
#include <algorithm>
#include <cstdlib>

#include "launch.hpp"

namespace mca
{

// ST: the storage type of grad_output (float16 / bfloat16 gradients of float32 kernels, else T).
template <typename T, typename ST = T>
struct PackedParams
{
    const int32_t* __restrict__ idx;
    const ST* __restrict__ gout;
    Acc* __restrict__ gin;  // double accumulator of grad_input (the output itself for float64); null: gathered
    ST* __restrict__ gin_gather;  // grad_input written by the gathering workgroups
    T* __restrict__ part;
    Geom g;
    int nchunks;
    int lds_bins;
    int64_t chunk;
    int wblocks;  // workgroups of the scatter; the ones after it gather grad_input (gin null)
};

// Output-channel slots of a gathering workgroup: GATHER_SLOTS threads share each input pixel, slot s
// taking the output channels s, s + GATHER_SLOTS, ...; BLOCK / GATHER_SLOTS pixels per workgroup.
constexpr int GATHER_SLOTS = 16;

// Slot `slot`'s share of the grad_input of input pixel n = ((b * Cin + c) * H + iy) * W + ix: the sum
// of the output gradients of the pixels (o, h, w), o = slot mod GATHER_SLOTS, whose packed winner is
// (c, tap k) with (h + pad_h - kh, w + pad_w - kw) = (iy, ix), in double, over o and then k in order
// (morpho_op_cpu_backward.hxx:39-88 adds the same terms per output pixel).
template <typename T, typename ST>
__device__ __forceinline__ Acc packed_gather_pixel(const PackedParams<T, ST>& p, int64_t n, int slot)
{
    const Geom& g = p.g;
    const int64_t plane = g.plane();
    const int64_t bc = n / plane;
    const int64_t pix = n - bc * plane;
    const int b = (int)(bc / g.Cin), c = (int)(bc - (int64_t)b * g.Cin);
    const int iy = (int)(pix / g.W), ix = (int)(pix - (int64_t)iy * g.W);
    const int ph = g.pad_h(), pw = g.pad_w();
    Acc s = Acc(0);
    for (int o = slot; o < g.Cout; o += GATHER_SLOTS)
    {
        const int64_t base = ((int64_t)b * g.Cout + o) * plane;
        for (int kh = 0; kh < g.KH; ++kh)
        {
            const int h = iy - ph + kh;
            if (h < 0 || h >= g.H) continue;
            for (int kw = 0; kw < g.KW; ++kw)
            {
                const int wc = ix - pw + kw;
                if (wc < 0 || wc >= g.W) continue;
                const int64_t q = base + (int64_t)h * g.W + wc;
                if (p.idx[q] == ((c << 16) | (kh * g.KW + kw))) s += (Acc)(T)p.gout[q];
            }
        }
    }
    return s;
}

template <typename T, int OP, typename ST = T>
__global__ __launch_bounds__(BLOCK) void morpho_bwd_packed_kernel(const PackedParams<T, ST> p)
{
    extern __shared__ __align__(16) unsigned char smem_raw[];
    Acc* bins = reinterpret_cast<Acc*>(smem_raw);
    const Geom g = p.g;
    const int work = xcd_work_index(blockIdx.x, gridDim.x);
    if (work >= p.wblocks)
    {
        // Gathering workgroup: each pixel's slots, then their sum in slot order (deterministic).
        __shared__ Acc slot_sums[BLOCK];
        constexpr int PIX = BLOCK / GATHER_SLOTS;
        const int lp = threadIdx.x % PIX, slot = threadIdx.x / PIX;
        const int64_t n = (int64_t)(work - p.wblocks) * PIX + lp;
        const bool in = n < (int64_t)g.B * g.Cin * g.plane();
        slot_sums[threadIdx.x] = in ? packed_gather_pixel(p, n, slot) : Acc(0);
        __syncthreads();
        if (in && slot == 0)
        {
            Acc s = Acc(0);
            for (int k = 0; k < GATHER_SLOTS; ++k) s += slot_sums[k * PIX + lp];
            p.gin_gather[n] = (ST)s;
        }
        return;
    }
    const int chunk = work % p.nchunks;
    const int o = work / p.nchunks;
    const int K = g.KH * g.KW, ph = g.pad_h(), pw = g.pad_w();
    const int64_t nb = (int64_t)g.Cin * K;
    const int64_t plane = g.plane();
    T* part = p.part + ((int64_t)chunk * g.Cout + o) * nb;
    if (p.lds_bins)
    {
        for (int64_t j = threadIdx.x; j < nb; j += BLOCK) bins[j] = Acc(0);
        __syncthreads();
    }
    const int64_t total = (int64_t)g.B * plane;
    const int64_t n_begin = (int64_t)chunk * p.chunk;
    const int64_t n_end = min(n_begin + p.chunk, total);
    const T sign = (T)OpTraits<OP, T>::sign;
    for (int64_t n = n_begin + threadIdx.x; n < n_end; n += BLOCK)
    {
        const int64_t b = n / plane;
        const int64_t pix = n - b * plane;
        const int h = (int)(pix / g.W), wc = (int)(pix - (int64_t)h * g.W);
        const int64_t gi = (b * g.Cout + o) * plane + pix;
        const T gv = (T)p.gout[gi];
        if (gv == T(0)) continue;
        const int32_t packed = p.idx[gi];
        const int c = packed >> 16, k = packed & 0xFFFF;
        const int kh = k / g.KW, kw = k - kh * g.KW;
        const int iy = h + ph - kh, ix = wc + pw - kw;
        if (p.gin && iy >= 0 && iy < g.H && ix >= 0 && ix < g.W) global_add(&p.gin[(b * g.Cin + c) * plane + (int64_t)iy * g.W + ix], (Acc)gv);
        if (p.lds_bins)
            lds_add(&bins[(int64_t)c * K + k], (Acc)(sign * gv));
        else
            global_add(&part[(int64_t)c * K + k], sign * gv);
    }
    if (p.lds_bins)
    {
        __syncthreads();
        for (int64_t j = threadIdx.x; j < nb; j += BLOCK) part[j] = (T)bins[j];
    }
}

template <typename T, typename ST = T>
struct TapsParams
{
    const void* __restrict__ taps;
    const ST* __restrict__ gout;
    ST* __restrict__ gin;
    T* __restrict__ part;
    Geom g;
    Tiling t;
    int ig;           // input channels per workgroup
    int nig;          // groups of input channels
    int oc;           // output channels per grad_weight flush
    int ncopy_log2;   // log2 of the lane-striped copies of each grad_weight bin
    unsigned kw_div;  // ceil(2^16 / KW): kh = (k * kw_div) >> 16 exactly for every k < 256
    T scale;
};

// Bits of v when keep, +0 otherwise (a select the compiler cannot turn into a branch around the
// load that produced v).
__device__ __forceinline__ float keep_bits(float v, bool keep) { return __uint_as_float(__float_as_uint(v) & (keep ? ~0u : 0u)); }
__device__ __forceinline__ double keep_bits(double v, bool keep)
{
    return __longlong_as_double(__double_as_longlong(v) & (keep ? ~0ll : 0ll));
}

// NI: channel pairs routed per step (IG input channels of one output channel; 1 for IDENTITY, whose
// steps walk the group's channels).
template <typename T, int OP, typename AT, bool IDENT, int RH, int NI>
__global__ __launch_bounds__(BLOCK) void morpho_bwd_taps_kernel(const TapsParams<T> p)
{
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const Geom g = p.g;
    const Tiling t = p.t;
    const int K = g.KH * g.KW;
    const int tile_elems = t.rows * t.pitch;
    const int ncopy = 1 << p.ncopy_log2;
    Acc* gx = reinterpret_cast<Acc*>(smem_raw);
    Acc* bins = gx + (size_t)p.ig * tile_elems;
    int* tapoff = reinterpret_cast<int*>(bins + (size_t)p.oc * p.ig * K * ncopy);
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    int work = xcd_work_index(blockIdx.x, gridDim.x);
    const int igi = work % p.nig;
    work /= p.nig;
    const int tile = work % t.ntiles();
    const int b = work / t.ntiles();
    const int ty = tile / t.ntx, tx = tile - ty * t.ntx;
    const int h0 = ty * t.th, w0 = tx * TILE_W, wc = w0 + lane;
    const int y0 = h0 + g.pad_h() - (g.KH - 1), x0 = w0 + g.pad_w() - (g.KW - 1);
    const int i0 = igi * p.ig;
    const int ni = min(p.ig, g.Cin - i0);
    const int64_t plane = g.plane();
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * K;
    T* part = p.part + ((int64_t)b * t.ntiles() + tile) * wnumel;
    const int copy = lane & (ncopy - 1);
    const int cpair = IDENT ? 1 : g.Cin;
    const AT* __restrict__ taps = static_cast<const AT*>(p.taps);

    // Tap k = kh * KW + kw lands kh * pitch + kw elements before the tap-0 position of the pixel.
    if constexpr (sizeof(AT) > 1)
        for (int k = threadIdx.x; k < K; k += BLOCK) tapoff[k] = (k / g.KW) * t.pitch + k % g.KW;
    for (int j = threadIdx.x; j < p.ig * tile_elems; j += BLOCK) gx[j] = Acc(0);
    const int nbins = p.oc * p.ig * K * ncopy;
    for (int j = threadIdx.x; j < nbins; j += BLOCK) bins[j] = Acc(0);
    __syncthreads();

    // Every load reads a valid (clamped) pixel of a valid (clamped) step, so that the loads of a step
    // are issued unconditionally, one step ahead of their use; pixels outside the image are masked
    // to a zero gradient where the values are used.
    const int wcc = min(wc, g.W - 1);
    int64_t pix[RH];
    bool inside[RH];
#pragma unroll
    for (int r = 0; r < RH; ++r)
    {
        const int h = h0 + wave * RH + r;
        pix[r] = (int64_t)min(h, g.H - 1) * g.W + wcc;
        inside[r] = h < g.H && wc < g.W;
    }
    // gx element of tap 0 of this lane's row-r pixel.
    const int base0 = (wave * RH + g.KH - 1) * t.pitch + lane + g.KW - 1;
    const int rowskip = t.pitch - g.KW;

    struct Step
    {
        T g[RH];
        int k[NI][RH];
    };
    // Output channel and first channel pair of step s of a chunk of output channels [oc0, oc0 + noc).
    auto load_step = [&](int oc0, int noc, int s, Step& st) {
        const int sc = min(s, (IDENT ? ni : noc) - 1);
        const int o = IDENT ? i0 + sc : oc0 + sc;
        const T* __restrict__ gp = p.gout + ((int64_t)b * g.Cout + o) * plane;
#pragma unroll
        for (int r = 0; r < RH; ++r) st.g[r] = gp[pix[r]];
#pragma unroll
        for (int j = 0; j < NI; ++j)
        {
            const int il = IDENT ? 0 : min(j, ni - 1);
            const AT* __restrict__ tp = taps + (((int64_t)b * g.Cout + o) * cpair + (IDENT ? 0 : i0 + il)) * plane;
#pragma unroll
            for (int r = 0; r < RH; ++r) st.k[j][r] = (int)tp[pix[r]];
        }
    };
    // Route step s: for every pair, g * scale to the pair's tap in grad_input and sign * g * scale to
    // its grad_weight bin. A tap outside the image lands in the staged halo, outside the image, and
    // is dropped when the tile is flushed.
    auto route = [&](const Step& st, int s) {
        Acc gd[RH];
#pragma unroll
        for (int r = 0; r < RH; ++r) gd[r] = (Acc)(keep_bits(st.g[r], inside[r]) * p.scale);
#pragma unroll
        for (int j = 0; j < NI; ++j)
        {
            if (!IDENT && j >= ni) break;
            const int il = IDENT ? s : j;
            Acc* gxl = gx + il * tile_elems + base0;
            Acc* bl = bins + (size_t)((IDENT ? 0 : s) * p.ig + il) * K * ncopy + copy;
#pragma unroll
            for (int r = 0; r < RH; ++r)
            {
                const int k = st.k[j][r];
                int off;
                if constexpr (sizeof(AT) == 1)
                    off = k + (int)__umul24(__umul24((unsigned)k, p.kw_div) >> 16, (unsigned)rowskip);
                else
                    off = tapoff[k];
                lds_add(&gxl[r * t.pitch - off], gd[r]);
                lds_add(&bl[k << p.ncopy_log2], OP == DILATION ? gd[r] : -gd[r]);
            }
        }
    };
    // Sum the copies of every bin of output channels [oc0, oc0 + noc) into this workgroup's slot.
    auto flush_bins = [&](int oc0, int noc) {
        __syncthreads();
        const int n = noc * p.ig * K;
        for (int j = threadIdx.x; j < n; j += BLOCK)
        {
            const int k = j % K;
            const int il = (j / K) % p.ig;
            const int ol = j / (K * p.ig);
            Acc s = Acc(0);
            for (int c = 0; c < ncopy; ++c)
            {
                s += bins[(size_t)j * ncopy + c];
                bins[(size_t)j * ncopy + c] = Acc(0);
            }
            if (il < ni)
            {
                const int o = IDENT ? i0 + il : oc0 + ol;
                part[((int64_t)o * g.Cw + (IDENT ? 0 : i0 + il)) * K + k] = (T)s;
            }
        }
        __syncthreads();
    };

    // Steps of one flush chunk, ping-ponging two register buffers: the loads of step s + 1 are in
    // flight while step s routes (the last one re-reads its own step, harmlessly).
    auto run_chunk = [&](int oc0, int noc) {
        const int nsteps = IDENT ? ni : noc;
        Step a, c;
        load_step(oc0, noc, 0, a);
        for (int s = 0; s < nsteps; s += 2)
        {
            load_step(oc0, noc, s + 1, c);
            route(a, s);
            load_step(oc0, noc, s + 2, a);
            if (s + 1 < nsteps) route(c, s + 1);
        }
        flush_bins(oc0, IDENT ? 1 : noc);
    };
    if constexpr (IDENT)
    {
        if (ni > 0) run_chunk(0, 1);
    }
    else
    {
        for (int oc0 = 0; oc0 < g.Cout; oc0 += p.oc) run_chunk(oc0, min(p.oc, g.Cout - oc0));
    }

    // grad_input of the tile and its halo. Rows [KH - 1, th) and columns [KW - 1, 64) of the staged
    // region receive contributions from this tile's outputs only: plain stores. The rest is shared
    // with the neighbouring tiles' footprints: atomics onto the zero-filled gradient.
    for (int il = 0; il < ni; ++il)
    {
        T* gplane = p.gin + ((int64_t)b * g.Cin + i0 + il) * plane;
        const Acc* gxl = gx + il * tile_elems;
        for (int ly = wave; ly < t.rows; ly += NWAVES)
        {
            const int iy = y0 + ly;
            if (iy < 0 || iy >= g.H) continue;
            for (int lx = lane; lx < t.cols; lx += WAVE)
            {
                const int ix = x0 + lx;
                if (ix < 0 || ix >= g.W) continue;
                const T v = (T)gxl[ly * t.pitch + lx];
                const bool own = ly >= g.KH - 1 && ly < t.th && lx >= g.KW - 1 && lx < TILE_W;
                if (own)
                    gplane[(int64_t)iy * g.W + ix] = v;
                else if (v != T(0))
                    global_add(&gplane[(int64_t)iy * g.W + ix], v);
            }
        }
    }
}

// Barrier for LDS traffic only: waits for this wave's LDS operations, not for its global loads in
// flight (prefetched steps stay in flight across it).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ADD / AVERAGE with small structuring elements: one workgroup per (batch element, tile, input
// channel i) walks every output channel o, routing the pair (o, i). grad_input accumulates in KW
// planes of the staged tile: plane kw, row y, column c holds the contributions to staged position
// (y, c + KW - 1 - kw), so every contribution of a lane lands in the lane's own column of some
// plane; with plane and row strides multiples of 32 doubles, the 64 lanes of each atomic add hit
// distinct banks. The planes are summed into grad_input once at the end. Loads run D steps ahead.
template <typename T, int OP, int RH>
__global__ __launch_bounds__(BLOCK) void morpho_bwd_planes_kernel(const TapsParams<T> p)
{
    constexpr int D = 3;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const Geom g = p.g;
    const Tiling t = p.t;
    const int K = g.KH * g.KW;
    const int ncopy = 1 << p.ncopy_log2;
    const int PS = t.rows * WAVE;  // plane stride (elements)
    Acc* planes = reinterpret_cast<Acc*>(smem_raw);
    Acc* bins = planes + (size_t)g.KW * PS;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    int work = xcd_work_index(blockIdx.x, gridDim.x);
    const int i = work % g.Cin;
    work /= g.Cin;
    const int tile = work % t.ntiles();
    const int b = work / t.ntiles();
    const int ty = tile / t.ntx, tx = tile - ty * t.ntx;
    const int h0 = ty * t.th, w0 = tx * TILE_W, wc = w0 + lane;
    const int y0 = h0 + g.pad_h() - (g.KH - 1), x0 = w0 + g.pad_w() - (g.KW - 1);
    const int64_t plane = g.plane();
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * K;
    T* part = p.part + ((int64_t)b * t.ntiles() + tile) * wnumel;
    const int copy = lane & (ncopy - 1);
    const uint8_t* __restrict__ taps = static_cast<const uint8_t*>(p.taps) + ((int64_t)b * g.Cout * g.Cin + i) * plane;
    const T* __restrict__ gout = p.gout + (int64_t)b * g.Cout * plane;
    const int64_t tap_ostride = (int64_t)g.Cin * plane;

    for (int j = threadIdx.x; j < g.KW * PS; j += BLOCK) planes[j] = Acc(0);
    for (int j = threadIdx.x; j < p.oc * K * ncopy; j += BLOCK) bins[j] = Acc(0);
    __syncthreads();

    const int wcc = min(wc, g.W - 1);
    int pix[RH];
    bool inside[RH];
#pragma unroll
    for (int r = 0; r < RH; ++r)
    {
        const int h = h0 + wave * RH + r;
        pix[r] = min(h, g.H - 1) * g.W + wcc;
        inside[r] = h < g.H && wc < g.W;
    }
    const int base0 = (wave * RH + g.KH - 1) * WAVE + lane;
    const int khstep = g.KW * PS + WAVE;

    struct Step
    {
        T g[RH];
        int k[RH];
    };
    // Loads of output channel o (clamped to the last one: the steps past the end re-read it).
    auto load = [&](int o, Step& st) {
        o = min(o, g.Cout - 1);
        const T* __restrict__ gp = gout + (int64_t)o * plane;
        const uint8_t* __restrict__ tp = taps + (int64_t)o * tap_ostride;
#pragma unroll
        for (int r = 0; r < RH; ++r) st.g[r] = gp[pix[r]];
#pragma unroll
        for (int r = 0; r < RH; ++r) st.k[r] = (int)tp[pix[r]];
    };
    auto flush_bins = [&](int oc0, int noc) {
        lds_barrier();
        const int n = noc * K;
        for (int j = threadIdx.x; j < n; j += BLOCK)
        {
            Acc s = Acc(0);
            for (int c = 0; c < ncopy; ++c)
            {
                s += bins[(size_t)j * ncopy + c];
                bins[(size_t)j * ncopy + c] = Acc(0);
            }
            const int ol = j / K, k = j - ol * K;
            part[((int64_t)(oc0 + ol) * g.Cw + i) * K + k] = (T)s;
        }
        lds_barrier();
    };
    int oc0 = 0;
    auto step = [&](const Step& st, int o) {
        if (o >= g.Cout) return;
        Acc* bl = bins + (size_t)(o - oc0) * K * ncopy + copy;
#pragma unroll
        for (int r = 0; r < RH; ++r)
        {
            const Acc gd = (Acc)(keep_bits(st.g[r], inside[r]) * p.scale);
            // Tap k = kh * KW + kw lands kw * PS - kh * 64 elements from the pixel's tap-0 position.
            const int k = st.k[r];
            const unsigned kh = __umul24((unsigned)k, p.kw_div) >> 16;
            const int off = (int)__umul24((unsigned)k, (unsigned)PS) - (int)__umul24(kh, (unsigned)khstep);
            lds_add(&planes[base0 + r * WAVE + off], gd);
            lds_add(&bl[k << p.ncopy_log2], OP == DILATION ? gd : -gd);
        }
        if (o + 1 == g.Cout || o + 1 - oc0 == p.oc)
        {
            flush_bins(oc0, o + 1 - oc0);
            oc0 = o + 1;
        }
    };
    // The prologue issues its loads in the loop's order (compiler barriers between the steps), so
    // that the first iteration waits for no more of them than the later ones do.
    Step s0, s1, s2, s3;
    load(0, s0);
    asm volatile("" ::: "memory");
    load(1, s1);
    asm volatile("" ::: "memory");
    load(2, s2);
    asm volatile("" ::: "memory");
    static_assert(D == 3, "four step buffers");
    for (int o = 0; o < g.Cout; o += D + 1)
    {
        load(o + 3, s3);
        step(s0, o);
        load(o + 4, s0);
        step(s1, o + 1);
        load(o + 5, s1);
        step(s2, o + 2);
        load(o + 6, s2);
        step(s3, o + 3);
    }

    // grad_input of the tile and its halo: the sum of the planes at each staged position. Rows
    // [KH - 1, th) and columns [KW - 1, 64) receive contributions from this tile's outputs only:
    // plain stores. The rest is shared with the neighbouring tiles' footprints: atomics onto the
    // zero-filled gradient.
    T* gplane = p.gin + ((int64_t)b * g.Cin + i) * plane;
    for (int ly = wave; ly < t.rows; ly += NWAVES)
    {
        const int iy = y0 + ly;
        if (iy < 0 || iy >= g.H) continue;
        for (int lx = lane; lx < t.cols; lx += WAVE)
        {
            const int ix = x0 + lx;
            if (ix < 0 || ix >= g.W) continue;
            Acc s = Acc(0);
            for (int kw = 0; kw < g.KW; ++kw)
            {
                const int c = lx - (g.KW - 1 - kw);
                if (c >= 0 && c < WAVE) s += planes[kw * PS + ly * WAVE + c];
            }
            const T v = (T)s;
            const bool own = ly >= g.KH - 1 && ly < t.th && lx >= g.KW - 1 && lx < TILE_W;
            if (own)
                gplane[(int64_t)iy * g.W + ix] = v;
            else if (v != T(0))
                global_add(&gplane[(int64_t)iy * g.W + ix], v);
        }
    }
}

// IDENTITY with 3x3 and 5x5 structuring elements, in gather form: output channel c reads
// input channel c only, so the grad_input of pixel q is the sum of g(p) over the window pixels
// p = q + (kh - KH/2, kw - KW/2) whose saved tap is k = kh * KW + kw, the tap that read q (a tap that
// read outside the image matches no pixel). One workgroup per (batch element, channel, tile)
// stages g and the taps of the tile plus halo in LDS, gathers from a register window, and writes
// each grad_input pixel of the tile once: no zero fill, no atomics on grad_input. grad_weight sums
// sign * g by saved tap in LDS bins with one copy per lane of a half wave (conflict free), one
// partial slot per (batch element, tile). IDENTITY has no 1 / Cin scale.
template <typename T, int OP, int KH, int KW, int RH, typename ST = T>
__global__ __launch_bounds__(BLOCK) void morpho_bwd_ident_gather_kernel(const TapsParams<T, ST> p)
{
    constexpr int K = KH * KW, PH = KH / 2, PW = KW / 2;
    constexpr int TH = NWAVES * RH, ROWS = TH + KH - 1, COLS = TILE_W + KW - 1, WR = RH + KH - 1;
    constexpr int ELEMS = ROWS * COLS, NS = (ELEMS + BLOCK - 1) / BLOCK;
    constexpr int NC = 32;
    __shared__ T gs[ELEMS];
    __shared__ int ts[ELEMS];
    __shared__ __align__(16) Acc bins[K * NC];
    const Geom g = p.g;
    const Tiling t = p.t;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    int work = xcd_work_index(blockIdx.x, gridDim.x);
    const int cgroup = work % p.nig;
    work /= p.nig;
    const int tile = work % t.ntiles();
    const int b = work / t.ntiles();
    const int ty = tile / t.ntx, tx = tile - ty * t.ntx;
    const int h0 = ty * TH, w0 = tx * TILE_W;
    const int y0 = h0 - PH, x0 = w0 - PW;
    const int64_t plane = g.plane();
    const int c_begin = cgroup * p.ig, c_end = min(c_begin + p.ig, g.Cin);
    const int wc = w0 + lane;

    // Staging plan (output pixels of the tile plus halo), the same for every channel: the clamped
    // in-image offset of each element this thread stages and whether it lies in the image (outside:
    // no gradient, a tap that matches none).
    int off[NS];
    bool ok[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j)
    {
        const int idx = min((int)threadIdx.x + j * BLOCK, ELEMS - 1);
        const int ly = idx / COLS, lx = idx - ly * COLS;
        const int y = y0 + ly, x = x0 + lx;
        ok[j] = y >= 0 && y < g.H && x >= 0 && x < g.W;
        off[j] = clampi(y, 0, g.H - 1) * g.W + clampi(x, 0, g.W - 1);
    }
    T pg[NS];
    int pt[NS];
    auto load = [&](int c) {
        const ST* __restrict__ gp = p.gout + ((int64_t)b * g.Cout + c) * plane;
        const uint8_t* __restrict__ tp = static_cast<const uint8_t*>(p.taps) + ((int64_t)b * g.Cout + c) * plane;
#pragma unroll
        for (int j = 0; j < NS; ++j)
        {
            pg[j] = (T)gp[off[j]];
            pt[j] = tp[off[j]];
        }
    };

    for (int j = threadIdx.x; j < K * NC; j += BLOCK) bins[j] = Acc(0);
    load(c_begin);
    for (int c = c_begin; c < c_end; ++c)
    {
#pragma unroll
        for (int j = 0; j < NS; ++j)
        {
            const int idx = threadIdx.x + j * BLOCK;
            if (j < NS - 1 || idx < ELEMS)
            {
                gs[idx] = ok[j] ? pg[j] : T(0);
                ts[idx] = ok[j] ? pt[j] : -1;
            }
        }
        __syncthreads();
        if (c + 1 < c_end) load(c + 1);  // in flight while this channel computes

        T gw[WR][KW];
        int tw[WR][KW];
#pragma unroll
        for (int rr = 0; rr < WR; ++rr)
#pragma unroll
            for (int kw = 0; kw < KW; ++kw)
            {
                gw[rr][kw] = gs[(wave * RH + rr) * COLS + lane + kw];
                tw[rr][kw] = ts[(wave * RH + rr) * COLS + lane + kw];
            }
        ST* __restrict__ gplane = p.gin + ((int64_t)b * g.Cin + c) * plane;
        Acc* bl = bins + (lane & (NC - 1));
#pragma unroll
        for (int r = 0; r < RH; ++r)
        {
            // Window rows r .. r + KH - 1 hold the pixels p of q = (row r, this lane's column).
            Acc s = Acc(0);
#pragma unroll
            for (int kh = 0; kh < KH; ++kh)
#pragma unroll
                for (int kw = 0; kw < KW; ++kw) s += tw[r + kh][kw] == kh * KW + kw ? (Acc)gw[r + kh][kw] : Acc(0);
            const int h = h0 + wave * RH + r;
            if (h < g.H && wc < g.W) gplane[(int64_t)h * g.W + wc] = (ST)(T)s;
            // grad_weight: this lane's own output pixel (h, wc), staged at (row r + PH, column PW).
            const int k = tw[r + PH][PW];
            if (k >= 0) lds_add(&bl[k * NC], (Acc)(OP == DILATION ? gw[r + PH][PW] : -gw[r + PH][PW]));
        }
        __syncthreads();
        // Channel c's bins: 8 threads per tap each add 4 copies and clear them, a butterfly over the
        // 8 finishes (K * 8 <= BLOCK: one pass; groups of 8 lanes are whole).
        static_assert(K * 8 <= BLOCK, "one pass over the bins");
        if (threadIdx.x < K * 8)
        {
            Acc* q = bins + threadIdx.x * 4;
            Acc v = (q[0] + q[1]) + (q[2] + q[3]);
            q[0] = q[1] = q[2] = q[3] = Acc(0);
#pragma unroll
            for (int d = 4; d >= 1; d /= 2) v += __shfl_xor(v, d, 8);
            if ((threadIdx.x & 7) == 0)
                p.part[((int64_t)b * t.ntiles() + tile) * g.Cout * K + (int64_t)c * K + (threadIdx.x >> 3)] = (T)v;
        }
        // The next channel's staging overwrites gs / ts, and its adds need the cleared bins.
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------------
// Launch
// ------------------------------------------------------------------------------------------------

struct PackedPlan
{
    int nchunks;
    int64_t chunk;
    bool lds_bins;
    bool gather;  // grad_input gathered (small problems)
    int gblocks;  // gathering workgroups
    size_t part_bytes;
    size_t lds;
};

// Gathered grad_input reads Cout * KH * KW winners per input pixel: taken while that is at most this
// many reads in all (a few microseconds), where launches, not the scatter's work, set the time.
constexpr int64_t PACKED_GATHER_READS = int64_t(1) << 25;

template <typename T>
static PackedPlan plan_packed(const Geom& g)
{
    PackedPlan s{};
    const int64_t total = (int64_t)g.B * g.plane();
    const int64_t wnumel = (int64_t)g.Cout * g.Cin * g.taps();
    const int64_t gin_n = (int64_t)g.B * g.Cin * g.plane();
    s.gather = gin_n > 0 && gin_n * g.Cout * g.taps() <= PACKED_GATHER_READS;
    s.gblocks = s.gather ? (int)((gin_n + BLOCK / GATHER_SLOTS - 1) / (BLOCK / GATHER_SLOTS)) : 0;
    int64_t nchunks = (4096 + g.Cout - 1) / std::max(g.Cout, 1);  // (no output channel: an empty launch)
    const int64_t max_chunks = (total + BLOCK - 1) / BLOCK;
    if (nchunks > max_chunks) nchunks = max_chunks;
    if (s.gather && nchunks > REDUCE_GROUP) nchunks = REDUCE_GROUP;  // one reduction launch
    while (nchunks > 1 && (size_t)nchunks * wnumel * sizeof(T) > ((size_t)256 << 20)) nchunks /= 2;
    if (nchunks < 1) nchunks = 1;
    s.nchunks = (int)nchunks;
    s.chunk = (total + nchunks - 1) / nchunks;
    const size_t bins = (size_t)g.Cin * g.taps() * sizeof(Acc);
    s.lds_bins = bins <= LDS_LIMIT;
    s.lds = s.lds_bins ? bins : 0;
    s.part_bytes = (size_t)nchunks * wnumel * sizeof(T);
    return s;
}

// Rows per wave of the IDENTITY gather kernel.
constexpr int GATHER_RH = 4;

struct TapsPlan
{
    Tiling t;
    int ig, nig, oc, ncopy;
    bool planes;  // morpho_bwd_planes_kernel
    bool gather;  // morpho_bwd_ident_gather_kernel (else morpho_bwd_taps_kernel)
    bool band;    // gathered by ident_band_gather (morpho_ident.hip): slots per (batch element, band)
    size_t part_bytes;
    size_t lds;
};

// band_ok: the row-band gather may run (its pointers are aligned; see ident_band_backward).
template <typename T>
static TapsPlan plan_taps(int merge, const Geom& g, bool band_ok = true)
{
    TapsPlan s{};
    s.t = make_tiling(g, rows_per_wave<T>());
    const size_t tile = (size_t)s.t.rows * s.t.pitch * sizeof(Acc);
    const size_t K = (size_t)g.taps();
    const size_t table = align16(K * sizeof(int));
    const bool ident = merge == MERGE_IDENTITY;
    // Three workgroups per CU (160 KiB of LDS each) when the accumulators of one output channel fit
    // that share, one launch's maximum otherwise.
    const size_t target = (160 * 1024) / 3 / 1024 * 1024;
    s.part_bytes = (size_t)g.B * s.t.ntiles() * g.Cout * g.Cw * K * sizeof(T);
    if (ident && g.KH == g.KW && (g.KH == 3 || g.KH == 5))
    {
        const IdentBands bands = band_ok ? ident_bands(g, sizeof(T), true) : IdentBands{0, 0, 0};
        if (bands.R > 0)
        {
            // Bands of whole rows, one (batch element, channel, band) per workgroup; the tiling's
            // "tiles" are the bands (one partial slot each per batch element).
            s.t = make_tiling(g, 1);
            s.t.th = bands.R;
            s.t.ntx = 1;
            s.t.nty = bands.nbands;
            s.gather = true;
            s.band = true;
            s.ig = 1;
            s.nig = 1;
            s.oc = 1;
            s.ncopy = 1;
            s.part_bytes = (size_t)g.B * bands.nbands * g.Cout * g.Cw * K * sizeof(T);
            s.lds = bands.lds;
            return s;
        }
        // 4 rows per wave for every dtype: 16-row tiles (float32 / 16-bit gathers 18-26% faster than
        // with 8 rows, measured at configs[3]'s shape).
        s.t = make_tiling(g, GATHER_RH);
        s.part_bytes = (size_t)g.B * s.t.ntiles() * g.Cout * g.Cw * K * sizeof(T);
        // Up to 8 consecutive channels per workgroup, the next channel's loads in flight behind
        // each channel's gather.
        s.gather = true;
        s.ig = std::max(1, std::min(g.Cin, 8));
        s.nig = (g.Cin + s.ig - 1) / s.ig;
        s.oc = 1;
        s.ncopy = 32;
        s.lds = 0;  // static
        return s;
    }
    if (!ident && g.plane() <= 0x7fffffff && K <= 256)
    {
        // The planes kernel, with 16-row (else 8-row) tiles when KW planes of the tile fit (never
        // the case for more than 256 taps, which would need two-byte taps).
        for (int rh = 4; rh >= 2; rh /= 2)
        {
            const Tiling t = make_tiling(g, rh);
            const size_t planes = (size_t)g.KW * t.rows * WAVE * sizeof(Acc);
            const size_t per_oc = K * 4 * sizeof(Acc);
            if (planes + per_oc > LDS_LIMIT) continue;
            const size_t budget = planes + per_oc <= target ? target : LDS_LIMIT;
            s.t = t;
            s.planes = true;
            s.ig = 1;
            s.nig = g.Cin;
            s.ncopy = 4;
            s.oc = (int)((budget - planes) / per_oc);
            if (s.oc > g.Cout) s.oc = g.Cout;
            s.lds = planes + (size_t)s.oc * per_oc;
            s.part_bytes = (size_t)g.B * t.ntiles() * g.Cout * g.Cw * K * sizeof(T);
            return s;
        }
    }
    auto need = [&](int ig, int oc, int ncopy) { return ig * tile + (size_t)oc * ig * K * ncopy * sizeof(Acc) + table; };
    s.ncopy = 4;
    s.ig = ident ? 4 : 2;
    while (s.ig > 1 && s.ig > g.Cin) s.ig /= 2;
    while (s.ig > 1 && need(s.ig, 1, s.ncopy) > target) s.ig /= 2;
    while (s.ncopy > 1 && need(s.ig, 1, s.ncopy) > LDS_LIMIT) s.ncopy /= 2;
    if (ident)
    {
        s.oc = 1;
    }
    else
    {
        const size_t budget = need(s.ig, 1, s.ncopy) <= target ? target : LDS_LIMIT;
        const size_t per_oc = (size_t)s.ig * K * s.ncopy * sizeof(Acc);
        const size_t fixed = s.ig * tile + table;
        s.oc = budget > fixed ? (int)((budget - fixed) / per_oc) : 1;
        if (s.oc > g.Cout) s.oc = g.Cout;
        if (s.oc < 1) s.oc = 1;
    }
    s.nig = (g.Cin + s.ig - 1) / s.ig;
    s.lds = need(s.ig, s.oc, s.ncopy);
    return s;
}

template <typename T>
size_t morpho_backward_lds(int merge, const Geom& g)
{
    if (packed_winners(merge)) return plan_packed<T>(g).lds;
    return plan_taps<T>(merge, g).lds;
}

// Partial slots of grad_weight (one per workgroup that writes them) and their count.
template <typename T>
static void partials(int merge, const Geom& g, size_t& part_bytes, int& nslots, bool band_ok = true)
{
    if (packed_winners(merge))
    {
        const PackedPlan s = plan_packed<T>(g);
        part_bytes = s.part_bytes;
        nslots = s.nchunks;
    }
    else
    {
        const TapsPlan s = plan_taps<T>(merge, g, band_ok);
        part_bytes = s.part_bytes;
        nslots = g.B * s.t.ntiles();
    }
}

// The larger partial slots of the two plans an IDENTITY gather may take (the row-band one, or the
// tiled one when its pointers are not aligned): the workspace is sized before the pointers are known.
template <typename T>
static void partials_bound(int merge, const Geom& g, size_t& part_bytes, int& nslots)
{
    size_t b2;
    int n2;
    partials<T>(merge, g, part_bytes, nslots, true);
    partials<T>(merge, g, b2, n2, false);
    part_bytes = std::max(part_bytes, b2);
    nslots = std::max(nslots, n2);
}

// Whether the row-band gather may take these buffers: 16-byte aligned gradients, 8-byte aligned taps.
static bool band_aligned(const void* grad_out, const void* grad_in, const void* taps)
{
    return ((uintptr_t)grad_out | (uintptr_t)grad_in) % 16 == 0 && (uintptr_t)taps % 8 == 0;
}

// When the forward kept no per-pair taps (sum / mean / identity), the backward recomputes them for
// this many batch elements at a time: as many as fit 1 GiB of taps and scratch output
// (MORPHOCORE_AMD_RECOMPUTE_BYTES overrides it), at least one, so that the fallback's memory stays
// bounded whatever the batch. (Max / min winners, one int32 per output pixel, are recomputed whole.)
static size_t recompute_bytes()
{
    const char* v = std::getenv("MORPHOCORE_AMD_RECOMPUTE_BYTES");
    return v && *v ? (size_t)std::strtoull(v, nullptr, 10) : (size_t(1) << 30);
}

template <typename T>
static int recompute_batch(int merge, const Geom& g)
{
    if (packed_winners(merge)) return g.B;
    Geom one = g;
    one.B = 1;
    const size_t per = indices_bytes(merge, one) + (size_t)one.Cout * one.plane() * sizeof(T);
    const int64_t fit = per > 0 ? (int64_t)(recompute_bytes() / per) : g.B;
    return (int)std::max<int64_t>(1, std::min<int64_t>(fit, g.B));
}

// Workspace layout: [partial slots | reduction scratch | (recomputed winners | scratch output, for
// recompute_batch batch elements)].
template <typename T>
size_t morpho_backward_workspace(int merge, bool has_indices, const Geom& g)
{
    size_t part_bytes;
    int nslots;
    partials_bound<T>(merge, g, part_bytes, nslots);
    size_t bytes = align_up(part_bytes) + align_up(reduce_slots_scratch<T>(nslots, (int64_t)g.Cout * g.Cw * g.taps()));
    if (!has_indices)
    {
        Geom c = g;
        c.B = recompute_batch<T>(merge, g);
        bytes += align_up(indices_bytes(merge, c)) + align_up((size_t)c.B * c.Cout * c.plane() * sizeof(T));
    }
    if (packed_winners(merge) && sizeof(T) != sizeof(Acc) && !plan_packed<T>(g).gather)
        bytes += align_up((size_t)g.B * g.Cin * g.plane() * sizeof(Acc));
    return bytes;
}

template <typename T, int OP>
static hipError_t backward_op(int merge, bool replicate, T fill, const T* x, const T* w, const void* indices, const T* grad_out,
                              T* grad_in, T* grad_w, const Geom& g, unsigned char* ws, hipStream_t stream)
{
    hipError_t err;
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * g.taps();
    const bool packed = packed_winners(merge);
    const bool nonempty = (int64_t)g.B * g.Cout * g.plane() > 0;
    // Recomputed taps live in the workspace (256-byte aligned).
    const bool band_ok = band_aligned(grad_out, grad_in, indices);
    // The gather kernels write every grad_input pixel themselves; the others accumulate onto zeros.
    const bool gather = nonempty && (packed ? plan_packed<T>(g).gather : plan_taps<T>(merge, g, band_ok).gather);
    const int64_t gin_n = (int64_t)g.B * g.Cin * g.plane();
    // float32 max / min round their double grad_input accumulator into every pixel at the end.
    const bool rounded = packed && sizeof(T) != sizeof(Acc) && nonempty;
    if (!gather && !rounded)
        if ((err = fill_async<T>(grad_in, gin_n, T(0), stream)) != hipSuccess) return err;
    if ((int64_t)g.B * g.Cout * g.plane() == 0) return fill_async<T>(grad_w, wnumel, T(0), stream);

    size_t part_bytes;
    int nslots;
    partials<T>(merge, g, part_bytes, nslots, band_ok);
    T* part = reinterpret_cast<T*>(ws);
    ws += align_up(part_bytes);
    T* scratch = reinterpret_cast<T*>(ws);
    ws += align_up(reduce_slots_scratch<T>(nslots, wnumel));
    if (!indices && packed)
    {
        // The forward pass did not keep its winners: recompute them (and a scratch output).
        void* idx = ws;
        T* tmp_out = reinterpret_cast<T*>(ws + align_up(indices_bytes(merge, g)));
        if ((err = morpho_forward<T>(OP, merge, replicate, fill, x, w, tmp_out, idx, g, stream)) != hipSuccess) return err;
        indices = idx;
        ws += align_up(indices_bytes(merge, g)) + align_up((size_t)g.B * g.Cout * g.plane() * sizeof(T));
    }

    if (packed)
    {
        const PackedPlan s = plan_packed<T>(g);
        if (!s.lds_bins)
            if ((err = fill_async<T>(part, (int64_t)s.nchunks * wnumel, T(0), stream)) != hipSuccess) return err;
        // float32: grad_input summed in a double buffer of the workspace, rounded once at the end
        // (gathered: written directly).
        Acc* gin_acc = s.gather ? nullptr : reinterpret_cast<Acc*>(grad_in);
        if constexpr (sizeof(T) != sizeof(Acc))
        {
            if (!s.gather)
            {
                gin_acc = reinterpret_cast<Acc*>(ws);
                if ((err = fill_async<Acc>(gin_acc, gin_n, Acc(0), stream)) != hipSuccess) return err;
            }
        }
        PackedParams<T> p{};
        p.idx = static_cast<const int32_t*>(indices);
        p.gout = grad_out;
        p.gin = gin_acc;
        p.gin_gather = grad_in;
        p.part = part;
        p.g = g;
        p.nchunks = s.nchunks;
        p.lds_bins = s.lds_bins ? 1 : 0;
        p.chunk = s.chunk;
        p.wblocks = s.nchunks * g.Cout;
        morpho_bwd_packed_kernel<T, OP><<<(unsigned)((int64_t)p.wblocks + s.gblocks), BLOCK, s.lds, stream>>>(p);
        if ((err = hipGetLastError()) != hipSuccess) return err;
        if constexpr (sizeof(T) != sizeof(Acc))
            if (!s.gather)
                if ((err = round_async<T>(gin_acc, grad_in, gin_n, stream)) != hipSuccess) return err;
        return reduce_slots_async<T>(part, nslots, wnumel, grad_w, scratch, stream);
    }

    const TapsPlan s = plan_taps<T>(merge, g, band_ok);
    // Without saved taps, batch chunks: each chunk's taps recomputed into the workspace, then routed
    // into its own grad_input rows and partial slots (slots are per batch element and tile).
    const int chunk = indices ? g.B : recompute_batch<T>(merge, g);
    void* idx_ws = ws;
    T* out_ws = nullptr;
    if (!indices)
    {
        Geom c = g;
        c.B = chunk;
        out_ws = reinterpret_cast<T*>(ws + align_up(indices_bytes(merge, c)));
    }
    const int64_t plane = g.plane();
    for (int b0 = 0; b0 < g.B; b0 += chunk)
    {
        Geom gc = g;
        gc.B = std::min(chunk, g.B - b0);
        const void* taps = indices;
        if (!indices)
        {
            if ((err = morpho_forward<T>(OP, merge, replicate, fill, x + (int64_t)b0 * g.Cin * plane, w + (int64_t)b0 * g.wbs, out_ws, idx_ws,
                                         gc, stream)) != hipSuccess)
                return err;
            taps = idx_ws;
        }
        TapsParams<T> p{};
        p.taps = taps;
        p.gout = grad_out + (int64_t)b0 * g.Cout * plane;
        p.gin = grad_in + (int64_t)b0 * g.Cin * plane;
        p.part = part + (int64_t)b0 * s.t.ntiles() * wnumel;
        p.g = gc;
        p.t = s.t;
        p.ig = s.ig;
        p.nig = s.nig;
        p.oc = s.oc;
        p.ncopy_log2 = __builtin_ctz((unsigned)s.ncopy);
        p.kw_div = (65536u + (unsigned)g.KW - 1) / (unsigned)g.KW;
        p.scale = merge == MERGE_AVERAGE ? T(1) / (T)g.Cin : T(1);
        constexpr int RH = rows_per_wave<T>();
        const unsigned blocks = (unsigned)((int64_t)gc.B * s.t.ntiles() * s.nig);
        const bool wide = pair_tap_bytes(g) == 2;
        if (s.band)
        {
            if ((err = ident_band_backward<T, T>(OP, static_cast<const uint8_t*>(taps), p.gout, p.gin, p.part, gc, stream)) != hipSuccess)
                return err;
        }
        else if (s.gather)
        {
            switch (g.KH)
            {
                case 3: morpho_bwd_ident_gather_kernel<T, OP, 3, 3, GATHER_RH><<<blocks, BLOCK, 0, stream>>>(p); break;
                default: morpho_bwd_ident_gather_kernel<T, OP, 5, 5, GATHER_RH><<<blocks, BLOCK, 0, stream>>>(p); break;
            }
        }
        else if (s.planes)
        {
            if (s.t.rh == 4)
                morpho_bwd_planes_kernel<T, OP, 4><<<blocks, BLOCK, s.lds, stream>>>(p);
            else
                morpho_bwd_planes_kernel<T, OP, 2><<<blocks, BLOCK, s.lds, stream>>>(p);
        }
        else if (merge == MERGE_IDENTITY)
        {
            if (wide)
                morpho_bwd_taps_kernel<T, OP, uint16_t, true, RH, 1><<<blocks, BLOCK, s.lds, stream>>>(p);
            else
                morpho_bwd_taps_kernel<T, OP, uint8_t, true, RH, 1><<<blocks, BLOCK, s.lds, stream>>>(p);
        }
        else if (s.ig == 2)
        {
            if (wide)
                morpho_bwd_taps_kernel<T, OP, uint16_t, false, RH, 2><<<blocks, BLOCK, s.lds, stream>>>(p);
            else
                morpho_bwd_taps_kernel<T, OP, uint8_t, false, RH, 2><<<blocks, BLOCK, s.lds, stream>>>(p);
        }
        else
        {
            if (wide)
                morpho_bwd_taps_kernel<T, OP, uint16_t, false, RH, 1><<<blocks, BLOCK, s.lds, stream>>>(p);
            else
                morpho_bwd_taps_kernel<T, OP, uint8_t, false, RH, 1><<<blocks, BLOCK, s.lds, stream>>>(p);
        }
        if ((err = hipGetLastError()) != hipSuccess) return err;
    }
    return reduce_slots_async<T>(part, nslots, wnumel, grad_w, scratch, stream);
}

template <typename T>
hipError_t morpho_backward(int op, int merge, bool replicate, compute_t<T> fill, const T* x, const T* w, const void* indices,
                           const T* grad_out, T* grad_in, T* grad_w, const Geom& g, void* workspace, size_t workspace_bytes,
                           hipStream_t stream)
{
    if (workspace_bytes < morpho_backward_workspace<T>(merge, indices != nullptr, g)) return hipErrorInvalidValue;
    if (g.Cin == 0) return hipSuccess;  // grad_input and grad_weight are empty
    unsigned char* ws = reinterpret_cast<unsigned char*>(workspace);
    return op == DILATION ? backward_op<T, DILATION>(merge, replicate, fill, x, w, indices, grad_out, grad_in, grad_w, g, ws, stream)
                          : backward_op<T, EROSION>(merge, replicate, fill, x, w, indices, grad_out, grad_in, grad_w, g, ws, stream);
}

// Float16 / bfloat16: the winners come from the forward (or the 16-bit forward kernels recompute them
// into the workspace); grad_output is converted to float32, the float32 kernels route it, and
// grad_input and grad_weight are rounded once into the 16-bit outputs. Workspace: [float32 workspace
// with winners | grad_output | grad_input | grad_weight (float32) | (recomputed winners | scratch output)].
template <typename ST>
static size_t half_parts(int merge, const Geom& g, size_t& inner, size_t& gout, size_t& gin, size_t& gw)
{
    inner = align_up(morpho_backward_workspace<float>(merge, true, g));
    gout = align_up((size_t)g.B * g.Cout * g.plane() * sizeof(float));
    gin = align_up((size_t)g.B * g.Cin * g.plane() * sizeof(float));
    gw = align_up((size_t)g.Cout * g.Cw * g.taps() * sizeof(float));
    return inner + gout + gin + gw;
}

template <typename ST>
size_t half_backward_workspace(int merge, bool has_indices, const Geom& g)
{
    size_t inner, gout, gin, gw;
    size_t bytes = half_parts<ST>(merge, g, inner, gout, gin, gw);
    if (!has_indices) bytes += align_up(indices_bytes(merge, g)) + align_up((size_t)g.B * g.Cout * g.plane() * sizeof(ST));
    return bytes;
}

// The kernels that read grad_output once per output pixel and write grad_input once per input pixel
// take the 16-bit data directly: the max / min scatter (double accumulator rounded into grad_input)
// and the IDENTITY gather. grad_weight is summed in float32 partial slots and rounded at the end.
template <typename ST, int OP>
static hipError_t half_direct(int merge, const void* indices, const ST* grad_out, ST* grad_in, ST* grad_w, const Geom& g, unsigned char* ws,
                              float* gw, hipStream_t stream)
{
    hipError_t err;
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * g.taps();
    const bool band_ok = band_aligned(grad_out, grad_in, indices);
    size_t part_bytes;
    int nslots;
    partials<float>(merge, g, part_bytes, nslots, band_ok);
    float* part = reinterpret_cast<float*>(ws);
    ws += align_up(part_bytes);
    float* scratch = reinterpret_cast<float*>(ws);
    ws += align_up(reduce_slots_scratch<float>(nslots, wnumel));
    if (packed_winners(merge))
    {
        const PackedPlan s = plan_packed<float>(g);
        const int64_t gin_n = (int64_t)g.B * g.Cin * g.plane();
        if (!s.lds_bins)
            if ((err = fill_async<float>(part, (int64_t)s.nchunks * wnumel, 0.0f, stream)) != hipSuccess) return err;
        Acc* gin_acc = s.gather ? nullptr : reinterpret_cast<Acc*>(ws);
        if (!s.gather)
            if ((err = fill_async<Acc>(gin_acc, gin_n, Acc(0), stream)) != hipSuccess) return err;
        PackedParams<float, ST> p{};
        p.idx = static_cast<const int32_t*>(indices);
        p.gout = grad_out;
        p.gin = gin_acc;
        p.gin_gather = grad_in;
        p.part = part;
        p.g = g;
        p.nchunks = s.nchunks;
        p.lds_bins = s.lds_bins ? 1 : 0;
        p.chunk = s.chunk;
        p.wblocks = s.nchunks * g.Cout;
        morpho_bwd_packed_kernel<float, OP, ST><<<(unsigned)((int64_t)p.wblocks + s.gblocks), BLOCK, s.lds, stream>>>(p);
        if ((err = hipGetLastError()) != hipSuccess) return err;
        if (!s.gather)
            if ((err = round_async<ST>(gin_acc, grad_in, gin_n, stream)) != hipSuccess) return err;
    }
    else
    {
        const TapsPlan s = plan_taps<float>(merge, g, band_ok);
        if (s.band)
        {
            if ((err = ident_band_backward<float, ST>(OP, static_cast<const uint8_t*>(indices), grad_out, grad_in, part, g, stream)) !=
                hipSuccess)
                return err;
            if ((err = reduce_slots_async<float>(part, nslots, wnumel, gw, scratch, stream)) != hipSuccess) return err;
            return convert_async<float, ST>(gw, grad_w, wnumel, stream);
        }
        TapsParams<float, ST> p{};
        p.taps = indices;
        p.gout = grad_out;
        p.gin = grad_in;
        p.part = part;
        p.g = g;
        p.t = s.t;
        p.ig = s.ig;
        p.nig = s.nig;
        const unsigned blocks = (unsigned)((int64_t)g.B * s.t.ntiles() * s.nig);
        if (g.KH == 3)
            morpho_bwd_ident_gather_kernel<float, OP, 3, 3, GATHER_RH, ST><<<blocks, BLOCK, 0, stream>>>(p);
        else
            morpho_bwd_ident_gather_kernel<float, OP, 5, 5, GATHER_RH, ST><<<blocks, BLOCK, 0, stream>>>(p);
        if ((err = hipGetLastError()) != hipSuccess) return err;
    }
    if ((err = reduce_slots_async<float>(part, nslots, wnumel, gw, scratch, stream)) != hipSuccess) return err;
    return convert_async<float, ST>(gw, grad_w, wnumel, stream);
}

template <typename ST>
hipError_t half_backward(int op, int merge, bool replicate, float fill, const ST* x, const ST* w, const void* indices, const ST* grad_out,
                         ST* grad_in, ST* grad_w, const Geom& g, void* workspace, size_t workspace_bytes, hipStream_t stream)
{
    if (workspace_bytes < half_backward_workspace<ST>(merge, indices != nullptr, g)) return hipErrorInvalidValue;
    if (g.Cin == 0) return hipSuccess;  // grad_input and grad_weight are empty
    size_t inner, gout_b, gin_b, gw_b;
    const size_t base = half_parts<ST>(merge, g, inner, gout_b, gin_b, gw_b);
    unsigned char* ws = reinterpret_cast<unsigned char*>(workspace);
    float* gout = reinterpret_cast<float*>(ws + inner);
    float* gin = reinterpret_cast<float*>(ws + inner + gout_b);
    float* gw = reinterpret_cast<float*>(ws + inner + gout_b + gin_b);
    hipError_t err;
    if (!indices)
    {
        void* idx = ws + base;
        ST* tmp_out = reinterpret_cast<ST*>(ws + base + align_up(indices_bytes(merge, g)));
        if ((err = morpho_forward<ST>(op, merge, replicate, fill, x, w, tmp_out, idx, g, stream)) != hipSuccess) return err;
        indices = idx;
    }
    const int64_t gout_n = (int64_t)g.B * g.Cout * g.plane(), gin_n = (int64_t)g.B * g.Cin * g.plane();
    const int64_t wnumel = (int64_t)g.Cout * g.Cw * g.taps();
    if (gout_n == 0)
    {
        // No output gradient: both gradients are zero.
        if ((err = fill_async<ST>(grad_in, gin_n, ST(0), stream)) != hipSuccess) return err;
        return fill_async<ST>(grad_w, wnumel, ST(0), stream);
    }
    if (packed_winners(merge) || plan_taps<float>(merge, g).gather)
        return op == DILATION ? half_direct<ST, DILATION>(merge, indices, grad_out, grad_in, grad_w, g, ws, gw, stream)
                              : half_direct<ST, EROSION>(merge, indices, grad_out, grad_in, grad_w, g, ws, gw, stream);
    if ((err = convert_async<ST, float>(grad_out, gout, gout_n, stream)) != hipSuccess) return err;
    // With the winners given, the float32 kernels read neither the input nor the element.
    if ((err = morpho_backward<float>(op, merge, replicate, fill, nullptr, nullptr, indices, gout, gin, gw, g, ws, inner, stream)) !=
        hipSuccess)
        return err;
    if ((err = convert_async<float, ST>(gin, grad_in, gin_n, stream)) != hipSuccess) return err;
    return convert_async<float, ST>(gw, grad_w, wnumel, stream);
}

#define MCA_INSTANTIATE_BWD(T)                                                                                                          \
    template size_t morpho_backward_workspace<T>(int, bool, const Geom&);                                                               \
    template size_t morpho_backward_lds<T>(int, const Geom&);                                                                           \
    template hipError_t morpho_backward<T>(int, int, bool, compute_t<T>, const T*, const T*, const void*, const T*, T*, T*, const Geom&, \
                                           void*, size_t, hipStream_t);

MCA_INSTANTIATE_BWD(float)
MCA_INSTANTIATE_BWD(double)

#define MCA_INSTANTIATE_BWD_HALF(ST)                                                                                                    \
    template <>                                                                                                                         \
    size_t morpho_backward_workspace<ST>(int merge, bool has_indices, const Geom& g)                                                    \
    {                                                                                                                                   \
        return half_backward_workspace<ST>(merge, has_indices, g);                                                                      \
    }                                                                                                                                   \
    template <>                                                                                                                         \
    size_t morpho_backward_lds<ST>(int merge, const Geom& g)                                                                            \
    {                                                                                                                                   \
        return morpho_backward_lds<float>(merge, g);                                                                                    \
    }                                                                                                                                   \
    template <>                                                                                                                         \
    hipError_t morpho_backward<ST>(int op, int merge, bool replicate, float fill, const ST* x, const ST* w, const void* indices,         \
                                   const ST* grad_out, ST* grad_in, ST* grad_w, const Geom& g, void* workspace, size_t workspace_bytes,  \
                                   hipStream_t stream)                                                                                  \
    {                                                                                                                                   \
        return half_backward<ST>(op, merge, replicate, fill, x, w, indices, grad_out, grad_in, grad_w, g, workspace, workspace_bytes,   \
                                 stream);                                                                                               \
    }

MCA_INSTANTIATE_BWD_HALF(_Float16)
MCA_INSTANTIATE_BWD_HALF(__bf16)

}  // namespace mca
