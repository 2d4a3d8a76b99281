// reduce.hip — Softmax and MaxPool for gfx950.
//
// Softmax (tensor_ops/tensor_ops.c:1231-1270): the tensor is viewed as
// [outer, L, inner] around the axis.  max over the axis (from -DBL_MAX),
// sum of exp(v - max) in double, output exp(v - max) / sum.  For inner == 1
// one 1024-thread block owns a row: the row is read once into registers,
// reduced with wave64 shuffles and an LDS exchange between the 16 waves, and
// written once.  The double sum is a tree instead of the reference's
// sequential loop (relative difference ~1e-16 before the final rounding).
//
// MaxPool (tensor_ops.c:1116-1165): -inf start, in-bounds taps only, strict >
// (NaN never wins, an all-padding window gives -inf, the first of +-0 wins).
#include <cfloat>

#include "runtime.h"

namespace tohip {
namespace {

constexpr int kRowThreads = 1024;
constexpr int kWaves = kRowThreads / 64;

__device__ __forceinline__ double wave_max(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const double t = __shfl_xor(v, o, 64);
        v = t > v ? t : v;
    }
    return v;
}
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Block-wide reduction across the NW waves of a block (NW * 64 threads).
template <bool MAX, int NW = kWaves> __device__ __forceinline__ double block_reduce(double v, double* lds) {
    v = MAX ? wave_max(v) : wave_sum(v);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    if (l == 0) lds[w] = v;
    __syncthreads();
    double r = lds[0];
#pragma unroll
    for (int i = 1; i < NW; i++) {
        const double t = lds[i];
        r = MAX ? (t > r ? t : r) : r + t;
    }
    __syncthreads();
    return r;
}

// One block per row (inner == 1), the row kept in registers (IPT per thread).
template <int IPT, int DIN, int DOUT>
__global__ __launch_bounds__(kRowThreads) void k_softmax_row(const void* __restrict__ X, void* __restrict__ Y, int L) {
    __shared__ double lds[kWaves];
    const size_t base = (size_t)blockIdx.x * (size_t)L;
    double v[IPT];
    double mx = -DBL_MAX;
#pragma unroll
    for (int t = 0; t < IPT; t++) {
        const int j = threadIdx.x + t * kRowThreads;
        v[t] = j < L ? ld_d<DIN>(X, (int64_t)(base + j)) : -DBL_MAX;
        mx = v[t] > mx ? v[t] : mx;
    }
    mx = block_reduce<true>(mx, lds);
    double sum = 0.0;
#pragma unroll
    for (int t = 0; t < IPT; t++) {
        const int j = threadIdx.x + t * kRowThreads;
        v[t] = j < L ? exp(v[t] - mx) : 0.0;
        sum += v[t];
    }
    sum = block_reduce<false>(sum, lds);
#pragma unroll
    for (int t = 0; t < IPT; t++) {
        const int j = threadIdx.x + t * kRowThreads;
        if (j < L) st_d<DOUT>(Y, (int64_t)(base + j), v[t] / sum);
    }
}

// Rows too long for registers, or uncommon dtypes: three passes over the row.
__global__ __launch_bounds__(kRowThreads) void k_softmax_row_rt(const void* __restrict__ X, int dtx,
                                                                void* __restrict__ Y, int dty, int64_t L) {
    __shared__ double lds[kWaves];
    const int64_t base = (int64_t)blockIdx.x * L;
    double mx = -DBL_MAX;
    for (int64_t j = threadIdx.x; j < L; j += kRowThreads) {
        const double v = ld_d_rt(dtx, X, base + j);
        mx = v > mx ? v : mx;
    }
    mx = block_reduce<true>(mx, lds);
    double sum = 0.0;
    for (int64_t j = threadIdx.x; j < L; j += kRowThreads) sum += exp(ld_d_rt(dtx, X, base + j) - mx);
    sum = block_reduce<false>(sum, lds);
    for (int64_t j = threadIdx.x; j < L; j += kRowThreads)
        st_d_rt(dty, Y, base + j, exp(ld_d_rt(dtx, X, base + j) - mx) / sum);
}

// Long rows, few of them (inner == 1, e.g. [64, 32000]): each row is split
// over G blocks of 256 threads so the fp64 exp / divide work spreads over the
// whole chip.  Three passes keep the reference's arithmetic: (1) block maxima,
// (2) every block folds the G maxima into the row max M and sums exp(v - M)
// over its chunk, (3) every block folds the G partial sums in a fixed order
// and writes exp(v - M) / sum.  part holds 2 * rows * G doubles.
constexpr int kSplitThreads = 256;

template <int DIN>
__global__ __launch_bounds__(kSplitThreads) void k_sm_split_max(const void* __restrict__ X, int dtx, int64_t L,
                                                                int G, double* __restrict__ part) {
    __shared__ double lds[kSplitThreads / 64];
    const int64_t row = blockIdx.y, chunk = (L + G - 1) / G;
    const int64_t j0 = blockIdx.x * chunk, j1 = j0 + chunk < L ? j0 + chunk : L;
    const int64_t base = row * L;
    double mx = -DBL_MAX;
    for (int64_t j = j0 + threadIdx.x; j < j1; j += kSplitThreads) {
        const double v = DIN >= 0 ? ld_d<(DIN >= 0 ? DIN : 0)>(X, base + j) : ld_d_rt(dtx, X, base + j);
        mx = v > mx ? v : mx;
    }
    mx = block_reduce<true, kSplitThreads / 64>(mx, lds);
    if (threadIdx.x == 0) part[row * G + blockIdx.x] = mx;
}

__device__ __forceinline__ double fold_max(const double* p, int G) {
    double m = -DBL_MAX;
    for (int g = 0; g < G; g++) m = p[g] > m ? p[g] : m;
    return m;
}

template <int DIN>
__global__ __launch_bounds__(kSplitThreads) void k_sm_split_sum(const void* __restrict__ X, int dtx, int64_t L,
                                                                int G, double* __restrict__ part) {
    __shared__ double lds[kSplitThreads / 64];
    const int64_t row = blockIdx.y, chunk = (L + G - 1) / G, rows = gridDim.y;
    const int64_t j0 = blockIdx.x * chunk, j1 = j0 + chunk < L ? j0 + chunk : L;
    const int64_t base = row * L;
    const double M = fold_max(part + row * G, G);
    double sum = 0.0;
    for (int64_t j = j0 + threadIdx.x; j < j1; j += kSplitThreads) {
        const double v = DIN >= 0 ? ld_d<(DIN >= 0 ? DIN : 0)>(X, base + j) : ld_d_rt(dtx, X, base + j);
        sum += exp(v - M);
    }
    sum = block_reduce<false, kSplitThreads / 64>(sum, lds);
    if (threadIdx.x == 0) part[rows * G + row * G + blockIdx.x] = sum;
}

template <int DIN, int DOUT>
__global__ __launch_bounds__(kSplitThreads) void k_sm_split_out(const void* __restrict__ X, int dtx,
                                                                void* __restrict__ Y, int dty, int64_t L, int G,
                                                                const double* __restrict__ part) {
    const int64_t row = blockIdx.y, chunk = (L + G - 1) / G, rows = gridDim.y;
    const int64_t j0 = blockIdx.x * chunk, j1 = j0 + chunk < L ? j0 + chunk : L;
    const int64_t base = row * L;
    const double M = fold_max(part + row * G, G);
    const double* ps = part + rows * G + row * G;
    double S = 0.0;
    for (int g = 0; g < G; g++) S += ps[g];
    for (int64_t j = j0 + threadIdx.x; j < j1; j += kSplitThreads) {
        const double v = DIN >= 0 ? ld_d<(DIN >= 0 ? DIN : 0)>(X, base + j) : ld_d_rt(dtx, X, base + j);
        const double r = exp(v - M) / S;
        if constexpr (DOUT >= 0) st_d<DOUT>(Y, base + j, r);
        else st_d_rt(dty, Y, base + j, r);
    }
}

// inner > 1: one thread per (outer, r) column; rows of the axis are coalesced across threads.
__global__ __launch_bounds__(256) void k_softmax_cols(const void* __restrict__ X, int dtx, void* __restrict__ Y,
                                                      int dty, int64_t L, int64_t inner) {
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r >= inner) return;
    const int64_t base = (int64_t)blockIdx.y * L * inner + r;
    double mx = -DBL_MAX;
    for (int64_t j = 0; j < L; j++) {
        const double v = ld_d_rt(dtx, X, base + j * inner);
        mx = v > mx ? v : mx;
    }
    double sum = 0.0;
    for (int64_t j = 0; j < L; j++) sum += exp(ld_d_rt(dtx, X, base + j * inner) - mx);
    for (int64_t j = 0; j < L; j++) {
        const int64_t i = base + j * inner;
        st_d_rt(dty, Y, i, exp(ld_d_rt(dtx, X, i) - mx) / sum);
    }
}

template <int DIN, int DOUT>
bool launch_row(const void* x, void* y, int64_t outer, int64_t L, hipStream_t s) {
    const int ipt = (int)((L + kRowThreads - 1) / kRowThreads);
    const dim3 g((unsigned)outer), b(kRowThreads);
    const int Li = (int)L;
    if (ipt <= 1) hipLaunchKernelGGL((k_softmax_row<1, DIN, DOUT>), g, b, 0, s, x, y, Li);
    else if (ipt <= 2) hipLaunchKernelGGL((k_softmax_row<2, DIN, DOUT>), g, b, 0, s, x, y, Li);
    else if (ipt <= 4) hipLaunchKernelGGL((k_softmax_row<4, DIN, DOUT>), g, b, 0, s, x, y, Li);
    else if (ipt <= 8) hipLaunchKernelGGL((k_softmax_row<8, DIN, DOUT>), g, b, 0, s, x, y, Li);
    else if (ipt <= 16) hipLaunchKernelGGL((k_softmax_row<16, DIN, DOUT>), g, b, 0, s, x, y, Li);
    else if (ipt <= 32) hipLaunchKernelGGL((k_softmax_row<32, DIN, DOUT>), g, b, 0, s, x, y, Li);
    else return false;
    return true;
}

// ------------------------------------------------------------------ MaxPool ---
struct PoolGeom {
    int N, C, H, W, OH, OW, KH, KW, pt, pl, sh, sw, dh, dw;
};

template <int DIN, int DOUT>
__global__ __launch_bounds__(256) void k_maxpool(const void* __restrict__ X, void* __restrict__ Y, PoolGeom g,
                                                 int64_t total) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < total; o += stride) {
        const int ow = (int)(o % g.OW);
        const int64_t t1 = o / g.OW;
        const int oh = (int)(t1 % g.OH);
        const int64_t plane = t1 / g.OH;              // n * C + c
        const int64_t xb = plane * (int64_t)g.H * g.W;
        double best = -__builtin_inf();
        for (int kh = 0; kh < g.KH; kh++) {
            const int ih = oh * g.sh + kh * g.dh - g.pt;
            if (ih < 0 || ih >= g.H) continue;
            for (int kw = 0; kw < g.KW; kw++) {
                const int iw = ow * g.sw + kw * g.dw - g.pl;
                if (iw < 0 || iw >= g.W) continue;
                const double v = ld_d<DIN>(X, xb + (int64_t)ih * g.W + iw);
                if (v > best) best = v;
            }
        }
        st_d<DOUT>(Y, o, best);
    }
}

// f32, LDS-tiled: block (tile, plane) stages the input rows that kTOH output
// rows need (rows outside the image hold -inf, which never wins a strict >
// against the -inf start, exactly like skipping them), then every thread
// reduces its windows from LDS.  Loads are coalesced along W; outputs are
// written along OW.
constexpr int kTOH = 8;
constexpr int kPoolLdsFloats = 8192;   // 32 KB

__global__ __launch_bounds__(256) void k_maxpool_lds(const float* __restrict__ X, float* __restrict__ Y, PoolGeom g,
                                                     int IR) {
    __shared__ float tile[kPoolLdsFloats];
    const int64_t plane = blockIdx.y;
    const int oh0 = blockIdx.x * kTOH;
    const int ih0 = oh0 * g.sh - g.pt;
    const float* xp = X + plane * (int64_t)g.H * g.W;
    const int total = IR * g.W;
    for (int i = threadIdx.x; i < total; i += 256) {
        const int r = i / g.W, c = i - r * g.W;
        const int ih = ih0 + r;
        tile[i] = (ih >= 0 && ih < g.H) ? xp[(int64_t)ih * g.W + c] : -__builtin_inff();
    }
    __syncthreads();
    const int nrow = (g.OH - oh0) < kTOH ? (g.OH - oh0) : kTOH;
    const int nout = nrow * g.OW;
    float* yp = Y + plane * (int64_t)g.OH * g.OW + (int64_t)oh0 * g.OW;
    for (int o = threadIdx.x; o < nout; o += 256) {
        const int r = o / g.OW, ow = o - r * g.OW;
        float best = -__builtin_inff();
        for (int kh = 0; kh < g.KH; kh++) {
            const float* trow = tile + (r * g.sh + kh * g.dh) * g.W;
            for (int kw = 0; kw < g.KW; kw++) {
                const int iw = ow * g.sw + kw * g.dw - g.pl;
                if (iw < 0 || iw >= g.W) continue;
                const float v = trow[iw];
                if (v > best) best = v;
            }
        }
        yp[o] = best;
    }
}

__global__ __launch_bounds__(256) void k_maxpool_rt(const void* __restrict__ X, int dtx, void* __restrict__ Y, int dty,
                                                    PoolGeom g, int64_t total) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < total; o += stride) {
        const int ow = (int)(o % g.OW);
        const int64_t t1 = o / g.OW;
        const int oh = (int)(t1 % g.OH);
        const int64_t plane = t1 / g.OH;
        const int64_t xb = plane * (int64_t)g.H * g.W;
        double best = -__builtin_inf();
        for (int kh = 0; kh < g.KH; kh++) {
            const int ih = oh * g.sh + kh * g.dh - g.pt;
            if (ih < 0 || ih >= g.H) continue;
            for (int kw = 0; kw < g.KW; kw++) {
                const int iw = ow * g.sw + kw * g.dw - g.pl;
                if (iw < 0 || iw >= g.W) continue;
                const double v = ld_d_rt(dtx, X, xb + (int64_t)ih * g.W + iw);
                if (v > best) best = v;
            }
        }
        st_d_rt(dty, Y, o, best);
    }
}

}  // namespace
}  // namespace tohip

using namespace tohip;

extern "C" {

void softmax_forward(const Tensor* input, Tensor* output, int axis) {
    const char* name = "softmax_forward";
    if (!tensor_sane(input, name) || !tensor_sane(output, name)) return;
    if (axis < 0) axis += input->ndim;
    if (axis < 0 || axis >= input->ndim) { set_error("%s: axis out of range", name); return; }
    if (output->size != input->size) { set_error("%s: output size differs from input", name); return; }
    if (!ensure_device()) return;
    int64_t outer = 1, inner = 1;
    const int64_t L = input->shape[axis];
    for (int d = 0; d < axis; d++) outer *= input->shape[d];
    for (int d = axis + 1; d < input->ndim; d++) inner *= input->shape[d];
    Staging st;
    const void* x = st.in(input);
    void* y = st.out(output, tensor_bytes(output));
    if (!x || !y) { st.finish(); return; }
    hipStream_t s = stream();
    const int dtx = (int)input->dtype, dty = (int)output->dtype;
    if (input->size) {
        // Split rows over G blocks when there are too few rows to fill the chip.
        int G = 1;
        if (inner == 1 && outer < 2 * num_cus() && outer <= 65535) {
            G = (int)((2 * num_cus() + outer - 1) / outer);
            const int64_t gmax = (L + 2047) / 2048;            // at least ~2K elements per block
            if (G > gmax) G = (int)gmax;
            if (G > 64) G = 64;
        }
        if (inner == 1 && G > 1) {
            double* part = (double*)pool_alloc(sizeof(double) * 2 * (size_t)outer * G);
            if (!part) { st.finish(); return; }
            const dim3 g((unsigned)G, (unsigned)outer), b(kSplitThreads);
            if (dtx == kF32) {
                hipLaunchKernelGGL((k_sm_split_max<kF32>), g, b, 0, s, x, dtx, L, G, part);
                hipLaunchKernelGGL((k_sm_split_sum<kF32>), g, b, 0, s, x, dtx, L, G, part);
                if (dty == kF32) hipLaunchKernelGGL((k_sm_split_out<kF32, kF32>), g, b, 0, s, x, dtx, y, dty, L, G, part);
                else hipLaunchKernelGGL((k_sm_split_out<kF32, -1>), g, b, 0, s, x, dtx, y, dty, L, G, part);
            } else {
                hipLaunchKernelGGL((k_sm_split_max<-1>), g, b, 0, s, x, dtx, L, G, part);
                hipLaunchKernelGGL((k_sm_split_sum<-1>), g, b, 0, s, x, dtx, L, G, part);
                hipLaunchKernelGGL((k_sm_split_out<-1, -1>), g, b, 0, s, x, dtx, y, dty, L, G, part);
            }
            const bool ok = check_launch(name);
            // The partials buffer returns to the pool once the stream has drained
            // past its last use (pool buffers are reused in stream order).
            pool_free(part);
            if (!ok) { st.finish(); return; }
        } else if (inner == 1) {
            bool done = false;
            if (outer <= 0x7FFFFFFF && L <= 0x7FFFFFFF) {
                if (dtx == kF32 && dty == kF32) done = launch_row<kF32, kF32>(x, y, outer, L, s);
                else if (dtx == kF16 && dty == kF16) done = launch_row<kF16, kF16>(x, y, outer, L, s);
                else if (dtx == kF32 && dty == kF64) done = launch_row<kF32, kF64>(x, y, outer, L, s);
            }
            if (!done)
                hipLaunchKernelGGL(k_softmax_row_rt, dim3((unsigned)outer), dim3(kRowThreads), 0, s, x, dtx, y, dty, L);
        } else {
            const dim3 g((unsigned)((inner + 255) / 256), (unsigned)outer);
            hipLaunchKernelGGL(k_softmax_cols, g, dim3(256), 0, s, x, dtx, y, dty, L, inner);
        }
        if (!check_launch(name)) { st.finish(); return; }
    }
    st.finish();
}

void max_pool_forward(const Tensor* X, Tensor* Y, PoolParams* p) {
    const char* name = "max_pool_forward";
    if (!tensor_sane(X, name) || !tensor_sane(Y, name)) return;
    if (!p || !p->pads || !p->strides || !p->dilations || !p->kernel_shape) { set_error("%s: NULL params", name); return; }
    if (X->ndim != 4 || Y->ndim != 4) { set_error("%s: X and Y must be 4-D (NCHW)", name); return; }
    PoolGeom g;
    g.N = X->shape[0]; g.C = X->shape[1]; g.H = X->shape[2]; g.W = X->shape[3];
    g.OH = Y->shape[2]; g.OW = Y->shape[3];
    g.KH = p->kernel_shape[0]; g.KW = p->kernel_shape[1];
    g.pt = p->pads[0]; g.pl = p->pads[1]; g.sh = p->strides[0]; g.sw = p->strides[1];
    g.dh = p->dilations[0]; g.dw = p->dilations[1];
    if (Y->shape[0] != g.N || Y->shape[1] != g.C) { set_error("%s: Y batch/channels differ from X", name); return; }
    if (!ensure_device()) return;
    const int64_t total = (int64_t)g.N * g.C * g.OH * g.OW;
    Staging st;
    const void* x = st.in(X);
    void* y = st.out(Y, (size_t)total * dt_bytes((int)Y->dtype));
    if (!x || !y) { st.finish(); return; }
    hipStream_t s = stream();
    if (total > 0) {
        const dim3 grid(grid_for((size_t)total, 256)), blk(256);
        const int IR = (kTOH - 1) * g.sh + (g.KH - 1) * g.dh + 1;
        const bool lds_fits = g.KH > 0 && g.KW > 0 && g.sh > 0 && g.dh > 0 && (int64_t)IR * g.W <= kPoolLdsFloats &&
                              (int64_t)g.N * g.C <= 65535;
        if (X->dtype == DTYPE_FLOAT32 && Y->dtype == DTYPE_FLOAT32 && lds_fits) {
            const dim3 tg((unsigned)((g.OH + kTOH - 1) / kTOH), (unsigned)(g.N * g.C));
            hipLaunchKernelGGL(k_maxpool_lds, tg, blk, 0, s, (const float*)x, (float*)y, g, IR);
        } else if (X->dtype == DTYPE_FLOAT32 && Y->dtype == DTYPE_FLOAT32)
            hipLaunchKernelGGL((k_maxpool<kF32, kF32>), grid, blk, 0, s, x, y, g, total);
        else
            hipLaunchKernelGGL(k_maxpool_rt, grid, blk, 0, s, x, (int)X->dtype, y, (int)Y->dtype, g, total);
        if (!check_launch(name)) { st.finish(); return; }
    }
    st.finish();
}

}  // extern "C"
