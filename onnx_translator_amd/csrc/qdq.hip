// qdq.hip — QuantizeLinear / DequantizeLinear for gfx950.
//
// tensor_ops/tensor_ops.c:999-1034:
//   quantize:   y = s != 0 ? rint(x / s) + zp : zp   (double), then the output encoder
//   dequantize: y = (x - zp) * s                     (double), then the output encoder
// The quotient is an fp64 division (an fp32 quotient can round onto or across
// a .5 tie, so it is not equivalent); rint is round-half-to-even.  Scale and
// zero point are indexed through a broadcast descriptor against Y (scalar,
// per-axis or full-size), so nothing is materialised.
//
// Fast kernels: f32 X (quantize) / 1-byte X (dequantize) with f32 scale,
// V = 16 elements per thread: four 16-byte f32 vectors and one 16-byte code
// vector per thread, all coalesced.  Other dtype combinations use a generic
// one-element-per-thread kernel with a run-time dtype switch.
#include "runtime.h"

namespace tohip {
namespace {

constexpr int kBlock = 256;
constexpr int kV = 16;

template <int YDT> __device__ __forceinline__ uint8_t code8(double r) {
    if constexpr (YDT == kU8) return (uint8_t)sat(cvt_i64(__builtin_rint(r)), 0, 255);
    else if constexpr (YDT == kI8) return (uint8_t)(int8_t)sat(cvt_i64(__builtin_rint(r)), -128, 127);
    else if constexpr (YDT == kI4) return (uint8_t)(int8_t)sat(cvt_i64(__builtin_rint(r)), -8, 7);
    else if constexpr (YDT == kE4M3) return enc_e4m3((float)r);
    else return enc_e5m2((float)r);
}

__device__ __forceinline__ double qval(double x, double s, double z) { return s != 0.0 ? __builtin_rint(x / s) + z : z; }

// Quantize f32 -> 1-byte code, V elements per thread along the innermost dim.
// Operand order in d: 0 = X, 1 = Scale, 2 = ZeroPoint.
template <int YDT, int ZDT, int ND>
__global__ __launch_bounds__(kBlock) void k_quant_v(const float* __restrict__ X, const float* __restrict__ S,
                                                    const void* __restrict__ Z, uint8_t* __restrict__ Y, BDesc d,
                                                    uint32_t nv) {
    const int inner = d.nd - 1;
    const int64_t ss = d.st[1][inner], sz = d.st[2][inner];
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t v = blockIdx.x * kBlock + threadIdx.x; v < nv; v += stride) {
        int64_t off[3];
        bd_offsets32<3, ND>(d, v * (uint32_t)kV, off);
        float x[kV];
#pragma unroll
        for (int q = 0; q < kV / 4; q++) {
            const float4 t = *reinterpret_cast<const float4*>(X + off[0] + 4 * q);
            x[4 * q] = t.x; x[4 * q + 1] = t.y; x[4 * q + 2] = t.z; x[4 * q + 3] = t.w;
        }
        uint32_t w[kV / 4];
        if (ss == 0 && sz == 0) {
            const double s = (double)S[off[1]], z = ld_d<ZDT>(Z, off[2]);
#pragma unroll
            for (int q = 0; q < kV / 4; q++) {
                uint32_t acc = 0;
#pragma unroll
                for (int b = 0; b < 4; b++) acc |= (uint32_t)code8<YDT>(qval((double)x[4 * q + b], s, z)) << (8 * b);
                w[q] = acc;
            }
        } else {
#pragma unroll
            for (int q = 0; q < kV / 4; q++) {
                uint32_t acc = 0;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const int t = 4 * q + b;
                    const double s = (double)S[off[1] + t * ss], z = ld_d<ZDT>(Z, off[2] + t * sz);
                    acc |= (uint32_t)code8<YDT>(qval((double)x[t], s, z)) << (8 * b);
                }
                w[q] = acc;
            }
        }
        *reinterpret_cast<uint4*>(Y + (size_t)v * kV) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// Dequantize 1-byte code -> f32, V elements per thread.
template <int XDT, int ZDT, int ND>
__global__ __launch_bounds__(kBlock) void k_dequant_v(const uint8_t* __restrict__ X, const float* __restrict__ S,
                                                      const void* __restrict__ Z, float* __restrict__ Y, BDesc d,
                                                      uint32_t nv) {
    const int inner = d.nd - 1;
    const int64_t ss = d.st[1][inner], sz = d.st[2][inner];
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t v = blockIdx.x * kBlock + threadIdx.x; v < nv; v += stride) {
        int64_t off[3];
        bd_offsets32<3, ND>(d, v * (uint32_t)kV, off);
        const uint4 raw = *reinterpret_cast<const uint4*>(X + off[0]);
        const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
        float y[kV];
        const bool uni = (ss == 0 && sz == 0);
        const double s0 = (double)S[off[1]], z0 = ld_d<ZDT>(Z, off[2]);
#pragma unroll
        for (int t = 0; t < kV; t++) {
            const uint8_t c = (uint8_t)(wv[t >> 2] >> (8 * (t & 3)));
            const double xv = ld_d<XDT>(&c, 0);
            const double s = uni ? s0 : (double)S[off[1] + t * ss];
            const double z = uni ? z0 : ld_d<ZDT>(Z, off[2] + t * sz);
            y[t] = (float)((xv - z) * s);
        }
        float* out = Y + (size_t)v * kV;
#pragma unroll
        for (int q = 0; q < kV / 4; q++)
            reinterpret_cast<float4*>(out)[q] = make_float4(y[4 * q], y[4 * q + 1], y[4 * q + 2], y[4 * q + 3]);
    }
}

// Generic: any dtypes, one element per thread, 64-bit indexing.
template <bool QUANT>
__global__ __launch_bounds__(kBlock) void k_qdq_rt(const void* __restrict__ X, int dtx, const void* __restrict__ S,
                                                   int dts, const void* __restrict__ Z, int dtz, void* __restrict__ Y,
                                                   int dty, BDesc d, size_t n) {
    const size_t stride = (size_t)gridDim.x * kBlock;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        int64_t off[3];
        if (n <= 0xFFFFFFFFull) bd_offsets32<3, 0>(d, (uint32_t)i, off);
        else bd_offsets64<3>(d, (int64_t)i, off);
        const double x = ld_d_rt(dtx, X, off[0]), s = ld_d_rt(dts, S, off[1]), z = ld_d_rt(dtz, Z, off[2]);
        st_d_rt(dty, Y, (int64_t)i, QUANT ? qval(x, s, z) : (x - z) * s);
    }
}

#define QND_SWITCH(nd, ...)                               \
    if (nd == 1) { constexpr int ND = 1; __VA_ARGS__; }   \
    else if (nd == 3) { constexpr int ND = 3; __VA_ARGS__; } \
    else { constexpr int ND = 0; __VA_ARGS__; }

#define ZDT_SWITCH(zdt, ...)                                          \
    switch (zdt) {                                                    \
    case kU8: { constexpr int ZD = kU8; __VA_ARGS__; } break;         \
    case kI8: { constexpr int ZD = kI8; __VA_ARGS__; } break;         \
    case kE4M3: { constexpr int ZD = kE4M3; __VA_ARGS__; } break;     \
    case kE5M2: { constexpr int ZD = kE5M2; __VA_ARGS__; } break;     \
    default: { constexpr int ZD = kF32; __VA_ARGS__; } break;         \
    }

inline bool is_code8(int dt) { return dt == kU8 || dt == kI8 || dt == kE4M3 || dt == kE5M2; }
inline bool zdt_fast(int dt) { return is_code8(dt) || dt == kF32; }

bool fast_ok(const BDesc& d, size_t n, const void* x, const void* y, size_t xalign) {
    return n < (size_t(1) << 31) && n % kV == 0 && d.dim[d.nd - 1] % kV == 0 && d.st[0][d.nd - 1] == 1 &&
           ((uintptr_t)x % xalign) == 0 && ((uintptr_t)y % 16) == 0;
}

template <bool QUANT>
void qdq_entry(const char* name, const Tensor* X, const Tensor* S, const Tensor* Z, Tensor* Y) {
    if (!tensor_sane(X, name) || !tensor_sane(S, name) || !tensor_sane(Z, name) || !tensor_sane(Y, name)) return;
    if (!ensure_device()) return;
    BDesc d;
    const Tensor* ops[3] = {X, S, Z};
    if (!make_bdesc_for(d, Y, ops, 3)) return;
    Staging st;
    const void* x = st.in(X);
    const void* s = st.in(S);
    const void* z = st.in(Z);
    void* y = st.out(Y, tensor_bytes(Y));
    if (!x || !s || !z || !y) { st.finish(); return; }
    const size_t n = Y->size;
    const int dtx = (int)X->dtype, dts = (int)S->dtype, dtz = (int)Z->dtype, dty = (int)Y->dtype;
    hipStream_t sm = stream();
    if (n) {
        bool launched = false;
        if (QUANT && dtx == kF32 && dts == kF32 && zdt_fast(dtz) && is_code8(dty) && fast_ok(d, n, x, y, 16)) {
            const uint32_t nv = (uint32_t)(n / kV);
            const dim3 g(grid_for(nv, kBlock)), b(kBlock);
#define QLAUNCH(YD)                                                                                           \
    ZDT_SWITCH(dtz, QND_SWITCH(d.nd, hipLaunchKernelGGL((k_quant_v<YD, ZD, ND>), g, b, 0, sm, (const float*)x,  \
                                                        (const float*)s, z, (uint8_t*)y, d, nv)))
            switch (dty) {
            case kU8: QLAUNCH(kU8); break;
            case kI8: QLAUNCH(kI8); break;
            case kE4M3: QLAUNCH(kE4M3); break;
            default: QLAUNCH(kE5M2); break;
            }
#undef QLAUNCH
            launched = true;
        } else if (!QUANT && is_code8(dtx) && dts == kF32 && zdt_fast(dtz) && dty == kF32 && fast_ok(d, n, x, y, 16)) {
            const uint32_t nv = (uint32_t)(n / kV);
            const dim3 g(grid_for(nv, kBlock)), b(kBlock);
#define DQLAUNCH(XD)                                                                                            \
    ZDT_SWITCH(dtz, QND_SWITCH(d.nd, hipLaunchKernelGGL((k_dequant_v<XD, ZD, ND>), g, b, 0, sm, (const uint8_t*)x, \
                                                        (const float*)s, z, (float*)y, d, nv)))
            switch (dtx) {
            case kU8: DQLAUNCH(kU8); break;
            case kI8: DQLAUNCH(kI8); break;
            case kE4M3: DQLAUNCH(kE4M3); break;
            default: DQLAUNCH(kE5M2); break;
            }
#undef DQLAUNCH
            launched = true;
        }
        if (!launched)
            hipLaunchKernelGGL((k_qdq_rt<QUANT>), dim3(grid_for(n, kBlock)), dim3(kBlock), 0, sm, x, dtx, s, dts, z,
                               dtz, y, dty, d, n);
        if (!check_launch(name)) { st.finish(); return; }
    }
    st.finish();
}

// Per-axis variant: 1-D Scale / ZeroPoint of length X->shape[axis] are viewed
// as [1, .., C, .., 1] (the reshape nn/Operators.py:439-445 does in Python).
template <bool QUANT>
void qdq_axis_entry(const char* name, const Tensor* X, const Tensor* S, const Tensor* Z, Tensor* Y, int axis) {
    if (!tensor_sane(X, name) || !tensor_sane(S, name) || !tensor_sane(Z, name) || !tensor_sane(Y, name)) return;
    if (axis < 0) axis += X->ndim;
    if (axis < 0 || axis >= X->ndim || X->ndim > 16) { set_error("%s: axis out of range", name); return; }
    const size_t c = (size_t)X->shape[axis];
    if ((S->size != c && S->size != 1) || (Z->size != c && Z->size != 1)) {
        set_error("%s: scale / zero point must have 1 or X.shape[axis] elements", name);
        return;
    }
    int shp[16];
    for (int i = 0; i < X->ndim; i++) shp[i] = (i == axis) ? (int)c : 1;
    Tensor sv = *S, zv = *Z;
    if (S->size == c) { sv.shape = shp; sv.ndim = X->ndim; }
    if (Z->size == c) { zv.shape = shp; zv.ndim = X->ndim; }
    // Y keeps X's shape; X itself indexes flat.
    Tensor yv = *Y;
    if (Y->size == X->size) { yv.shape = X->shape; yv.ndim = X->ndim; }
    qdq_entry<QUANT>(name, X, &sv, &zv, &yv);
}

}  // namespace
}  // namespace tohip

using namespace tohip;

extern "C" {
void quantize_linear_forward(const Tensor* X, const Tensor* Scale, const Tensor* ZeroPoint, Tensor* Y) {
    qdq_entry<true>("quantize_linear_forward", X, Scale, ZeroPoint, Y);
}
void dequantize_linear_forward(const Tensor* X, const Tensor* Scale, const Tensor* ZeroPoint, Tensor* Y) {
    qdq_entry<false>("dequantize_linear_forward", X, Scale, ZeroPoint, Y);
}
void quantize_linear_axis_forward(const Tensor* X, const Tensor* Scale, const Tensor* ZeroPoint, Tensor* Y,
                                  int axis) {
    qdq_axis_entry<true>("quantize_linear_axis_forward", X, Scale, ZeroPoint, Y, axis);
}
void dequantize_linear_axis_forward(const Tensor* X, const Tensor* Scale, const Tensor* ZeroPoint, Tensor* Y,
                                    int axis) {
    qdq_axis_entry<false>("dequantize_linear_axis_forward", X, Scale, ZeroPoint, Y, axis);
}
}
