// qdq.hip — QuantizeLinear / DequantizeLinear for gfx950.
//
// tensor_ops/tensor_ops.c:999-1034:
//   quantize:   y = s != 0 ? rint(x / s) + zp : zp   (double), then the output encoder
//   dequantize: y = (x - zp) * s                     (double), then the output encoder
// Scale and zero point are indexed through a broadcast descriptor against Y
// (scalar, per-axis or full-size), so nothing is materialised.
//
// Quantize fast path (exact).  The reference rounds the fp64 quotient
// q64 = RN64(x / s).  We form q32 = RN32(x * RN32(1 / s)), which is within
// 2^-23 |x/s| of the exact quotient, and q64 is within 2^-53 of it.  When q32
// lies more than 2^-22 |q32| away from the nearest half-integer (and
// |q32| < 2^22) all three values fall strictly inside the same rounding
// interval, so rint(q32) == rint(q64); the remaining lanes (about 2^-21 of
// them: near-ties, huge quotients, NaN / inf, s == 0) take the fp64 division.
// For integer outputs the fast path also needs an integral zero point, so
// that rint(q) + zp stays an exactly representable integer in fp32; fp8
// outputs are rounded once to fp32 exactly as the reference's (float)res.
//
// Launch shapes (measured on MI355X): quantize — one 16-byte f32 load per
// thread per iteration, 512-thread blocks, grid-stride over 2048 blocks;
// dequantize — four 4-byte code loads per thread, 256-thread blocks.  Both
// read and write with nontemporal (streaming) accesses.
#include "runtime.h"

namespace tohip {
namespace {

constexpr int kBlock = 256;
constexpr int kQBlock = 512;
constexpr int kQGrid = 2048;
constexpr int kU = 4;        // dequantize: 4-element groups per thread, group u of a block is one contiguous span

template <int YDT> __device__ __forceinline__ uint8_t code8(double r) {
    if constexpr (YDT == kU8) return (uint8_t)sat(cvt_i64(__builtin_rint(r)), 0, 255);
    else if constexpr (YDT == kI8) return (uint8_t)(int8_t)sat(cvt_i64(__builtin_rint(r)), -128, 127);
    else if constexpr (YDT == kI4) return (uint8_t)(int8_t)sat(cvt_i64(__builtin_rint(r)), -8, 7);
    else if constexpr (YDT == kE4M3) return enc_e4m3((float)r);
    else return enc_e5m2((float)r);
}

__device__ __forceinline__ double qval(double x, double s, double z) { return s != 0.0 ? __builtin_rint(x / s) + z : z; }

// Integral zero point small enough that rint(q) + zp (|rint(q)| < 2^22) stays
// an exact fp32 integer below 2^23, far from the int64 conversion limits.
__device__ __forceinline__ bool zint_ok(float zf, double z) {
    return __builtin_fabsf(zf) < 0x1p22f && __builtin_rintf(zf) == zf && (double)zf == z;
}

// Code of one element: fp32 fast path with the fp64 fallback described above.
// rs = RN32(1 / s); zint: the zero point is an integer (needed for int outputs).
template <int YDT>
__device__ __forceinline__ uint32_t qcode(float x, float s, float rs, float zf, double zd, bool zint) {
    const float q = x * rs;
    const float aq = __builtin_fabsf(q);
    const float d = __builtin_fabsf(__builtin_amdgcn_fractf(aq) - 0.5f);
    const bool ok = (aq < 0x1p22f) && (d > aq * 0x1p-22f) && (s != 0.0f) && (YDT == kE4M3 || YDT == kE5M2 || zint);
    if (__builtin_expect(ok, 1)) {
        const float r = __builtin_rintf(q) + zf;
        if constexpr (YDT == kU8) return (uint32_t)(int)__builtin_amdgcn_fmed3f(r, 0.0f, 255.0f);
        else if constexpr (YDT == kI8) return (uint32_t)(uint8_t)(int8_t)(int)__builtin_amdgcn_fmed3f(r, -128.0f, 127.0f);
        else if constexpr (YDT == kE4M3) return enc_e4m3(r);
        else return enc_e5m2(r);
    }
    return code8<YDT>(qval((double)x, (double)s, zd));
}

// Quantize f32 -> 1-byte code.  X and Y are flat (X has Y's size); Scale and
// ZeroPoint go through the descriptor (operands 1 and 2).  A thread handles
// 4 consecutive elements per iteration (one 16-byte load, one 4-byte store),
// so each load / store instruction is contiguous across the wave.
// Requires n % 4 == 0 and dim[nd-1] % 4 == 0.
template <int YDT, int ZDT, int ND>
__global__ __launch_bounds__(kQBlock) void k_quant_v(const float* __restrict__ X, const float* __restrict__ S,
                                                     const void* __restrict__ Z, uint8_t* __restrict__ Y, BDesc d,
                                                     uint32_t nv) {
    const int inner = d.nd - 1;
    const int64_t ss = d.st[1][inner], sz = d.st[2][inner];
    const bool uniform = (ND == 1) && ss == 0 && sz == 0;      // per-tensor scale / zero point
    const float su = S[0];
    const double zu = ld_d<ZDT>(Z, 0);
    const float rsu = 1.0f / su, zfu = (float)zu;
    const bool zintu = zint_ok(zfu, zu);
    const float4* X4 = reinterpret_cast<const float4*>(X);
    uint32_t* Y4 = reinterpret_cast<uint32_t*>(Y);
    for (uint32_t v = blockIdx.x * kQBlock + threadIdx.x; v < nv; v += gridDim.x * kQBlock) {
        const float4 xv = ld_stream(X4 + v);
        const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
        uint32_t w = 0;
        if (uniform) {
#pragma unroll
            for (int b = 0; b < 4; b++) w |= qcode<YDT>(xs[b], su, rsu, zfu, zu, zintu) << (8 * b);
        } else {
            int64_t off[3];
            bd_offsets32<3, ND>(d, v * 4u, off);
            if (ss == 0 && sz == 0) {                           // per-axis: one channel per group
                const float s = S[off[1]];
                const double z = ld_d<ZDT>(Z, off[2]);
                const float rs = 1.0f / s, zf = (float)z;
                const bool zi = zint_ok(zf, z);
#pragma unroll
                for (int b = 0; b < 4; b++) w |= qcode<YDT>(xs[b], s, rs, zf, z, zi) << (8 * b);
            } else {
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const float s = S[off[1] + b * ss];
                    const double z = ld_d<ZDT>(Z, off[2] + b * sz);
                    const float zf = (float)z;
                    w |= qcode<YDT>(xs[b], s, 1.0f / s, zf, z, zint_ok(zf, z)) << (8 * b);
                }
            }
        }
        st_stream(Y4 + v, w);
    }
}

// Dequantize 1-byte code -> f32: kU 4-byte code loads per thread, float4
// streaming stores.  (x - zp) * s is evaluated in fp64 and rounded once.
template <int XDT, int ZDT, int ND>
__global__ __launch_bounds__(kBlock) void k_dequant_v(const uint8_t* __restrict__ X, const float* __restrict__ S,
                                                      const void* __restrict__ Z, float* __restrict__ Y, BDesc d,
                                                      uint32_t nv) {
    const int inner = d.nd - 1;
    const int64_t ss = d.st[1][inner], sz = d.st[2][inner];
    const bool uniform = (ND == 1) && ss == 0 && sz == 0;
    const double su = (double)S[0], zu = ld_d<ZDT>(Z, 0);
    const uint32_t* X4 = reinterpret_cast<const uint32_t*>(X);
    float4* Y4 = reinterpret_cast<float4*>(Y);
    for (uint32_t base = blockIdx.x * (kBlock * kU); base < nv; base += gridDim.x * (kBlock * kU)) {
        uint32_t xv[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const uint32_t v = base + u * kBlock + threadIdx.x;
            if (v < nv) xv[u] = X4[v];
        }
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const uint32_t v = base + u * kBlock + threadIdx.x;
            if (v >= nv) continue;
            float y[4];
            int64_t off[3] = {0, 0, 0};
            if (!uniform) bd_offsets32<3, ND>(d, v * 4u, off);
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const uint8_t c = (uint8_t)(xv[u] >> (8 * b));
                const double x = ld_d<XDT>(&c, 0);
                const double s = uniform ? su : (double)S[off[1] + b * ss];
                const double z = uniform ? zu : ld_d<ZDT>(Z, off[2] + b * sz);
                y[b] = (float)((x - z) * s);
            }
            st_stream(Y4 + v, make_float4(y[0], y[1], y[2], y[3]));
        }
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

// Fast kernels: X flat with Y's size, 4-element groups sharing outer coordinates.
bool fast_ok(const BDesc& d, const Tensor* X, size_t n, const void* x, const void* y) {
    return X->size == n && n < (size_t(1) << 31) && n % 4 == 0 && d.dim[d.nd - 1] % 4 == 0 &&
           ((uintptr_t)x % 16) == 0 && ((uintptr_t)y % 16) == 0;
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
        if (QUANT && dtx == kF32 && dts == kF32 && zdt_fast(dtz) && is_code8(dty) && fast_ok(d, X, n, x, y)) {
            const uint32_t nv = (uint32_t)(n / 4);
            const dim3 g(grid_for(nv, kQBlock, kQGrid)), b(kQBlock);
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
        } else if (!QUANT && is_code8(dtx) && dts == kF32 && zdt_fast(dtz) && dty == kF32 && fast_ok(d, X, n, x, y)) {
            const uint32_t nv = (uint32_t)(n / 4);
            const dim3 g(grid_for(nv, kBlock * kU)), b(kBlock);
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
