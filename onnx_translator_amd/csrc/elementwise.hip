// elementwise.hip — Relu, Abs, Cos, Add, Sub, Mul, Div and their fused chain for gfx950.
//
// Memory-bound kernels: each thread moves 16-byte vectors along the
// innermost (collapsed) dimension, broadcast operands are indexed through a
// collapsed stride descriptor (no materialised copies), and launches cover
// the tensor once with 256-thread blocks.  Numerics follow
// tensor_ops/tensor_ops.c:708-997 exactly:
//   * f32 (+-*/) f32 -> f32 runs natively in fp32: double-then-round equals
//     the correctly rounded fp32 op because 53 >= 2*24 + 2;
//   * every other float combination computes in fp64 and rounds through the
//     output encoder; integer outputs use the int64 path with saturation;
//   * Cos replays the reference's 4097-entry table lookup in fp64 with
//     contraction off, which reproduces its bits.
#include "runtime.h"

namespace tohip {
namespace {

enum { OP_ADD = 0, OP_SUB = 1, OP_MUL = 2, OP_DIV = 3 };
enum { U_RELU = 0, U_ABS = 1, U_COS = 2 };

constexpr int kBlock = 256;

template <int OP> __device__ __forceinline__ float fop(float a, float b) {
    if constexpr (OP == OP_ADD) return a + b;
    else if constexpr (OP == OP_SUB) return a - b;
    else if constexpr (OP == OP_MUL) return a * b;
    else return a / b;
}
template <int OP> __device__ __forceinline__ double dop(double a, double b) {
    if constexpr (OP == OP_ADD) return a + b;
    else if constexpr (OP == OP_SUB) return a - b;
    else if constexpr (OP == OP_MUL) return a * b;
    else return a / b;
}
// tensor_ops.c:681-684 with two's-complement wrap (the x86 build wraps).
template <int OP> __device__ __forceinline__ int64_t iop(int64_t a, int64_t b) {
    const uint64_t ua = (uint64_t)a, ub = (uint64_t)b;
    if constexpr (OP == OP_ADD) return (int64_t)(ua + ub);
    else if constexpr (OP == OP_SUB) return (int64_t)(ua - ub);
    else if constexpr (OP == OP_MUL) return (int64_t)(ua * ub);
    else {
        if (b == 0) return a >= 0 ? INT64_MAX : INT64_MIN;
        if (a == INT64_MIN && b == -1) return INT64_MIN;
        return a / b;
    }
}

// fmod(a, 2pi) for a = |x|, exactly.  Below 2^30 the quotient q = trunc(a / 2pi)
// is found from a * (1 / 2pi) to within one, and fma(-q, 2pi, a) is exact
// for the right q (the remainder of fmod is representable and the fma rounds
// the exact value a - q * 2pi once); an off-by-one q shows as r < 0 or
// r >= 2pi and is corrected the same way.  Larger (or non-finite) a uses fmod.
__device__ __forceinline__ double fmod_two_pi(double a) {
    const double two_pi = 2.0 * 3.141592653589793238462643383279502884197;
    if (!(a < 0x1p30)) return fmod(a, two_pi);
    const double q = __builtin_trunc(a * (1.0 / two_pi));
    double r = __builtin_fma(-q, two_pi, a);
    if (r < 0.0) r = __builtin_fma(-(q - 1.0), two_pi, a);
    else if (r >= two_pi) r = __builtin_fma(-(q + 1.0), two_pi, a);
    return r;
}

// tensor_ops.c:815-833: r = fmod(|x|, 2pi); pos = r * 4096 / 2pi; lerp.
__device__ __forceinline__ double lut_cos(double x, const double* __restrict__ T) {
    const double two_pi = 2.0 * 3.141592653589793238462643383279502884197;
    const double r = fmod_two_pi(fabs(x));
    if (r != r) return r;                              // NaN / inf input
    const double pos = r * 4096.0 / two_pi;
    int k = (int)pos;
    double w = pos - (double)k;
    if (k >= 4096) { k = 4095; w = 0.0; }
    return T[k] * (1.0 - w) + T[k + 1] * w;
}

__device__ __forceinline__ float abs_f32(float v) {
    uint32_t u = f2u(v) & 0x7FFFFFFFu;
    if (u > 0x7F800000u) u |= 0x00400000u;            // fabs through double quiets NaN
    return u2f(u);
}

template <int U> __device__ __forceinline__ float unary_f32(float v, const double* T) {
    if constexpr (U == U_RELU) return v > 0.0f ? v : 0.0f;
    else if constexpr (U == U_ABS) return abs_f32(v);
    else return (float)lut_cos((double)v, T);
}

// ---------------------------------------------------------------- unary ---
template <int U>
__global__ __launch_bounds__(kBlock) void k_unary_f32(const float* __restrict__ X, float* __restrict__ Y,
                                                      size_t n, const double* __restrict__ T) {
    const size_t nv = n / 4;
    const size_t stride = (size_t)gridDim.x * kBlock;
    for (size_t v = (size_t)blockIdx.x * kBlock + threadIdx.x; v < nv; v += stride) {
        const float4 x = ld_stream(reinterpret_cast<const float4*>(X) + v);
        float4 y;
        y.x = unary_f32<U>(x.x, T);
        y.y = unary_f32<U>(x.y, T);
        y.z = unary_f32<U>(x.z, T);
        y.w = unary_f32<U>(x.w, T);
        st_stream(reinterpret_cast<float4*>(Y) + v, y);
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        const size_t i = nv * 4 + threadIdx.x;
        Y[i] = unary_f32<U>(X[i], T);
    }
}

// Any dtypes: tensor_ops.c:708-757 (int input -> int64 path), :840-854 (cos, double path).
template <int U>
__global__ __launch_bounds__(kBlock) void k_unary_rt(const void* __restrict__ X, int dtx, void* __restrict__ Y,
                                                     int dty, size_t n, const double* __restrict__ T) {
    const size_t stride = (size_t)gridDim.x * kBlock;
    const bool int_in = (U != U_COS) && dt_is_int(dtx);
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        if (int_in) {
            const int64_t v = ld_i_rt(dtx, X, (int64_t)i);
            int64_t r;
            if constexpr (U == U_RELU) r = v > 0 ? v : 0;
            else r = v == INT64_MIN ? INT64_MAX : (v < 0 ? -v : v);
            st_i_rt(dty, Y, (int64_t)i, r);
        } else {
            const double v = ld_d_rt(dtx, X, (int64_t)i);
            double r;
            if constexpr (U == U_RELU) r = v > 0 ? v : 0.0;
            else if constexpr (U == U_ABS) r = fabs(v);
            else r = lut_cos(v, T);
            st_d_rt(dty, Y, (int64_t)i, r);
        }
    }
}

// --------------------------------------------------------------- binary ---
// stream: the operand is read once (full size), so use nontemporal loads.
__device__ __forceinline__ float4 load4(const float* __restrict__ p, int64_t off, int64_t st, bool stream) {
    if (st == 1) return stream ? ld_stream(reinterpret_cast<const float4*>(p + off))
                               : *reinterpret_cast<const float4*>(p + off);
    if (st == 0) { const float v = p[off]; return make_float4(v, v, v, v); }
    return make_float4(p[off], p[off + st], p[off + 2 * st], p[off + 3 * st]);
}

// f32 x f32 -> f32, vectorised; requires dim[nd-1] % 4 == 0 and 16-byte aligned bases.
template <int OP, int ND>
__global__ __launch_bounds__(kBlock) void k_bin_f32_v4(const float* __restrict__ A, const float* __restrict__ B,
                                                       float* __restrict__ O, BDesc d, uint32_t nv,
                                                       int stream_a, int stream_b) {
    const int64_t sa = d.st[0][d.nd - 1], sb = d.st[1][d.nd - 1];
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t v = blockIdx.x * kBlock + threadIdx.x; v < nv; v += stride) {
        int64_t off[2];
        bd_offsets32<2, ND>(d, v * 4u, off);
        const float4 a = load4(A, off[0], sa, stream_a != 0);
        const float4 b = load4(B, off[1], sb, stream_b != 0);
        float4 o;
        o.x = fop<OP>(a.x, b.x);
        o.y = fop<OP>(a.y, b.y);
        o.z = fop<OP>(a.z, b.z);
        o.w = fop<OP>(a.w, b.w);
        st_stream(reinterpret_cast<float4*>(O) + v, o);
    }
}

// f32 x f32 -> f32, one element per thread (any broadcast pattern).
template <int OP, int ND>
__global__ __launch_bounds__(kBlock) void k_bin_f32_s(const float* __restrict__ A, const float* __restrict__ B,
                                                      float* __restrict__ O, BDesc d, uint32_t n) {
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t i = blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        int64_t off[2];
        bd_offsets32<2, ND>(d, i, off);
        O[i] = fop<OP>(A[off[0]], B[off[1]]);
    }
}

// Typed fp64 path for the hot mixed combinations (e.g. int32 + f32 -> f64 / f32).
template <int OP, int DA, int DB, int DO, int ND>
__global__ __launch_bounds__(kBlock) void k_bin_typed(const void* __restrict__ A, const void* __restrict__ B,
                                                      void* __restrict__ O, BDesc d, uint32_t n) {
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t i = blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        int64_t off[2];
        bd_offsets32<2, ND>(d, i, off);
        st_d<DO>(O, (int64_t)i, dop<OP>(ld_d<DA>(A, off[0]), ld_d<DB>(B, off[1])));
    }
}

// Any dtypes (runtime switch); 64-bit indexing.
template <int OP, bool INTOUT>
__global__ __launch_bounds__(kBlock) void k_bin_rt(const void* __restrict__ A, int dta, const void* __restrict__ B,
                                                   int dtb, void* __restrict__ O, int dto, BDesc d, size_t n) {
    const size_t stride = (size_t)gridDim.x * kBlock;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        int64_t off[2];
        if (n <= 0xFFFFFFFFull) bd_offsets32<2, 0>(d, (uint32_t)i, off);
        else bd_offsets64<2>(d, (int64_t)i, off);
        if constexpr (INTOUT) {
            st_i_rt(dto, O, (int64_t)i, iop<OP>(ld_i_rt(dta, A, off[0]), ld_i_rt(dtb, B, off[1])));
        } else {
            st_d_rt(dto, O, (int64_t)i, dop<OP>(ld_d_rt(dta, A, off[0]), ld_d_rt(dtb, B, off[1])));
        }
    }
}

#define ND_SWITCH(nd, ...)                              \
    switch (nd) {                                       \
    case 1: { constexpr int ND = 1; __VA_ARGS__; } break; \
    case 2: { constexpr int ND = 2; __VA_ARGS__; } break; \
    case 3: { constexpr int ND = 3; __VA_ARGS__; } break; \
    case 4: { constexpr int ND = 4; __VA_ARGS__; } break; \
    default: { constexpr int ND = 0; __VA_ARGS__; } break; \
    }

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <int OP>
bool launch_binary(const void* A, int dta, const void* B, int dtb, void* O, int dto, const BDesc& d, size_t n,
                   size_t sz_a, size_t sz_b) {
    hipStream_t s = stream();
    if (n == 0) return true;
    const bool small = n < (size_t(1) << 31);   // 32-bit loop counters cannot wrap
    if (dt_is_int(dto)) {
        hipLaunchKernelGGL((k_bin_rt<OP, true>), dim3(grid_for(n, kBlock)), dim3(kBlock), 0, s, A, dta, B, dtb, O,
                           dto, d, n);
        return check_launch("binary (int)");
    }
    if (small && dta == kF32 && dtb == kF32 && dto == kF32) {
        const float* a = (const float*)A;
        const float* b = (const float*)B;
        float* o = (float*)O;
        const bool v4 = (d.dim[d.nd - 1] % 4u == 0) && aligned16(a) && aligned16(b) && aligned16(o);
        if (v4) {
            const uint32_t nv = (uint32_t)(n / 4);
            ND_SWITCH(d.nd, hipLaunchKernelGGL((k_bin_f32_v4<OP, ND>), dim3(grid_for(nv, kBlock)), dim3(kBlock), 0, s,
                                               a, b, o, d, nv, sz_a == n, sz_b == n));
        } else {
            ND_SWITCH(d.nd, hipLaunchKernelGGL((k_bin_f32_s<OP, ND>), dim3(grid_for(n, kBlock)), dim3(kBlock), 0, s,
                                               a, b, o, d, (uint32_t)n));
        }
        return check_launch("binary f32");
    }
    if (small && dta == kI32 && dtb == kF32 && (dto == kF64 || dto == kF32)) {
        const uint32_t nn = (uint32_t)n;
        if (dto == kF64) {
            ND_SWITCH(d.nd, hipLaunchKernelGGL((k_bin_typed<OP, kI32, kF32, kF64, ND>), dim3(grid_for(n, kBlock)),
                                               dim3(kBlock), 0, s, A, B, O, d, nn));
        } else {
            ND_SWITCH(d.nd, hipLaunchKernelGGL((k_bin_typed<OP, kI32, kF32, kF32, ND>), dim3(grid_for(n, kBlock)),
                                               dim3(kBlock), 0, s, A, B, O, d, nn));
        }
        return check_launch("binary i32/f32");
    }
    hipLaunchKernelGGL((k_bin_rt<OP, false>), dim3(grid_for(n, kBlock)), dim3(kBlock), 0, s, A, dta, B, dtb, O, dto,
                       d, n);
    return check_launch("binary");
}

template <int OP>
void binary_entry(const char* name, const Tensor* A, const Tensor* B, Tensor* O) {
    if (!tensor_sane(A, name) || !tensor_sane(B, name) || !tensor_sane(O, name)) return;
    if (!ensure_device()) return;
    BDesc d;
    const Tensor* ops[2] = {A, B};
    // Equal sizes index flat (the reference); otherwise numpy broadcasting to
    // O's shape (the reference returns there; its Python caller broadcasts first).
    if (!make_bdesc_for(d, O, ops, 2)) return;
    Staging st;
    const void* a = st.in(A);
    const void* b = st.in(B);
    void* o = st.out(O, tensor_bytes(O));
    if (!a || !b || !o) { st.finish(); return; }
    if (!launch_binary<OP>(a, (int)A->dtype, b, (int)B->dtype, o, (int)O->dtype, d, O->size, A->size, B->size)) {
        st.finish();
        return;
    }
    st.finish();
}

template <int U>
void unary_entry(const char* name, const Tensor* X, Tensor* Y) {
    if (!tensor_sane(X, name) || !tensor_sane(Y, name)) return;
    if (X->size != Y->size) { set_error("%s: input and output sizes differ", name); return; }
    if (!ensure_device()) return;
    const double* T = nullptr;
    if (U == U_COS && !(T = device_cos_lut())) return;
    Staging st;
    const void* x = st.in(X);
    void* y = st.out(Y, tensor_bytes(Y));
    if (!x || !y) { st.finish(); return; }
    const size_t n = X->size;
    hipStream_t s = stream();
    if (n) {
        if (X->dtype == DTYPE_FLOAT32 && Y->dtype == DTYPE_FLOAT32 && aligned16(x) && aligned16(y)) {
            hipLaunchKernelGGL((k_unary_f32<U>), dim3(grid_for(n / 4 + 1, kBlock)), dim3(kBlock), 0, s,
                               (const float*)x, (float*)y, n, T);
        } else {
            hipLaunchKernelGGL((k_unary_rt<U>), dim3(grid_for(n, kBlock)), dim3(kBlock), 0, s, x, (int)X->dtype, y,
                               (int)Y->dtype, n, T);
        }
        if (!check_launch(name)) { st.finish(); return; }
    }
    st.finish();
}

// ------------------------------------------------------------ fused chain ---
// One pass over X applying a sequence of the operators above (the config-1
// chain Add -> Mul -> Sub -> Div -> Relu -> Abs -> Cos, or any other), f32
// throughout.  Each step rounds to f32 exactly as the standalone operator
// writes its output (native fp32 + - * /, Relu / Abs bit rules, the Cos table
// in fp64), so the result is the op-by-op result bit for bit while the
// intermediates never leave registers.  Operand k (at most 3) is broadcast
// to X's shape through the descriptor (operand k + 1 of d).
// The program is packed 8 bits per step (op | operand << 3 | reversed << 5)
// into two 64-bit words held in scalar registers, so the unrolled step loop
// decodes it with shifts instead of indexing the kernel argument memory.
constexpr int kChainMaxSteps = 16, kChainMaxOperands = kMaxOperands - 1;
struct ChainProg {
    int n;
    uint64_t code[2];
};

// One step on the W values of a thread: one (uniform) dispatch per step.
template <int W>
__device__ __forceinline__ void chain_step(int op, float (&v)[W], const float (&b)[W], int rev, const double* T) {
    switch (op) {
    case TENSOR_OPS_CHAIN_ADD:
#pragma unroll
        for (int e = 0; e < W; e++) v[e] = rev ? b[e] + v[e] : v[e] + b[e];
        break;
    case TENSOR_OPS_CHAIN_SUB:
#pragma unroll
        for (int e = 0; e < W; e++) v[e] = rev ? b[e] - v[e] : v[e] - b[e];
        break;
    case TENSOR_OPS_CHAIN_MUL:
#pragma unroll
        for (int e = 0; e < W; e++) v[e] = rev ? b[e] * v[e] : v[e] * b[e];
        break;
    case TENSOR_OPS_CHAIN_DIV:
#pragma unroll
        for (int e = 0; e < W; e++) v[e] = rev ? b[e] / v[e] : v[e] / b[e];
        break;
    case TENSOR_OPS_CHAIN_RELU:
#pragma unroll
        for (int e = 0; e < W; e++) v[e] = unary_f32<U_RELU>(v[e], T);
        break;
    case TENSOR_OPS_CHAIN_ABS:
#pragma unroll
        for (int e = 0; e < W; e++) v[e] = unary_f32<U_ABS>(v[e], T);
        break;
    default:
#pragma unroll
        for (int e = 0; e < W; e++) v[e] = unary_f32<U_COS>(v[e], T);
        break;
    }
}

// V4: eight consecutive elements per thread as two float4 (inner dim % 8 == 0,
// 16-byte aligned), which amortises the per-step dispatch; else one element.
template <int ND, bool V4>
__global__ __launch_bounds__(kBlock) void k_chain_f32(const float* __restrict__ X, const float* __restrict__ B0,
                                                      const float* __restrict__ B1, const float* __restrict__ B2,
                                                      float* __restrict__ Y, BDesc d, ChainProg prog, uint32_t nitems,
                                                      int stream_x, const double* __restrict__ T) {
    constexpr int W = V4 ? 8 : 1;
    const float* Bp[3] = {B0, B1, B2};
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t it = blockIdx.x * kBlock + threadIdx.x; it < nitems; it += stride) {
        int64_t off[kMaxOperands];
        bd_offsets32<kMaxOperands, ND>(d, it * W, off);
        float v[W], b[kChainMaxOperands][W];
        if constexpr (V4) {
            const int64_t sx = d.st[0][d.nd - 1];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const float4 x = load4(X, off[0] + 4 * h * sx, sx, stream_x != 0);
                v[4 * h] = x.x; v[4 * h + 1] = x.y; v[4 * h + 2] = x.z; v[4 * h + 3] = x.w;
            }
        } else {
            v[0] = X[off[0]];
        }
#pragma unroll
        for (int k = 0; k < kChainMaxOperands; k++) {
            if (!Bp[k]) continue;
            if constexpr (V4) {
                const int64_t sb = d.st[k + 1][d.nd - 1];
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const float4 t = load4(Bp[k], off[k + 1] + 4 * h * sb, sb, false);
                    b[k][4 * h] = t.x; b[k][4 * h + 1] = t.y; b[k][4 * h + 2] = t.z; b[k][4 * h + 3] = t.w;
                }
            } else {
                b[k][0] = Bp[k][off[k + 1]];
            }
        }
        for (int sidx = 0; sidx < prog.n; sidx++) {
            const uint32_t c = (uint32_t)(prog.code[sidx >> 3] >> (8 * (sidx & 7))) & 0xFFu;
            const int a = (c >> 3) & 3;
            float bb[W];
#pragma unroll
            for (int e = 0; e < W; e++) bb[e] = a == 0 ? b[0][e] : (a == 1 ? b[1][e] : b[2][e]);
            chain_step<W>((int)(c & 7u), v, bb, (int)((c >> 5) & 1u), T);
        }
        if constexpr (V4) {
            st_stream(reinterpret_cast<float4*>(Y) + 2 * it, make_float4(v[0], v[1], v[2], v[3]));
            st_stream(reinterpret_cast<float4*>(Y) + 2 * it + 1, make_float4(v[4], v[5], v[6], v[7]));
        } else {
            Y[it] = v[0];
        }
    }
}

void chain_entry(const Tensor* X, const Tensor* const* operands, int noperands, const TensorOpsChainStep* steps,
                 int nsteps, Tensor* Y) {
    const char* name = "elementwise_chain_forward";
    if (!tensor_sane(X, name) || !tensor_sane(Y, name)) return;
    if (noperands < 0 || noperands > kChainMaxOperands) { set_error("%s: at most %d operands", name, kChainMaxOperands); return; }
    if (nsteps < 0 || nsteps > kChainMaxSteps || (nsteps && !steps)) { set_error("%s: 0..%d steps", name, kChainMaxSteps); return; }
    if (X->dtype != DTYPE_FLOAT32 || Y->dtype != DTYPE_FLOAT32) { set_error("%s: float32 X and Y only", name); return; }
    if (X->size != Y->size) { set_error("%s: X and Y sizes differ", name); return; }
    ChainProg prog{};
    prog.n = nsteps;
    bool cos = false;
    for (int i = 0; i < nsteps; i++) {
        const int op = steps[i].op;
        if (op < TENSOR_OPS_CHAIN_ADD || op > TENSOR_OPS_CHAIN_COS) { set_error("%s: step %d: unknown op %d", name, i, op); return; }
        const bool bin = op <= TENSOR_OPS_CHAIN_DIV;
        if (bin && (steps[i].operand < 0 || steps[i].operand >= noperands)) {
            set_error("%s: step %d: operand %d out of range", name, i, steps[i].operand);
            return;
        }
        const uint64_t c = (uint64_t)op | ((uint64_t)(bin ? steps[i].operand : 0) << 3) |
                           ((uint64_t)(bin && steps[i].reversed ? 1 : 0) << 5);
        prog.code[i >> 3] |= c << (8 * (i & 7));
        cos |= op == TENSOR_OPS_CHAIN_COS;
    }
    const Tensor* ops[kMaxOperands] = {Y, nullptr, nullptr, nullptr};
    ops[0] = X;
    for (int k = 0; k < noperands; k++) {
        if (!tensor_sane(operands[k], name)) return;
        if (operands[k]->dtype != DTYPE_FLOAT32) { set_error("%s: float32 operands only", name); return; }
        ops[k + 1] = operands[k];
    }
    if (!ensure_device()) return;
    const double* T = nullptr;
    if (cos && !(T = device_cos_lut())) return;
    BDesc d;
    if (!make_bdesc_for(d, Y, ops, 1 + noperands)) return;
    Staging st;
    const float* x = (const float*)st.in(X);
    const float* b[kChainMaxOperands] = {nullptr, nullptr, nullptr};
    for (int k = 0; k < noperands; k++)
        if (!(b[k] = (const float*)st.in(operands[k]))) { st.finish(); return; }
    float* y = (float*)st.out(Y, tensor_bytes(Y));
    if (!x || !y) { st.finish(); return; }
    const size_t n = Y->size;
    if (n) {
        if (n >= ((size_t)1 << 31)) { set_error("%s: more than 2^31 elements", name); st.finish(); return; }
        bool v4 = d.dim[d.nd - 1] % 8u == 0 && aligned16(x) && aligned16(y);
        for (int k = 0; k < noperands; k++) v4 = v4 && aligned16(b[k]);
        hipStream_t s = stream();
        if (v4) {
            const uint32_t nv = (uint32_t)(n / 8);
            ND_SWITCH(d.nd, hipLaunchKernelGGL((k_chain_f32<ND, true>), dim3(grid_for(nv, kBlock)), dim3(kBlock), 0, s,
                                               x, b[0], b[1], b[2], y, d, prog, nv, 1, T));
        } else {
            ND_SWITCH(d.nd, hipLaunchKernelGGL((k_chain_f32<ND, false>), dim3(grid_for(n, kBlock)), dim3(kBlock), 0, s,
                                               x, b[0], b[1], b[2], y, d, prog, (uint32_t)n, 0, T));
        }
        if (!check_launch(name)) { st.finish(); return; }
    }
    st.finish();
}

}  // namespace
}  // namespace tohip

using namespace tohip;

extern "C" {
void elementwise_chain_forward(const Tensor* X, const Tensor* const* operands, int noperands,
                               const TensorOpsChainStep* steps, int nsteps, Tensor* Y) {
    chain_entry(X, operands, noperands, steps, nsteps, Y);
}
void relu_forward(const Tensor* input, Tensor* output) { unary_entry<U_RELU>("relu_forward", input, output); }
void abs_forward(const Tensor* input, Tensor* output) { unary_entry<U_ABS>("abs_forward", input, output); }
void cos_forward(const Tensor* input, Tensor* output) { unary_entry<U_COS>("cos_forward", input, output); }
void add_forward(const Tensor* A, const Tensor* B, Tensor* O) { binary_entry<OP_ADD>("add_forward", A, B, O); }
void sub_forward(const Tensor* A, const Tensor* B, Tensor* O) { binary_entry<OP_SUB>("sub_forward", A, B, O); }
void mul_forward(const Tensor* A, const Tensor* B, Tensor* O) { binary_entry<OP_MUL>("mul_forward", A, B, O); }
void div_forward(const Tensor* A, const Tensor* B, Tensor* O) { binary_entry<OP_DIV>("div_forward", A, B, O); }
}
