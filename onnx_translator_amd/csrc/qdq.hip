// qdq.hip — QuantizeLinear / DequantizeLinear / DynamicQuantizeLinear for gfx950.
//
// tensor_ops/tensor_ops.c:999-1034:
//   quantize:   y = s != 0 ? rint(x / s) + zp : zp   (double), then the output encoder
//   dequantize: y = (x - zp) * s                     (double), then the output encoder
// Scale and zero point are indexed through a broadcast descriptor against Y
// (scalar, per-axis or full-size), so nothing is materialised.
//
// Quantize fast path (exact, branch-free).  The reference rounds the fp64
// quotient: rint(RN64(x / s)).  For fp32 x and s that equals the
// round-half-even of the exact rational x / s whenever |x / s| < 2^27: for a
// quotient that is not a half-integer, x / s - (k + 1/2) = (2x - (2k+1)s) / 2s,
// whose numerator is a nonzero multiple of 2^(min(ex,es)-23), so the distance
// to the nearest half-integer is at least 2^-25 once ex >= es (and larger
// otherwise), while RN64's error is at most 2^(ex-es-52) < 2^-25 below 2^27:
// RN64 neither creates nor crosses a tie.  Per element the kernel forms
//     r = rint(x * rcp(s))            (any approximation of 1/s will do)
//     rho = fma(-r, s, x)             (= RN32(x - r s), one rounding)
// and accepts r when |rho| < |s| / 2.  RN32 is monotone and |s| / 2 is exact, so
// |rho| < |s|/2 implies |x - r s| < |s|/2, i.e. r is the unique nearest integer
// to x / s.  Every other lane (ties, a poor r, s == 0, s or x NaN / inf, huge
// quotients) takes the fp64 division, under one wave-level branch.
// The zero point must be integral with |zp| < 2^22 for the fast path, so that
// v = r + zp is an exact fp32 integer below 2^24 whenever |r| < 2^23; beyond
// that every output format saturates (or, e5m2, overflows to inf) for both v
// and the reference's value, so the result is the same code.  Codes are formed
// by hardware conversions, each checked against the reference encoders over
// all 2^32 fp32 inputs on gfx950:
//   u8 / i8  v_cvt_pk_u8_f32 rounds half-even and clamps to [0, 255]; on an
//            exact integer v it is the reference's saturate((int64_t)rint(v))
//            (i8 adds 128 first and flips bit 7 after);
//   e4m3     v_cvt_pk_fp8_f32 equals the reference encoder for every input of
//            magnitude >= 2^-6 up to 464 and for +-0; integers are clamped to
//            +-448 first (the reference saturates to 0x7E);
//   e5m2     v_cvt_pk_bf8_f32 equals the reference encoder for every non-NaN
//            input of magnitude >= 2^-14 (including overflow to inf) and +-0.
// Integral v never falls in the flush-to-zero band, so the hardware's
// subnormal outputs never arise.
//
// Launch shapes (swept on MI355X; 64 MiB f32 <-> 16 MiB codes, not cache-resident):
// quantize — software-pipelined grid-stride loop, kQU 16-byte nontemporal
// loads per thread, plain 4-byte stores (nontemporal 4-byte stores cost ~1 us),
// 256-thread blocks, 8 blocks per CU; dequantize — four 4-byte code loads per
// thread issued together, one 16-byte nontemporal store per code word,
// 256-thread blocks, full grid.
#include <algorithm>
#include <mutex>
#include <cfloat>

#include "quant.h"
#include "runtime.h"

namespace tohip {
namespace {

constexpr int kBlock = 256;

// Codes of four fast-path values, little-endian in one word.
template <int YDT>
__device__ __forceinline__ uint32_t qpack4(float v0, float v1, float v2, float v3) {
    uint32_t w;
    if constexpr (YDT == kU8 || YDT == kI8) {
        w = __builtin_amdgcn_cvt_pk_u8_f32(v0, 0, 0u);
        w = __builtin_amdgcn_cvt_pk_u8_f32(v1, 1, w);
        w = __builtin_amdgcn_cvt_pk_u8_f32(v2, 2, w);
        w = __builtin_amdgcn_cvt_pk_u8_f32(v3, 3, w);
        if constexpr (YDT == kI8) w ^= 0x80808080u;
    } else if constexpr (YDT == kE4M3) {
        v0 = __builtin_amdgcn_fmed3f(v0, -448.0f, 448.0f);
        v1 = __builtin_amdgcn_fmed3f(v1, -448.0f, 448.0f);
        v2 = __builtin_amdgcn_fmed3f(v2, -448.0f, 448.0f);
        v3 = __builtin_amdgcn_fmed3f(v3, -448.0f, 448.0f);
        w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
        w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v2, v3, (int)w, true);
    } else {
        w = (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(v0, v1, 0, false);
        w = (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(v2, v3, (int)w, true);
    }
    return w;
}

// The reference's arithmetic for four elements: fp64 quotient, rint, + zp.
template <int YDT>
__device__ __forceinline__ uint32_t qslow4(float x0, float x1, float x2, float x3, float s, double zd) {
    const double sd = (double)s;
    return (uint32_t)code8<YDT>(qval((double)x0, sd, zd)) | ((uint32_t)code8<YDT>(qval((double)x1, sd, zd)) << 8) |
           ((uint32_t)code8<YDT>(qval((double)x2, sd, zd)) << 16) |
           ((uint32_t)code8<YDT>(qval((double)x3, sd, zd)) << 24);
}

template <int YDT>
__device__ __forceinline__ uint8_t qslow1(float x, float s, double zd) {
    return code8<YDT>(qval((double)x, (double)s, zd));
}

// One unit of work: 4 consecutive elements (one 16-byte X load or one 4-byte
// code word) with the scale / zero-point values they need, loaded together so
// that the parameter loads overlap the data loads.  MODE 0: one pair for the
// tensor (not stored per unit); 1: one pair per unit; 2: one pair per element;
// 3: one pair per wave — a wave's units are one run of consecutive elements
// (256 for dequantize, 256 * kQU per tile for quantize) starting at a multiple
// of the run, and the parameters change only every `inner` elements, a
// multiple of the run, so the wave shares one pair, located from its first
// unit's index (uniform: its address math and loads go to the scalar unit).
template <int ZDT> using zraw_t = typename std::conditional<ZDT == kF32, float, uint8_t>::type;

template <int ZDT, int MODE>
struct Params {
    static constexpr int kN = MODE == 2 ? 4 : 1;
    float s[kN];
    zraw_t<ZDT> z[kN];
};

// Per-axis parameters (MODE 1 and 3): element e uses Scale[(e / inner) % C]
// and ZeroPoint[zs * ((e / inner) % C)], zs = 0 for a single zero point.
// MODE 3 reads them through buffer resources of this extent (the indices stay
// inside the tensors; the extent only has to cover them).
constexpr uint32_t kParamReach = 0x7FFFFFF0u;
struct AxisDesc {
    FastDiv inner, c;
    uint32_t zs;
};

template <int ZDT, int MODE, int ND>
__device__ __forceinline__ void load_params(Params<ZDT, MODE>& p, const float* S, const void* Z, const BDesc& d,
                                            const AxisDesc& ax, uint32_t v) {
    if constexpr (MODE == 3) {
        // v is the wave's first unit (uniform), so the index math runs on the
        // scalar unit.  The two loads are vector loads through buffer resources
        // (every lane reads the same word): they complete in order with the
        // tile's X loads, so the wait for the tile's data covers them, where
        // scalar loads, which may complete out of order, made the tile wait for
        // every scalar load in flight.  A 1-byte zero point is read as the
        // aligned 32-bit word that holds it (the host selects this mode only
        // when ZeroPoint's byte size and address are multiples of 4, so that
        // word lies inside the tensor).
        const uint32_t q = ax.inner.div(v * 4u);
        const uint32_t ch = q - ax.c.div(q) * ax.c.d;
        const uint32_t zi = ch * ax.zs;
        p.s[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(buffer_rsrc(S, kParamReach), ch * 4u, 0, 0));
        const uint32_t zw = __builtin_amdgcn_raw_buffer_load_b32(
            buffer_rsrc(Z, kParamReach), ZDT == kF32 ? zi * 4u : (zi >> 2) * 4u, 0, 0);
        if constexpr (ZDT == kF32) p.z[0] = __builtin_bit_cast(float, zw);
        else p.z[0] = (uint8_t)(zw >> (8 * (zi & 3)));
    } else if constexpr (MODE == 1) {
        const uint32_t q = ax.inner.div(v * 4u);
        const uint32_t ch = q - ax.c.div(q) * ax.c.d;
        const uint32_t zi = ch * ax.zs;
        p.s[0] = S[ch];
        p.z[0] = reinterpret_cast<const zraw_t<ZDT>*>(Z)[zi];
    } else if constexpr (MODE == 2) {
        int64_t off[3];
        bd_offsets32<3, ND>(d, v * 4u, off);
        const zraw_t<ZDT>* Zt = reinterpret_cast<const zraw_t<ZDT>*>(Z);
        const int inner = d.nd - 1;
        const int64_t ss = d.st[1][inner], sz = d.st[2][inner];
#pragma unroll
        for (int b = 0; b < 4; b++) {
            p.s[b] = S[off[1] + b * ss];
            p.z[b] = Zt[off[2] + b * sz];
        }
    }
}

constexpr int kQU = 4;         // quantize: float4 units per thread and iteration
// Quantize grid: blocks per CU.  8 (two tiles per block at config 2, loads of
// the second issued before the first is converted); per-axis MODE 3 takes 16
// (one tile per block), which measured 15.0 -> 14.5 us at config 2 where the
// per-tensor kernels measured slower with 16 (fp8: 14.8 -> 15.1 us).
constexpr int kQBlocksPerCU = 8, kQBlocksPerCUAxis = 16;
constexpr uint32_t kMaxUnitsPerLaunch = 1u << 27;   // 2 GiB of f32 per launch: buffer offsets stay below 2^32

// Codes of the 4 elements of one float4 of X.
template <int YDT, int ZDT, int MODE>
__device__ __forceinline__ uint32_t quant_unit(const float4 xv, const Params<ZDT, MODE>& pp, const QParm& pu) {
    const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
    uint32_t w;
    if constexpr (MODE == 2) {
        float q[4];
        double zd[4];
        bool good = true;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            zd[b] = ld_d<ZDT>(&pp.z[b], 0);
            q[b] = qfast(xs[b], qparm<YDT>(pp.s[b], zd[b]), good);
        }
        w = qpack4<YDT>(q[0], q[1], q[2], q[3]);
        if (!good) {
            w = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) w |= (uint32_t)qslow1<YDT>(xs[b], pp.s[b], zd[b]) << (8 * b);
        }
    } else {
        const QParm p = (MODE == 0) ? pu : qparm<YDT>(pp.s[0], ld_d<ZDT>(&pp.z[0], 0));
        bool good = true;
        const float q0 = qfast(xs[0], p, good), q1 = qfast(xs[1], p, good);
        const float q2 = qfast(xs[2], p, good), q3 = qfast(xs[3], p, good);
        w = qpack4<YDT>(q0, q1, q2, q3);
        if (!good) w = qslow4<YDT>(xs[0], xs[1], xs[2], xs[3], p.s, p.zd);
    }
    return w;
}

// One tile: kQU float4 units per thread.  Unit u of thread (wave, lane):
//   MODE 3: t * kBlock * kQU + wave * 64 * kQU + u * 64 + lane — each wave
//           covers one contiguous run of 64 * kQU units (4 * 64 * kQU
//           elements), which the host guarantees lies inside one channel, so
//           the wave loads one scale / zero point and forms its quantization
//           parameters once per tile;
//   else:   t * kBlock * kQU + u * kBlock + threadIdx.x (unit u of the block
//           is one contiguous span).
// Either way a wave's 64 lanes read 64 consecutive units (1 KB).
template <int ZDT, int MODE>
struct QTile {
    static constexpr int kP = MODE == 3 ? 1 : kQU;
    float4 x[kQU];
    Params<ZDT, MODE> p[kP];
};

template <int MODE>
__device__ __forceinline__ uint32_t qunit(uint32_t t, int u) {
    if constexpr (MODE == 3)
        return t * (kBlock * kQU) + (threadIdx.x >> 6) * (64 * kQU) + u * 64 + (threadIdx.x & 63u);
    else
        return t * (kBlock * kQU) + u * kBlock + threadIdx.x;
}

// Loads tile t.  X goes through the buffer resource (units at or beyond nv
// read as zero without touching memory); parameter indices are clamped to the
// last unit, so every parameter load stays inside Scale / ZeroPoint.
template <int ZDT, int MODE, int ND>
__device__ __forceinline__ void qload(QTile<ZDT, MODE>& q, __amdgpu_buffer_rsrc_t xr, const float* S, const void* Z,
                                      const BDesc& d, const AxisDesc& ax, uint32_t vbase, uint32_t nv, uint32_t t) {
#pragma unroll
    for (int u = 0; u < kQU; u++) q.x[u] = ld_buf_stream(xr, qunit<MODE>(t, u) * 16u);
    if constexpr (MODE == 3) {
        // the wave's first unit, as a uniform value: address math and loads go to the scalar unit
        const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x) >> 6;
        const uint32_t vp = t * (kBlock * kQU) + wave * (64 * kQU);
        load_params<ZDT, MODE, ND>(q.p[0], S, Z, d, ax, vbase + min(vp, nv - 1));
    } else {
#pragma unroll
        for (int u = 0; u < kQU; u++)
            load_params<ZDT, MODE, ND>(q.p[u], S, Z, d, ax, vbase + min(qunit<MODE>(t, u), nv - 1));
    }
}

template <int YDT, int ZDT, int MODE>
__device__ __forceinline__ void qstore(const QTile<ZDT, MODE>& q, uint32_t* Y4, const QParm& pu, uint32_t nv,
                                       uint32_t t) {
    if constexpr (MODE == 3) {
        // one channel per wave and tile: the per-tensor arithmetic with this channel's parameters
        const QParm pc = qparm<YDT>(q.p[0].s[0], ld_d<ZDT>(&q.p[0].z[0], 0));
        const Params<ZDT, 0> none{};
#pragma unroll
        for (int u = 0; u < kQU; u++) {
            const uint32_t v = qunit<MODE>(t, u);
            const uint32_t w = quant_unit<YDT, ZDT, 0>(q.x[u], none, pc);
            if (v < nv) Y4[v] = w;
        }
    } else {
#pragma unroll
        for (int u = 0; u < kQU; u++) {
            const uint32_t v = qunit<MODE>(t, u);
            const uint32_t w = quant_unit<YDT, ZDT, MODE>(q.x[u], q.p[u], pu);
            if (v < nv) Y4[v] = w;
        }
    }
}

// Quantize f32 -> 1-byte code.  X and Y are flat (X has Y's size) and hold
// the nv units starting at unit vbase of the tensor; Scale and ZeroPoint go
// through the descriptor (operands 1 and 2).  MODE 0: one scale / zero point
// for the tensor; 1: constant across each 4-element group (per-axis on a
// non-innermost axis); 2: anything else (per-element parameters).
// Requires n % 4 == 0, dim[nd-1] % 4 == 0 and nv * 16 < 2^32.
// Block b handles tiles b, b + G, b + 2G, ... (G = gridDim.x) with two tiles
// of registers in ping-pong: the loads of the next tile are issued before
// the current tile is converted, and since those loads are unconditional the
// compiler waits only for the current tile's data.
template <int YDT, int ZDT, int MODE, int ND>
__global__ __launch_bounds__(kBlock) void k_quant_v(const float* __restrict__ X, const float* __restrict__ S,
                                                    const void* __restrict__ Z, uint8_t* __restrict__ Y, BDesc d,
                                                    AxisDesc ax, uint32_t vbase, uint32_t nv) {
    uint32_t* Y4 = reinterpret_cast<uint32_t*>(Y);
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X, nv * 16u);
    QParm pu{};
    if constexpr (MODE == 0) pu = qparm<YDT>(S[0], ld_d<ZDT>(Z, 0));
    const uint32_t ntiles = (nv + kBlock * kQU - 1) / (kBlock * kQU);
    uint32_t t = blockIdx.x;
    QTile<ZDT, MODE> A, B;
    qload<ZDT, MODE, ND>(A, xr, S, Z, d, ax, vbase, nv, t);
    while (t < ntiles) {
        const uint32_t t1 = t + gridDim.x;
        qload<ZDT, MODE, ND>(B, xr, S, Z, d, ax, vbase, nv, t1);
        qstore<YDT, ZDT, MODE>(A, Y4, pu, nv, t);
        if (t1 >= ntiles) break;
        const uint32_t t2 = t1 + gridDim.x;
        qload<ZDT, MODE, ND>(A, xr, S, Z, d, ax, vbase, nv, t2);
        qstore<YDT, ZDT, MODE>(B, Y4, pu, nv, t1);
        t = t2;
    }
}

// Four codes of one word -> fp32 values (exact).  fp8 codes use the gfx950
// conversions v_cvt_pk_f32_fp8 / _bf8, which equal the reference decoders
// (tensor_ops.c:236-256, 295-316) on all 256 codes; NaN codes give a NaN.
template <int XDT>
__device__ __forceinline__ void decode4(uint32_t w, float (&x)[4]) {
    if constexpr (XDT == kE4M3 || XDT == kE5M2) {
        typedef float f32x2_t __attribute__((ext_vector_type(2)));
        f32x2_t lo, hi;
        if constexpr (XDT == kE4M3) {
            lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
            hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
        } else {
            lo = __builtin_amdgcn_cvt_pk_f32_bf8((int)w, false);
            hi = __builtin_amdgcn_cvt_pk_f32_bf8((int)w, true);
        }
        x[0] = lo.x; x[1] = lo.y; x[2] = hi.x; x[3] = hi.y;
    } else {
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint8_t c = (uint8_t)(w >> (8 * b));
            x[b] = (float)ld_d<XDT>(&c, 0);
        }
    }
}

// Dequantize 1-byte code -> f32: each thread takes kDQU code words (4 codes
// each) kBlock words apart, all loaded before any is converted, and writes
// each as one nontemporal float4; grid-stride beyond 2^20 blocks.
// (x - zp) * s is the reference's fp64 expression rounded once to f32
// (tensor_ops.c:1018-1034).  It is evaluated in f32 where that gives the
// same bits: for integer codes with an integer zero point x - zp is an exact
// integer of at most 9 bits, so the f32 product is the correctly rounded
// exact product, which is what rounding the (exact) fp64 product gives; for
// fp8 codes with a zero zero point x * s is likewise one correctly rounded
// product.  Otherwise (fp8 with a non-zero zero point, a float zero point
// of integer codes) it stays in fp64.
// kDQU = 4 measured against one word per thread (config 2, full grid either
// way): each launch alone 12.8 -> 13.5-14.1 us, but the Q -> DQ round trip,
// where the codes were just written, 119.5 -> 118.4 us per 8 launches (the
// fp64 -> f32 change alone about 0.3 us of that).
constexpr int kDQU = 4;

template <int XDT, int ZDT, int MODE, int ND>
__global__ __launch_bounds__(kBlock) void k_dequant_v(const uint8_t* __restrict__ X, const float* __restrict__ S,
                                                      const void* __restrict__ Z, float* __restrict__ Y, BDesc d,
                                                      AxisDesc ax, uint32_t vbase, uint32_t nv) {
    float4* Y4 = reinterpret_cast<float4*>(Y);
    double su = 0.0, zu = 0.0;
    if constexpr (MODE == 0) {
        su = (double)S[0];
        zu = ld_d<ZDT>(Z, 0);
    }
    constexpr bool kIntCodes = (XDT == kU8 || XDT == kI8) && (ZDT == kU8 || ZDT == kI8);
    // code words through a buffer resource: words at or past nv read as zero
    // without a memory access (plain cached loads: measured against global
    // loads, the same per launch and 0.4% faster in the Q -> DQ round trip)
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X, nv * 4u);
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wbase = __builtin_amdgcn_readfirstlane(threadIdx.x) & ~63u;
    // vw0: the wave's first word of this pass (uniform); lanes past nv skip
    // their store
    for (uint32_t vw0 = blockIdx.x * kBlock * kDQU + wbase; vw0 < nv; vw0 += gridDim.x * kBlock * kDQU) {
        uint32_t w[kDQU];
#pragma unroll
        for (int u = 0; u < kDQU; u++) w[u] = __builtin_amdgcn_raw_buffer_load_b32(xr, (vw0 + u * kBlock + lane) * 4u, 0, 0);
#pragma unroll
        for (int u = 0; u < kDQU; u++) {
            const uint32_t vw = vw0 + u * kBlock, v = vw + lane;
            if (v >= nv) continue;
            Params<ZDT, MODE> p;
            load_params<ZDT, MODE, ND>(p, S, Z, d, ax, vbase + (MODE == 3 ? vw : v));
            float x[4], y[4];
            decode4<XDT>(w[u], x);
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int k = MODE == 2 ? b : 0;
                const double s = MODE == 0 ? su : (double)p.s[k];
                const double z = MODE == 0 ? zu : ld_d<ZDT>(&p.z[k], 0);
                if (kIntCodes || z == 0.0) y[b] = (x[b] - (float)z) * (float)s;
                else y[b] = (float)(((double)x[b] - z) * s);
            }
            st_stream(Y4 + v, make_float4(y[0], y[1], y[2], y[3]));
        }
    }
}

// QuantizeLinear then DequantizeLinear, one scale / zero point each, in one
// pass (tensor_ops.c:999-1016 then :1018-1034): the codes stay in registers.
// The quantize step is k_quant_v's (MODE 0) and the dequantize step
// k_dequant_v's (MODE 0), so Y equals the two operators' result bit for bit.
// The zero points have the code's dtype (as ONNX requires); two float4 units
// per thread per iteration.
template <int CDT>
__global__ __launch_bounds__(kBlock) void k_qdq_fused(const float* __restrict__ X, const float* __restrict__ SQ,
                                                      const void* __restrict__ ZQ, const float* __restrict__ SD,
                                                      const void* __restrict__ ZD, float* __restrict__ Y, uint32_t nv) {
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X, nv * 16u);
    const QParm pu = qparm<CDT>(SQ[0], ld_d<CDT>(ZQ, 0));
    const double sd = (double)SD[0], zd = ld_d<CDT>(ZD, 0);
    // the dequantize step in f32 where k_dequant_v uses it (integer codes, or
    // a zero zero point): the same bits as the fp64 expression rounded once
    const bool f32dq = CDT == kU8 || CDT == kI8 || zd == 0.0;
    const float sdf = SD[0], zdf = (float)zd;
    const Params<CDT, 0> none{};
    float4* Y4 = reinterpret_cast<float4*>(Y);
    for (uint32_t v0 = blockIdx.x * (kBlock * 2) + threadIdx.x; v0 < nv; v0 += gridDim.x * (kBlock * 2)) {
        float4 xv[2];
#pragma unroll
        for (int u = 0; u < 2; u++) xv[u] = ld_buf_stream(xr, (v0 + u * kBlock) * 16u);   // past nv: zero
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const uint32_t v = v0 + u * kBlock;
            if (v >= nv) continue;
            float c[4], y[4];
            decode4<CDT>(quant_unit<CDT, CDT, 0>(xv[u], none, pu), c);
            if (f32dq) {      // uniform
#pragma unroll
                for (int b = 0; b < 4; b++) y[b] = (c[b] - zdf) * sdf;
            } else {
#pragma unroll
                for (int b = 0; b < 4; b++) y[b] = (float)(((double)c[b] - zd) * sd);
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
        const bool qfast_ok = QUANT && dtx == kF32 && dts == kF32 && zdt_fast(dtz) && is_code8(dty);
        const bool dqfast_ok = !QUANT && is_code8(dtx) && dts == kF32 && zdt_fast(dtz) && dty == kF32;
        if ((qfast_ok || dqfast_ok) && fast_ok(d, X, n, x, y)) {
            // Per-axis parameters: Scale varies along exactly one collapsed dimension
            // (not the innermost) with unit stride; ZeroPoint along the same one or not at all.
            int axis = -1;
            bool axis_ok = true;
            for (int a = 0; a < d.nd; a++) {
                if (d.st[1][a] == 0) continue;
                if (axis >= 0 || d.st[1][a] != 1) axis_ok = false;
                axis = a;
            }
            uint32_t zs = 0;
            for (int a = 0; a < d.nd; a++) {
                if (d.st[2][a] == 0) continue;
                if (a != axis || d.st[2][a] != 1) axis_ok = false;
                zs = 1;
            }
            bool uniform = true;
            for (int a = 0; a < d.nd; a++) uniform = uniform && d.st[1][a] == 0 && d.st[2][a] == 0;
            AxisDesc ax{};
            int mode = 2;
            if (uniform && d.nd == 1) {
                mode = 0;
            } else if (axis_ok && axis >= 0 && axis < d.nd - 1) {
                uint64_t inner = 1;
                for (int a = axis + 1; a < d.nd; a++) inner *= d.dim[a];
                ax.inner = make_fastdiv((uint32_t)inner);
                ax.c = make_fastdiv(d.dim[axis]);
                ax.zs = zs;
                // A wave's units stay inside one channel when the channel's run of
                // elements is a multiple of the wave's run: dequantize — 64 units of
                // 4 elements at a multiple of 64 units; quantize — 64 * kQU units
                // at a multiple of that (see QTile).
                const uint64_t wave_run = QUANT ? 4u * 64u * kQU : 4u * 64u;
                const bool zword = dtz == kF32 || (tensor_bytes(Z) % 4 == 0 && ((uintptr_t)z % 4) == 0);
                mode = (inner % wave_run == 0 && zword && ((uintptr_t)s % 4) == 0) ? 3 : 1;
            }
#define QDQ_MODES(LAUNCH_K)                                          \
    if (mode == 0) { LAUNCH_K(0, 1); }                               \
    else if (mode == 3) { LAUNCH_K(3, 0); }                          \
    else if (mode == 1) { LAUNCH_K(1, 0); }                          \
    else { LAUNCH_K(2, 0); }
#define CODE_SWITCH(dt, ...)                                         \
    switch (dt) {                                                    \
    case kU8: { constexpr int CD = kU8; __VA_ARGS__; } break;        \
    case kI8: { constexpr int CD = kI8; __VA_ARGS__; } break;        \
    case kE4M3: { constexpr int CD = kE4M3; __VA_ARGS__; } break;    \
    default: { constexpr int CD = kE5M2; __VA_ARGS__; } break;       \
    }
            const uint32_t nv_all = (uint32_t)(n / 4);
            // Launch in chunks of at most kMaxUnitsPerLaunch units so that buffer
            // byte offsets stay below 2^32; vbase keeps the descriptor indexing global.
            for (uint32_t vbase = 0; vbase < nv_all; vbase += kMaxUnitsPerLaunch) {
                const uint32_t nv = nv_all - vbase < kMaxUnitsPerLaunch ? nv_all - vbase : kMaxUnitsPerLaunch;
                const dim3 b(kBlock);
                if (QUANT) {
                    const dim3 g(grid_for(nv, kBlock * kQU, (mode == 3 ? kQBlocksPerCUAxis : kQBlocksPerCU) * num_cus()));
                    const float* xc = (const float*)x + (size_t)vbase * 4;
                    uint8_t* yc = (uint8_t*)y + (size_t)vbase * 4;
#define QK(M, NDV) \
    hipLaunchKernelGGL((k_quant_v<CD, ZD, M, NDV>), g, b, 0, sm, xc, (const float*)s, z, yc, d, ax, vbase, nv)
                    CODE_SWITCH(dty, ZDT_SWITCH(dtz, QDQ_MODES(QK)))
#undef QK
                } else {
                    const dim3 g(grid_for(nv, kBlock * kDQU));
                    const uint8_t* xc = (const uint8_t*)x + (size_t)vbase * 4;
                    float* yc = (float*)y + (size_t)vbase * 4;
#define DQK(M, NDV) \
    hipLaunchKernelGGL((k_dequant_v<CD, ZD, M, NDV>), g, b, 0, sm, xc, (const float*)s, z, yc, d, ax, vbase, nv)
                    CODE_SWITCH(dtx, ZDT_SWITCH(dtz, QDQ_MODES(DQK)))
#undef DQK
                }
            }
#undef CODE_SWITCH
#undef QDQ_MODES
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

// ------------------------------------------------------- DynamicQuantizeLinear ---
// tensor_ops.c:3760-3809.  f32 -> uint8 runs one launch that reads x once
// (k_dql_one, below); other dtypes, graph capture, the no-allocation entry
// point and tensors too large for its grid take three launches:
//  * k_dql_minmax: each block reduces min / max of its grid-stride share with
//    the reference's compares (v < lo, v > hi: NaN never enters), so the
//    result does not depend on the order; f32 input is read as float4;
//  * k_dql_params: one block folds the partials and derives scale and zero
//    point in double exactly as the reference (y_scale / y_zp written here);
//  * k_dql_quant: y = clamp(rint(x / scale) + zp, 0, 255) with the double
//    scale, four elements per thread.
constexpr int kDqlThreads = 256, kDqlMaxParts = 2048;

template <int DIN> __device__ __forceinline__ double dql_ld(const void* p, int64_t i, int rdt) {
    if constexpr (DIN >= 0) return ld_d<DIN>(p, i);
    else return ld_d_rt(rdt, p, i);
}

__device__ __forceinline__ void dql_fold(double& lo, double& hi, double* lds) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const double a = __shfl_xor(lo, o, 64), b = __shfl_xor(hi, o, 64);
        lo = a < lo ? a : lo;
        hi = b > hi ? b : hi;
    }
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) { lds[2 * w] = lo; lds[2 * w + 1] = hi; }
    __syncthreads();
    lo = lds[0];
    hi = lds[1];
#pragma unroll
    for (int i = 1; i < kDqlThreads / 64; i++) {
        lo = lds[2 * i] < lo ? lds[2 * i] : lo;
        hi = lds[2 * i + 1] > hi ? lds[2 * i + 1] : hi;
    }
}

template <int DIN>
__global__ __launch_bounds__(kDqlThreads) void k_dql_minmax(const void* __restrict__ X, int dtx, int64_t n,
                                                            double* __restrict__ part) {
    __shared__ double lds[2 * kDqlThreads / 64];
    double lo = DBL_MAX, hi = -DBL_MAX;
    const int64_t stride = (int64_t)gridDim.x * kDqlThreads;
    int64_t tail = 0;
    if constexpr (DIN == kF32) {
        const int64_t nv = n / 4;
        for (int64_t v = (int64_t)blockIdx.x * kDqlThreads + threadIdx.x; v < nv; v += stride) {
            // ordinary loads: the quantize pass reads x again, from the Infinity Cache when it fits
            const float4 x = reinterpret_cast<const float4*>(X)[v];
            const float e[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const double d = (double)e[k];
                if (d < lo) lo = d;
                if (d > hi) hi = d;
            }
        }
        tail = nv * 4;
    }
    for (int64_t i = tail + (int64_t)blockIdx.x * kDqlThreads + threadIdx.x; i < n; i += stride) {
        const double v = dql_ld<DIN>(X, i, dtx);
        if (v < lo) lo = v;
        if (v > hi) hi = v;
    }
    dql_fold(lo, hi, lds);
    if (threadIdx.x == 0) { part[2 * blockIdx.x] = lo; part[2 * blockIdx.x + 1] = hi; }
}

// Scale and zero point from the tensor's min / max, in double exactly as the
// reference (tensor_ops.c:3760-3809).
__device__ __forceinline__ void dql_params(double lo, double hi, double& scale, double& zpd) {
    // fmin(lo, 0.0) / fmax(hi, 0.0) as x86 libm returns them (a zero gives +0)
    lo = lo < 0.0 ? lo : 0.0;
    hi = hi > 0.0 ? hi : 0.0;
    scale = (hi - lo) / 255.0;
    if (scale == 0.0) scale = 1.0;
    zpd = round(0.0 - lo / scale);
    if (zpd < 0.0) zpd = 0.0;
    if (zpd > 255.0) zpd = 255.0;
}

// params[0] = scale, params[1] = zero point (an integer in [0, 255]).
__global__ __launch_bounds__(kDqlThreads) void k_dql_params(const double* __restrict__ part, int nparts,
                                                            double* __restrict__ params, void* __restrict__ ys,
                                                            int dts, void* __restrict__ yz, int dtz) {
    __shared__ double lds[2 * kDqlThreads / 64];
    double lo = DBL_MAX, hi = -DBL_MAX;
    for (int i = threadIdx.x; i < nparts; i += kDqlThreads) {
        lo = part[2 * i] < lo ? part[2 * i] : lo;
        hi = part[2 * i + 1] > hi ? part[2 * i + 1] : hi;
    }
    dql_fold(lo, hi, lds);
    if (threadIdx.x != 0) return;
    double scale, zpd;
    dql_params(lo, hi, scale, zpd);
    params[0] = scale;
    params[1] = zpd;
    st_d_rt(dts, ys, 0, scale);
    st_d_rt(dtz, yz, 0, zpd);       // zpd is an integer in [0, 255]: the code is zpd itself
}

// rint(v / scale) + zp, clamped to [0, 255].  The quotient is formed as
// p = RN(v * RN(1 / scale)), within 2^-52 |v / scale| of the exact quotient;
// rint(p) equals rint(v / scale) unless the quotient lies within that distance
// of a half-integer.  Lanes whose p is within 2^-40 |p| of one (and NaN / inf,
// whose comparisons fail) take the correctly rounded fp64 division instead, so
// every code equals the reference's.
__device__ __forceinline__ double dql_q(double v, double scale, double inv, double zpd) {
    const double p = v * inv;
    double r = __builtin_rint(p);
    if (!(__builtin_fabs(__builtin_fabs(p - r) - 0.5) > 0x1p-40 * __builtin_fabs(p))) r = __builtin_rint(v / scale);
    double q = r + zpd;
    if (q < 0.0) q = 0.0;
    if (q > 255.0) q = 255.0;
    return q;
}

// The codes of the four values of v: rint(v / scale) + zp clamped to [0, 255].
// With an f32 reciprocal (fast: 2^-120 < scale < 2^120, so 1 / scale is a
// normal float and |v / scale| <= 255 + |zp| cannot overflow) p = RN(v * RN(1 /
// scale)) lies within 2^-22.8 |p| of the exact quotient, and of its double
// rounding, which is what the reference rounds; rint(p) is that quotient's
// rint unless p is within 2^-21 |p| of a half-integer.  rint(p) + zp is then
// an integer, which v_cvt_pk_u8_f32 clamps to [0, 255] and packs.  A word
// with any lane out of that case (near a tie, NaN / inf, whose compares fail)
// takes dql_q, the double path, for its four values: both paths give the
// reference's code, so the word is the same either way.
__device__ __forceinline__ uint32_t dql_code4(const float4& v, bool fast, float invf, float zpf, double scale,
                                              double inv, double zpd) {
    const float e[4] = {v.x, v.y, v.z, v.w};
    bool ok = fast;
    uint32_t w = 0;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const float p = e[b] * invf;
        const float r = __builtin_rintf(p);
        ok = ok && __builtin_fabsf(__builtin_fabsf(p - r) - 0.5f) > 0x1p-21f * __builtin_fabsf(p);
        w = __builtin_amdgcn_cvt_pk_u8_f32(r + zpf, b, w);
    }
    if (!ok) {
        w = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) w |= (uint32_t)dql_q((double)e[b], scale, inv, zpd) << (8 * b);
    }
    return w;
}


template <int DIN, int DY>
__global__ __launch_bounds__(kDqlThreads) void k_dql_quant(const void* __restrict__ X, int dtx, int64_t n,
                                                           const double* __restrict__ params, void* __restrict__ Y,
                                                           int dty) {
    const double scale = params[0], zpd = params[1], inv = 1.0 / scale;
    const int64_t stride = (int64_t)gridDim.x * kDqlThreads;
    int64_t tail = 0;
    if constexpr (DIN == kF32 && DY == kU8) {
        // the one-launch kernel's codes (dql_code4), so the two forms agree bit for bit
        const bool fast = scale > 0x1p-120 && scale < 0x1p120;
        const float invf = (float)inv, zpf = (float)zpd;
        const int64_t nv = n / 4;
        for (int64_t v = (int64_t)blockIdx.x * kDqlThreads + threadIdx.x; v < nv; v += stride) {
            const float4 x = ld_stream(reinterpret_cast<const float4*>(X) + v);
            st_stream(reinterpret_cast<uint32_t*>(Y) + v, dql_code4(x, fast, invf, zpf, scale, inv, zpd));
        }
        tail = nv * 4;
    }
    for (int64_t i = tail + (int64_t)blockIdx.x * kDqlThreads + threadIdx.x; i < n; i += stride) {
        const double q = dql_q(dql_ld<DIN>(X, i, dtx), scale, inv, zpd);
        if constexpr (DY >= 0) st_d<DY>(Y, i, q);
        else st_d_rt(dty, Y, i, q);
    }
}

// One launch, x read once (f32 x, uint8 y, x 16-byte and y 4-byte aligned,
// n % 4 == 0, at most one block per CU (256 blocks) x 1024 threads x 16
// float4s): block b holds its chunk of cv float4s in registers (thread t:
// float4s t + 1024 k), reduces its min / max
// (on the floats: the same compares on the same exactly converted values as the
// double fold, a +inf / -inf result standing for the DBL_MAX / -DBL_MAX start
// that nothing beat), publishes them as two tagged words (xchg_pub), waits for
// every other block's pair with a bounded poll (recomputing from x, with the
// same min / max, any pair that does not arrive), derives scale and zero point
// as k_dql_params does and writes the codes of its chunk from registers.  The
// min / max of a set does not depend on the fold order (the sign of a zero
// aside, which dql_params maps to +0), so every block derives the same scale
// and zero point, equal to the three-launch path's.
constexpr int kDqlOneThreads = 1024, kDqlOneMaxEpt4 = 16, kDqlOneMaxBlocks = 256;

// A buffer resource over the n units (of `unit` bytes) at p; none when n <= 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dql_rsrc(const void* p, int n, int unit) {
    return buffer_rsrc(p, n > 0 ? (uint32_t)n * (uint32_t)unit : 0u);
}

// This thread's (min, max) over its float4s t + 1024 k (k < EPT4) of the n4
// float4s at p; KEEP: the float4s are also kept in x (else loaded one at a time).
template <int EPT4, bool KEEP>
__device__ __forceinline__ void dql_thread_minmax(const float* __restrict__ p, int n4, float4 (&x)[EPT4], float& lo,
                                                  float& hi) {
    const int tid = (int)threadIdx.x;
    typedef unsigned int u32x4_t __attribute__((__vector_size__(16)));
    lo = __builtin_inff();
    hi = -__builtin_inff();
    // one buffer resource per k (scalar registers), over float4s k * 1024 ..,
    // so every load takes the same per-lane offset tid * 16
    const auto load = [&](int k) {
        return __builtin_bit_cast(float4, (u32x4_t)__builtin_amdgcn_raw_buffer_load_b128(
                                              dql_rsrc(p + 4 * k * kDqlOneThreads, n4 - k * kDqlOneThreads, 16),
                                              (uint32_t)(tid * 16), 0, 0));
    };
    const auto fold = [&](float e) {
        lo = e < lo ? e : lo;
        hi = e > hi ? e : hi;
    };
    if constexpr (KEEP) {
#pragma unroll
        for (int k = 0; k < EPT4; k++) x[k] = load(k);
    }
#pragma unroll
    for (int k = 0; k < EPT4; k++) {
        const float4 v = KEEP ? x[k] : load(k);
        if (tid + k * kDqlOneThreads < n4) { fold(v.x); fold(v.y); fold(v.z); fold(v.w); }
    }
}

// Block-wide (min, max) of the n4 float4s at p (see dql_thread_minmax); every
// thread returns the block's pair.
template <int EPT4, bool KEEP>
__device__ __forceinline__ void dql_chunk_minmax(const float* __restrict__ p, int n4, float4 (&x)[EPT4], float& lo,
                                                 float& hi, float* lds) {
    const int tid = (int)threadIdx.x;
    dql_thread_minmax<EPT4, KEEP>(p, n4, x, lo, hi);
    lo = wave_allreduce(lo, [](float a, float b) { return b < a ? b : a; });
    hi = wave_allreduce(hi, [](float a, float b) { return b > a ? b : a; });
    const int w = tid >> 6;
    if ((tid & 63) == 0) { lds[2 * w] = lo; lds[2 * w + 1] = hi; }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kDqlOneThreads / 64; i++) {
        lo = lds[2 * i] < lo ? lds[2 * i] : lo;
        hi = lds[2 * i + 1] > hi ? lds[2 * i + 1] : hi;
    }
    __syncthreads();
}

// (1024, 4): at most 128 registers per lane (4 waves per SIMD), so a block fits
// on every CU and the whole grid (one block per CU) is resident at once.
template <int EPT4>
__global__ __launch_bounds__(kDqlOneThreads, 4) void k_dql_one(const float* __restrict__ X, int64_t nv, int64_t cv,
                                                            unsigned char* __restrict__ Y,
                                                            unsigned long long* __restrict__ slots, uint32_t tag,
                                                            int spin, void* __restrict__ ys, int dts,
                                                            void* __restrict__ yz, int dtz) {
    __shared__ float lds[2 * kDqlOneThreads / 64];
    __shared__ unsigned long long s_miss[kDqlOneMaxBlocks / 64];
    __shared__ int s_any;
    __shared__ float s_lo, s_hi;
    __shared__ double s_scale, s_zp;
    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int nblk = (int)gridDim.x;
    const auto chunk_n4 = [&](int b) { return (int)max<int64_t>(0, min<int64_t>(cv, nv - (int64_t)b * cv)); };
    const int n4 = chunk_n4((int)blockIdx.x);
    float4 x[EPT4];
    float lo, hi;
    dql_chunk_minmax<EPT4, true>(X + 4 * (int64_t)blockIdx.x * cv, n4, x, lo, hi, lds);
    if (tid == 0) {
        xchg_pub(slots + 2 * blockIdx.x, tag, __builtin_bit_cast(uint32_t, lo));
        xchg_pub(slots + 2 * blockIdx.x + 1, tag, __builtin_bit_cast(uint32_t, hi));
    }
    // Wave 0, lane l: the pairs of blocks l + 64 i (i < 16), polled together.
    const auto params = [&](float flo, float fhi) {
        double scale, zpd;
        dql_params(flo == __builtin_inff() ? DBL_MAX : (double)flo, fhi == -__builtin_inff() ? -DBL_MAX : (double)fhi,
                   scale, zpd);
        s_scale = scale;
        s_zp = zpd;
        if (blockIdx.x == 0) {
            st_d_rt(dts, ys, 0, scale);
            st_d_rt(dtz, yz, 0, zpd);       // an integer in [0, 255]: the code is zpd itself
        }
    };
    if (tid < 64) {
        // fold each pair as it arrives (this block's own pair is already in)
        float flo = lo, fhi = hi;
        unsigned need = 0;
#pragma unroll
        for (int i = 0; i < kDqlOneMaxBlocks / 64; i++) {
            const int b = lane + 64 * i;
            if (b < nblk && b != (int)blockIdx.x) need |= 1u << i;
        }
        for (int it = 0; need && it < spin; it++) {
#pragma unroll
            for (int i = 0; i < kDqlOneMaxBlocks / 64; i++) {
                if (need >> i & 1) {
                    const int b = lane + 64 * i;
                    uint32_t wl, wh;
                    const bool a = xchg_get(slots + 2 * b, tag, wl), c = xchg_get(slots + 2 * b + 1, tag, wh);
                    if (a & c) {
                        need &= ~(1u << i);
                        const float pl = __builtin_bit_cast(float, wl), ph = __builtin_bit_cast(float, wh);
                        flo = pl < flo ? pl : flo;
                        fhi = ph > fhi ? ph : fhi;
                    }
                }
            }
            if (need) __builtin_amdgcn_s_sleep(1);
        }
        flo = wave_allreduce(flo, [](float a, float b) { return b < a ? b : a; });
        fhi = wave_allreduce(fhi, [](float a, float b) { return b > a ? b : a; });
        int any = 0;
#pragma unroll
        for (int i = 0; i < kDqlOneMaxBlocks / 64; i++) {
            const unsigned long long m = __ballot(need >> i & 1);
            if (lane == 0) s_miss[i] = m;
            any |= m != 0;
        }
        if (lane == 0) {
            s_any = any;
            s_lo = flo;
            s_hi = fhi;
            if (!any) params(flo, fhi);
        }
    }
    __syncthreads();
    if (s_any) {        // uniform over the block: recompute the pairs that did not arrive
        for (int i = 0; i < kDqlOneMaxBlocks / 64; i++)
            for (unsigned long long m = s_miss[i]; m; m &= m - 1) {
                const int b = 64 * i + __builtin_ctzll(m);
                float bl, bh;
                dql_chunk_minmax<EPT4, false>(X + 4 * (int64_t)b * cv, chunk_n4(b), x, bl, bh, lds);
                if (tid == 0) {
                    s_lo = bl < s_lo ? bl : s_lo;
                    s_hi = bh > s_hi ? bh : s_hi;
                }
            }
        __syncthreads();
        if (tid == 0) params(s_lo, s_hi);
        __syncthreads();
    }
    const double scale = s_scale, zpd = s_zp, inv = 1.0 / scale;
    const bool fast = scale > 0x1p-120 && scale < 0x1p120;
    const float invf = (float)inv, zpf = (float)zpd;
    unsigned char* yb = Y + 4 * (int64_t)blockIdx.x * cv;
#pragma unroll
    for (int k = 0; k < EPT4; k++) {
        const uint32_t c = dql_code4(x[k], fast, invf, zpf, scale, inv, zpd);
        __builtin_amdgcn_raw_buffer_store_b32(c, dql_rsrc(yb + 4 * k * kDqlOneThreads, n4 - k * kDqlOneThreads, 4),
                                              (uint32_t)(tid * 4), 0, 2 /* nt */);
    }
}

// Scratch of dynamic_quantize_linear_forward_noalloc and of calls captured into
// a graph (whose workspace must outlive the call): the min / max partials of
// k_dql_minmax and the (scale, zero point) pair of k_dql_params, in a
// file-scope device array (each GPU holds its own copy until the process
// ends).  In host code `scratch` names a host-side stand-in, not device
// memory: host code uses only the address that init_qdq_workspace resolves
// with hipGetSymbolAddress, once per device with that device current, at
// library initialisation (dql_scratch).  Every such call on one GPU shares the
// array, so those that overlap on one GPU (different streams or threads, or
// concurrent replays of captured graphs) race.  Nothing in it needs to start at
// zero: k_dql_minmax writes every partial it launches and k_dql_params the
// pair before any kernel reads them.
constexpr int kDqlScratch = 2 * kDqlMaxParts + 2;             // 32,784 bytes
static __device__ __align__(256) double scratch[kDqlScratch];

constexpr int kMaxScratchDevices = 64;
double* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the library's device; nullptr with the error
// set when initialisation could not resolve it.
double* dql_scratch() {
    const int dev = device_id();
    double* p = (dev >= 0 && dev < kMaxScratchDevices) ? g_scratch_ptr[dev] : nullptr;
    if (!p) set_error("dynamic_quantize_linear: fixed scratch of device %d unavailable", dev);
    return p;
}

// Workspace of the three-launch path: `scratch` for noalloc and captured calls
// (nothing is allocated), an HBM pool buffer otherwise.  The noalloc entry
// point also requires device-resident tensors (host tensors would need staging
// buffers).
void dql_entry(const Tensor* x, Tensor* y, Tensor* y_scale, Tensor* y_zp, bool noalloc = false) {
    const char* name = noalloc ? "dynamic_quantize_linear_forward_noalloc" : "dynamic_quantize_linear_forward";
    if (!tensor_sane(x, name) || !tensor_sane(y, name) || !tensor_sane(y_scale, name) || !tensor_sane(y_zp, name))
        return;
    if (y->size < x->size || y_scale->size < 1 || y_zp->size < 1) { set_error("%s: output too small", name); return; }
    if (!ensure_device()) return;
    if (noalloc) {
        const Tensor* all[4] = {x, y, y_scale, y_zp};
        for (const Tensor* t : all)
            if (t->size && !is_dev(classify(t->data))) {
                set_error("%s: every tensor must be device-resident (host tensors need staging buffers)", name);
                return;
            }
    }
    const int64_t n = (int64_t)x->size;
    Staging st;
    const void* xd = st.in(x);
    void* yd = st.out(y, (size_t)n * dt_bytes((int)y->dtype));
    void* sd = st.out(y_scale, dt_bytes((int)y_scale->dtype));
    void* zd = st.out(y_zp, dt_bytes((int)y_zp->dtype));
    if (!xd || !yd || !sd || !zd) { st.finish(); return; }
    const int dtx = (int)x->dtype, dty = (int)y->dtype;
    const bool v4 = dtx == kF32 && ((uintptr_t)xd & 15) == 0;
    const int64_t items = v4 ? n / 4 : n;
    const int nparts = (int)std::min<int64_t>(kDqlMaxParts, std::max<int64_t>(1, (items + 4 * kDqlThreads - 1) /
                                                                                     (4 * kDqlThreads)));
    const unsigned qblocks = grid_for((size_t)std::max<int64_t>(items, 1), kDqlThreads, 8192);
    hipStream_t s = stream();
    const bool captured = stream_capturing(s);
    // f32 -> uint8 in one launch that reads x once (k_dql_one), unless captured
    // into a graph (its exchange tags are per call) or too large for its grid
    if (!noalloc && !captured && v4 && dty == kU8 && ((uintptr_t)yd & 3) == 0 && n % 4 == 0) {
        const int64_t nv = n / 4, maxblk = std::min(num_cus(), kDqlOneMaxBlocks);
        int ept4 = 0;
        for (int e : {4, 8, kDqlOneMaxEpt4})
            if (!ept4 && nv <= maxblk * kDqlOneThreads * (int64_t)e) ept4 = e;
        if (ept4) {
            const int64_t nblk = (nv + (int64_t)kDqlOneThreads * ept4 - 1) / ((int64_t)kDqlOneThreads * ept4);
            const int64_t cv = (nv + nblk - 1) / nblk;
            uint32_t tag = 0;
            unsigned long long* slots =
                (unsigned long long*)xchg_alloc(sizeof(unsigned long long) * 2 * nblk, &tag);
            if (!slots) { st.finish(); return; }
            const int spin = exchange_spin();
            const int dts = (int)y_scale->dtype, dtz = (int)y_zp->dtype;
            unsigned char* y8 = (unsigned char*)yd;
            const float* xf = (const float*)xd;
            if (ept4 == 4)
                hipLaunchKernelGGL((k_dql_one<4>), dim3((unsigned)nblk), dim3(kDqlOneThreads), 0, s, xf, nv, cv, y8,
                                   slots, tag, spin, sd, dts, zd, dtz);
            else if (ept4 == 8)
                hipLaunchKernelGGL((k_dql_one<8>), dim3((unsigned)nblk), dim3(kDqlOneThreads), 0, s, xf, nv, cv, y8,
                                   slots, tag, spin, sd, dts, zd, dtz);
            else
                hipLaunchKernelGGL((k_dql_one<kDqlOneMaxEpt4>), dim3((unsigned)nblk), dim3(kDqlOneThreads), 0, s, xf,
                                   nv, cv, y8, slots, tag, spin, sd, dts, zd, dtz);
            check_launch(name);         // sets the error on failure; the buffer goes back either way
            xchg_free(slots);
            st.finish();
            return;
        }
    }
    const bool pooled = !noalloc && !captured;
    double* part = pooled ? (double*)pool_alloc(sizeof(double) * kDqlScratch) : dql_scratch();
    if (!part) { st.finish(); return; }
    double* params = part + 2 * kDqlMaxParts;
    if (v4) hipLaunchKernelGGL((k_dql_minmax<kF32>), dim3(nparts), dim3(kDqlThreads), 0, s, xd, dtx, n, part);
    else hipLaunchKernelGGL((k_dql_minmax<-1>), dim3(nparts), dim3(kDqlThreads), 0, s, xd, dtx, n, part);
    hipLaunchKernelGGL(k_dql_params, dim3(1), dim3(kDqlThreads), 0, s, part, nparts, params, sd, (int)y_scale->dtype,
                       zd, (int)y_zp->dtype);
    if (v4 && dty == kU8 && ((uintptr_t)yd & 3) == 0)
        hipLaunchKernelGGL((k_dql_quant<kF32, kU8>), dim3(qblocks), dim3(kDqlThreads), 0, s, xd, dtx, n, params, yd, dty);
    else if (dtx == kF32)
        hipLaunchKernelGGL((k_dql_quant<kF32, -1>), dim3(qblocks), dim3(kDqlThreads), 0, s, xd, dtx, n, params, yd, dty);
    else
        hipLaunchKernelGGL((k_dql_quant<-1, -1>), dim3(qblocks), dim3(kDqlThreads), 0, s, xd, dtx, n, params, yd, dty);
    const bool ok = check_launch(name);
    if (pooled) pool_free(part);        // pool buffers are reused in stream order
    if (!ok) { st.finish(); return; }
    st.finish();
}

// QuantizeLinear(X, QScale, QZeroPoint) as code_dtype, then DequantizeLinear
// with DScale / DZeroPoint.  The one-pass kernel covers f32 X and Y of one
// shape, one-element f32 scales and one-element zero points of the code dtype
// (uint8 / int8 / e4m3 / e5m2); anything else runs the two operators through
// a temporary code tensor, which is also what the kernel returns.
void qdq_fused_entry(const Tensor* X, const Tensor* QS, const Tensor* QZ, const Tensor* DS, const Tensor* DZ, Tensor* Y,
                     int code_dtype) {
    const char* name = "quantize_dequantize_linear_forward";
    if (!tensor_sane(X, name) || !tensor_sane(QS, name) || !tensor_sane(QZ, name) || !tensor_sane(DS, name) ||
        !tensor_sane(DZ, name) || !tensor_sane(Y, name))
        return;
    if (Y->size != X->size) { set_error("%s: Y must have X's size", name); return; }
    const size_t n = X->size;
    const bool fast = X->dtype == DTYPE_FLOAT32 && Y->dtype == DTYPE_FLOAT32 && is_code8(code_dtype) &&
                      QS->dtype == DTYPE_FLOAT32 && DS->dtype == DTYPE_FLOAT32 && QS->size == 1 && DS->size == 1 &&
                      QZ->size == 1 && DZ->size == 1 && (int)QZ->dtype == code_dtype &&
                      (int)DZ->dtype == code_dtype && n % 4 == 0 && n < (size_t(1) << 31);
    if (fast && ensure_device()) {
        Staging st;
        const void* x = st.in(X);
        const void* qs = st.in(QS);
        const void* qz = st.in(QZ);
        const void* ds = st.in(DS);
        const void* dz = st.in(DZ);
        void* y = st.out(Y, tensor_bytes(Y));
        if (!x || !qs || !qz || !ds || !dz || !y) { st.finish(); return; }
        if (((uintptr_t)x % 16) == 0 && ((uintptr_t)y % 16) == 0) {
            // chunks of at most kMaxUnitsPerLaunch float4 units: buffer byte offsets stay below 2^32
            const uint32_t nv_all = (uint32_t)(n / 4);
            hipStream_t sm = stream();
            for (uint32_t vbase = 0; vbase < nv_all; vbase += kMaxUnitsPerLaunch) {
                const uint32_t nv = nv_all - vbase < kMaxUnitsPerLaunch ? nv_all - vbase : kMaxUnitsPerLaunch;
                const dim3 g(grid_for(nv, kBlock * 2)), b(kBlock);
                const float *xf = (const float*)x + (size_t)vbase * 4, *qsf = (const float*)qs, *dsf = (const float*)ds;
                float* yf = (float*)y + (size_t)vbase * 4;
                switch (code_dtype) {
                case kU8: hipLaunchKernelGGL((k_qdq_fused<kU8>), g, b, 0, sm, xf, qsf, qz, dsf, dz, yf, nv); break;
                case kI8: hipLaunchKernelGGL((k_qdq_fused<kI8>), g, b, 0, sm, xf, qsf, qz, dsf, dz, yf, nv); break;
                case kE4M3: hipLaunchKernelGGL((k_qdq_fused<kE4M3>), g, b, 0, sm, xf, qsf, qz, dsf, dz, yf, nv); break;
                default: hipLaunchKernelGGL((k_qdq_fused<kE5M2>), g, b, 0, sm, xf, qsf, qz, dsf, dz, yf, nv); break;
                }
                if (!check_launch(name)) { st.finish(); return; }
            }
            st.finish();
            return;
        }
        st.finish();
    }
    if (code_dtype < 0 || code_dtype > DTYPE_INT64) { set_error("%s: unknown code dtype %d", name, code_dtype); return; }
    Tensor* C = (X->data && tensor_is_device(X)) ? create_tensor_device_empty(X->shape, X->ndim, (DataType)code_dtype)
                                                 : create_tensor(X->shape, X->ndim, (DataType)code_dtype);
    if (!C) { set_error("%s: no memory for the codes", name); return; }
    tensor_ops_hip_clear_error();
    qdq_entry<true>("quantize_linear_forward", X, QS, QZ, C);
    if (tensor_ops_hip_last_error()[0] == 0) qdq_entry<false>("dequantize_linear_forward", C, DS, DZ, Y);
    free_tensor(C);
}

}  // namespace

// Resolves `scratch` on the library's device (current during initialisation)
// and keeps its address per device.
void init_qdq_workspace() {
    const int dev = device_id();
    if (dev < 0 || dev >= kMaxScratchDevices) { set_error("no-allocation scratch: device %d out of range", dev); return; }
    void* p = nullptr;
    if (check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"))
        g_scratch_ptr[dev] = (double*)p;
}
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
void dynamic_quantize_linear_forward(const Tensor* x, Tensor* y, Tensor* y_scale, Tensor* y_zp) {
    dql_entry(x, y, y_scale, y_zp);
}
void dynamic_quantize_linear_forward_noalloc(const Tensor* x, Tensor* y, Tensor* y_scale, Tensor* y_zp) {
    dql_entry(x, y, y_scale, y_zp, true);
}
void dequantize_linear_axis_forward(const Tensor* X, const Tensor* Scale, const Tensor* ZeroPoint, Tensor* Y,
                                    int axis) {
    qdq_axis_entry<false>("dequantize_linear_axis_forward", X, Scale, ZeroPoint, Y, axis);
}
void quantize_dequantize_linear_forward(const Tensor* X, const Tensor* QScale, const Tensor* QZeroPoint,
                                        const Tensor* DScale, const Tensor* DZeroPoint, Tensor* Y, int code_dtype) {
    qdq_fused_entry(X, QScale, QZeroPoint, DScale, DZeroPoint, Y, code_dtype);
}
}
