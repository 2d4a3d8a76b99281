// quant.h — the per-element quantize arithmetic shared by the Q/DQ kernels
// (qdq.hip, whose header comment proves the fast path exact) and the fused
// fake-quantization epilogue of the convolution kernels (conv.hip).
//
// tensor_ops/tensor_ops.c:999-1034: quantize y = s != 0 ? rint(x / s) + zp : zp in
// double, then the output encoder; dequantize y = (x - zp) * s in double.
#pragma once

#include "runtime.h"

namespace tohip {

template <int YDT> __device__ __forceinline__ uint8_t code8(double r) {
    if constexpr (YDT == kU8) return (uint8_t)sat(cvt_i64(__builtin_rint(r)), 0, 255);
    else if constexpr (YDT == kI8) return (uint8_t)(int8_t)sat(cvt_i64(__builtin_rint(r)), -128, 127);
    else if constexpr (YDT == kI4) return (uint8_t)(int8_t)sat(cvt_i64(__builtin_rint(r)), -8, 7);
    else if constexpr (YDT == kE4M3) return enc_e4m3((float)r);
    else return enc_e5m2((float)r);
}

__device__ __forceinline__ double qval(double x, double s, double z) { return s != 0.0 ? __builtin_rint(x / s) + z : z; }

// Quantization parameters of one scale / zero-point pair.
struct QParm {
    float s, rs, hs, zf;   // scale, ~1/s, |s|/2, zero point (+128 for i8 outputs)
    double zd;             // zero point as the reference reads it
    bool fast;             // zero point integral with |zp| < 2^22
};

template <int YDT>
__device__ __forceinline__ QParm qparm(float s, double zd) {
    QParm p;
    p.s = s;
    p.rs = __builtin_amdgcn_rcpf(s);
    p.hs = __builtin_fabsf(s) * 0.5f;
    p.zd = zd;
    const float zf = (float)p.zd;
    p.fast = (double)zf == p.zd && __builtin_rintf(zf) == zf && __builtin_fabsf(zf) < 0x1p22f;
    p.zf = (YDT == kI8) ? zf + 128.0f : zf;
    return p;
}

// r + zp of one element through the fast path; good becomes false when the
// lane must be recomputed exactly.
__device__ __forceinline__ float qfast(float x, const QParm& p, bool& good) {
    const float r = __builtin_rintf(x * p.rs);
    const float rho = __builtin_fmaf(-r, p.s, x);
    good = good && p.fast && (__builtin_fabsf(rho) < p.hs);
    return r + p.zf;
}

// Fake quantization, DequantizeLinear(QuantizeLinear(v)), of one fp32 value
// with one-element parameters and uint8 (kind 1) or int8 (kind 2) codes.  The
// quantize step is the Q kernels' (fast path with the fp64 fallback per
// element, the v_cvt_pk_u8_f32 encoder; int8 adds 128 first, so the code is
// the unsigned byte minus 128), the dequantize step k_dequant_v's ((c - zp) * s
// rounded once, here in f32, which gives those bits for integer codes), so the
// value equals the operator pair bit for bit.
struct FakeQuant {           // device pointers to one-element tensors; kind 0: none
    const float* qs;         // QuantizeLinear scale
    const void* qz;          // its zero point (code dtype), or null for 0
    const float* ds;         // DequantizeLinear scale
    const void* dz;          // its zero point (code dtype), or null for 0
    int kind;
};

struct FQParm {
    QParm p;
    double sd, zd;           // dequantize scale and zero point
    float shift;             // 0 (uint8) or 128 (int8)
    int kind;
};

__device__ __forceinline__ double fq_code(const void* z, bool i8) {
    return z ? (i8 ? (double)*(const int8_t*)z : (double)*(const uint8_t*)z) : 0.0;
}

__device__ __forceinline__ FQParm fq_parm(const FakeQuant& f) {
    FQParm r;
    const bool i8 = f.kind == 2;
    const double zq = fq_code(f.qz, i8);
    r.p = i8 ? qparm<kI8>(f.qs[0], zq) : qparm<kU8>(f.qs[0], zq);
    r.sd = (double)f.ds[0];
    r.zd = fq_code(f.dz, i8);
    r.shift = i8 ? 128.0f : 0.0f;
    r.kind = f.kind;
    return r;
}

__device__ __forceinline__ float fq_apply(float v, const FQParm& f) {
    bool good = true;
    const float q = qfast(v, f.p, good);
    float c = (float)(__builtin_amdgcn_cvt_pk_u8_f32(q, 0, 0u) & 0xFFu) - f.shift;
    if (!good) {
        const double r = qval((double)v, (double)f.p.s, f.p.zd);
        c = f.kind == 2 ? (float)(int8_t)code8<kI8>(r) : (float)code8<kU8>(r);
    }
    // c - zp is an exact integer of at most 9 bits, so the f32 product is the
    // correctly rounded exact product: the double expression's value
    return (c - (float)f.zd) * (float)f.sd;
}

}  // namespace tohip
