// common.h — element codecs, typed access and broadcast indexing shared by all
// kernels of libtensor_ops_hip.so.  Everything here is __host__ __device__ so
// the host-side runtime and the gfx950 kernels use one definition.
//
// Numeric contract (tensor_ops/tensor_ops.c:104-588): every element is decoded
// to double, the operator computes in double, and the result is written
// through the output encoder; narrow float outputs are rounded double ->
// float -> code.  Integer outputs of a float computation use rint and the x86
// cvttsd2si rule (out of range or NaN gives INT64_MIN) before saturation.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define TO_HD __host__ __device__ __forceinline__

namespace tohip {

enum Dt : int {
    kE4M3 = 0, kE5M2 = 1, kF16 = 2, kBF16 = 3, kF32 = 4, kF64 = 5,
    kI4 = 6, kI8 = 7, kU8 = 8, kI16 = 9, kI32 = 10, kI64 = 11, kNumDt = 12
};

TO_HD bool dt_is_int(int dt) { return dt >= kI4 && dt <= kI64; }
TO_HD bool dt_valid(int dt) { return dt >= 0 && dt < kNumDt; }
TO_HD size_t dt_bytes(int dt) {
    switch (dt) {
    case kF16: case kBF16: case kI16: return 2;
    case kF32: case kI32: return 4;
    case kF64: case kI64: return 8;
    default: return 1;
    }
}

TO_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
TO_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// (int64_t)d with x86 semantics: NaN and values outside [-2^63, 2^63) -> INT64_MIN.
TO_HD int64_t cvt_i64(double d) {
    return (d >= -9223372036854775808.0 && d < 9223372036854775808.0) ? (int64_t)d : INT64_MIN;
}
TO_HD int64_t sat(int64_t v, int64_t lo, int64_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

// ----------------------------------------------------------------------------
// Encoders (float -> storage code).  Bit-level definitions:
//  f16  : IEEE round-to-nearest-even with subnormals, except |x| < 2^-24 -> +-0
//         and NaN -> sign|0x7FFF  (tensor_ops.c:104-152)
//  bf16 : RNE on the top 16 bits; NaN -> (bits >> 16) | 0x40  (tensor_ops.c:192-210)
//  e4m3 : RNE, |x| < 2^-6 -> +-0, saturate to 0x7E (also inf), NaN -> 0x7F|s  (:258-287)
//  e5m2 : RNE, |x| < 2^-14 -> +-0, >= 2^16 after rounding and inf -> 0x7C|s,
//         NaN -> 0x7D|s  (:318-347)
// All four work on the magnitude bits a = |x| and add rounding bias in the
// integer domain: (a + half - 1 + lsb) >> drop is RNE on the dropped bits.
// ----------------------------------------------------------------------------
TO_HD uint16_t enc_f16(float f) {
    const uint32_t u = f2u(f), a = u & 0x7FFFFFFFu;
    const uint16_t s = (uint16_t)((u >> 16) & 0x8000u);
#ifdef __HIP_DEVICE_COMPILE__
    // v_cvt_f16_f32 under the default round-to-nearest-even mode with f16
    // denormals kept is the integer rounding below for every |f| >= 2^-24
    // (subnormal results included, overflow to inf from 65520 up); the
    // reference's two departures from it are selected in, branch-free: NaN
    // gives sign | 0x7FFF, and magnitudes below 2^-24 give a signed zero
    // where the hardware would round (2^-25, 2^-24) up to 2^-24.  Checked
    // against the reference over all 2^32 inputs on the GPU.
    const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)f);
    const uint16_t r = a > 0x7F800000u ? (uint16_t)(s | 0x7FFF) : h;
    return a < 0x33800000u ? s : r;
#else
    if (a > 0x7F800000u) return s | 0x7FFF;
    if (a < 0x33800000u) return s;                         // below 2^-24
    if (a >= 0x38800000u) {                                // normal f16 range start 2^-14
        if (a >= 0x477FF000u) return s | 0x7C00;           // rounds to >= 2^16 (or inf)
        const uint32_t r = (a + 0xFFFu + ((a >> 13) & 1u)) >> 13;
        return (uint16_t)(s | (r - (112u << 10)));
    }
    // subnormal result: significand with hidden bit, shifted by 14..23
    const uint32_t sig = (a & 0x7FFFFFu) | 0x800000u;
    const int drop = 126 - (int)(a >> 23);                 // = -1 - e, e = exp - 127
    const uint32_t half = 1u << (drop - 1);
    const uint32_t r = (sig + half - 1u + ((sig >> drop) & 1u)) >> drop;
    return (uint16_t)(s | r);
#endif
}

TO_HD uint16_t enc_bf16(float f) {
    const uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

TO_HD uint8_t enc_e4m3(float f) {
    const uint32_t u = f2u(f), a = u & 0x7FFFFFFFu;
    const uint8_t s = (uint8_t)((u >> 24) & 0x80u);
    if (a > 0x7F800000u) return s | 0x7F;
    if (a < 0x3C800000u) return s;                         // below 2^-6
    if (a >= 0x44000000u) return s | 0x7E;                 // >= 2^9, inf
    const uint32_t q = (a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20;
    const uint32_t c = q - (120u << 3);
    return (uint8_t)(s | (c > 0x7Eu ? 0x7Eu : c));
}

TO_HD uint8_t enc_e5m2(float f) {
    const uint32_t u = f2u(f), a = u & 0x7FFFFFFFu;
    const uint8_t s = (uint8_t)((u >> 24) & 0x80u);
    if (a > 0x7F800000u) return s | 0x7D;
    if (a < 0x38800000u) return s;                         // below 2^-14
    if (a >= 0x47800000u) return s | 0x7C;                 // >= 2^16, inf
    const uint32_t q = (a + 0xFFFFFu + ((a >> 21) & 1u)) >> 21;
    const uint32_t c = q - (112u << 2);
    return (uint8_t)(s | (c > 0x7Cu ? 0x7Cu : c));
}

// ----------------------------------------------------------------------------
// Decoders (storage code -> float), exact (tensor_ops.c:160-184, 218-228, 236-256, 295-316).
// ----------------------------------------------------------------------------
TO_HD float dec_f16(uint16_t h) {
    const uint32_t s = ((uint32_t)h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 31) return u2f(s | 0x7F800000u | (m << 13));
    if (e == 0) return u2f(s | f2u((float)m * 0x1p-24f));
    return u2f(s | ((((uint32_t)h & 0x7FFFu) << 13) + (112u << 23)));
}
TO_HD float dec_bf16(uint16_t h) { return u2f((uint32_t)h << 16); }
TO_HD float dec_e4m3(uint8_t c) {
    const uint32_t s = ((uint32_t)c & 0x80u) << 24, mag = c & 0x7Fu;
    if (mag == 0x7Fu) return u2f(s | 0x7FC00000u);
    if (mag < 8u) return u2f(s | f2u((float)mag * 0x1p-9f));
    return u2f(s | ((mag << 20) + (120u << 23)));
}
TO_HD float dec_e5m2(uint8_t c) {
    const uint32_t s = ((uint32_t)c & 0x80u) << 24, mag = c & 0x7Fu;
    if (mag >= 0x7Cu) {
        const uint32_t m = mag & 3u;
        return u2f(s | 0x7F800000u | (m << 21) | (m ? 0x400000u : 0u));
    }
    if (mag < 4u) return u2f(s | f2u((float)mag * 0x1p-16f));
    return u2f(s | ((mag << 21) + (112u << 23)));
}
TO_HD int64_t dec_i4(int8_t v) { return (v & 0x08) ? (int64_t)(int8_t)(v | 0xF0) : (int64_t)(v & 0x0F); }

// ----------------------------------------------------------------------------
// Typed element access.  DT is the element type of the buffer.
// ----------------------------------------------------------------------------
template <int DT> TO_HD double ld_d(const void* p, int64_t i) {
    if constexpr (DT == kE4M3) return (double)dec_e4m3(((const uint8_t*)p)[i]);
    else if constexpr (DT == kE5M2) return (double)dec_e5m2(((const uint8_t*)p)[i]);
    else if constexpr (DT == kF16) return (double)dec_f16(((const uint16_t*)p)[i]);
    else if constexpr (DT == kBF16) return (double)dec_bf16(((const uint16_t*)p)[i]);
    else if constexpr (DT == kF32) return (double)((const float*)p)[i];
    else if constexpr (DT == kF64) return ((const double*)p)[i];
    else if constexpr (DT == kI4) return (double)dec_i4(((const int8_t*)p)[i]);
    else if constexpr (DT == kI8) return (double)((const int8_t*)p)[i];
    else if constexpr (DT == kU8) return (double)((const uint8_t*)p)[i];
    else if constexpr (DT == kI16) return (double)((const int16_t*)p)[i];
    else if constexpr (DT == kI32) return (double)((const int32_t*)p)[i];
    else return (double)((const int64_t*)p)[i];
}

// tensor_ops.c:520-546 — narrow floats use rintf, f64 uses rint, both then the x86 cast.
template <int DT> TO_HD int64_t ld_i(const void* p, int64_t i) {
    if constexpr (DT == kF64) return cvt_i64(__builtin_rint(((const double*)p)[i]));
    else if constexpr (DT <= kF32) return cvt_i64((double)__builtin_rintf((float)ld_d<DT>(p, i)));
    else if constexpr (DT == kI4) return dec_i4(((const int8_t*)p)[i]);
    else if constexpr (DT == kI8) return ((const int8_t*)p)[i];
    else if constexpr (DT == kU8) return ((const uint8_t*)p)[i];
    else if constexpr (DT == kI16) return ((const int16_t*)p)[i];
    else if constexpr (DT == kI32) return ((const int32_t*)p)[i];
    else return ((const int64_t*)p)[i];
}

template <int DT> TO_HD void st_int(void* p, int64_t i, int64_t v) {
    if constexpr (DT == kI4) ((int8_t*)p)[i] = (int8_t)sat(v, -8, 7);
    else if constexpr (DT == kI8) ((int8_t*)p)[i] = (int8_t)sat(v, -128, 127);
    else if constexpr (DT == kU8) ((uint8_t*)p)[i] = (uint8_t)sat(v, 0, 255);
    else if constexpr (DT == kI16) ((int16_t*)p)[i] = (int16_t)sat(v, -32768, 32767);
    else if constexpr (DT == kI32) ((int32_t*)p)[i] = (int32_t)sat(v, INT32_MIN, INT32_MAX);
    else ((int64_t*)p)[i] = v;
}

// Code of a float value for the narrow float types (the float -> code step).
template <int DT> TO_HD void st_code(void* p, int64_t i, float f) {
    if constexpr (DT == kE4M3) ((uint8_t*)p)[i] = enc_e4m3(f);
    else if constexpr (DT == kE5M2) ((uint8_t*)p)[i] = enc_e5m2(f);
    else if constexpr (DT == kF16) ((uint16_t*)p)[i] = enc_f16(f);
    else if constexpr (DT == kBF16) ((uint16_t*)p)[i] = enc_bf16(f);
    else ((float*)p)[i] = f;
}

// tensor_ops.c:571-588 (set_tensor_value_from_float)
template <int DT> TO_HD void st_d(void* p, int64_t i, double v) {
    if constexpr (DT == kF64) ((double*)p)[i] = v;
    else if constexpr (DT <= kF32) st_code<DT>(p, i, (float)v);
    else st_int<DT>(p, i, cvt_i64(__builtin_rint(v)));
}

// tensor_ops.c:552-569 (set_tensor_value_from_int)
template <int DT> TO_HD void st_i(void* p, int64_t i, int64_t v) {
    if constexpr (DT == kF64) ((double*)p)[i] = (double)v;
    else if constexpr (DT <= kF32) st_code<DT>(p, i, (float)v);
    else st_int<DT>(p, i, v);
}

// Runtime-dtype dispatch (the dtype is uniform per launch, so the switch is a
// scalar branch on the GPU).
#define TOHIP_DT_SWITCH(dt, BODY)                 \
    switch (dt) {                                 \
    case kE4M3: { constexpr int D = kE4M3; BODY; } break; \
    case kE5M2: { constexpr int D = kE5M2; BODY; } break; \
    case kF16: { constexpr int D = kF16; BODY; } break;   \
    case kBF16: { constexpr int D = kBF16; BODY; } break; \
    case kF32: { constexpr int D = kF32; BODY; } break;   \
    case kF64: { constexpr int D = kF64; BODY; } break;   \
    case kI4: { constexpr int D = kI4; BODY; } break;     \
    case kI8: { constexpr int D = kI8; BODY; } break;     \
    case kU8: { constexpr int D = kU8; BODY; } break;     \
    case kI16: { constexpr int D = kI16; BODY; } break;   \
    case kI32: { constexpr int D = kI32; BODY; } break;   \
    default: { constexpr int D = kI64; BODY; } break;     \
    }

TO_HD double ld_d_rt(int dt, const void* p, int64_t i) {
    double r = 0.0;
    TOHIP_DT_SWITCH(dt, r = ld_d<D>(p, i));
    return r;
}
TO_HD int64_t ld_i_rt(int dt, const void* p, int64_t i) {
    int64_t r = 0;
    TOHIP_DT_SWITCH(dt, r = ld_i<D>(p, i));
    return r;
}
TO_HD void st_d_rt(int dt, void* p, int64_t i, double v) { TOHIP_DT_SWITCH(dt, st_d<D>(p, i, v)); }
TO_HD void st_i_rt(int dt, void* p, int64_t i, int64_t v) { TOHIP_DT_SWITCH(dt, st_i<D>(p, i, v)); }

// ----------------------------------------------------------------------------
// Streaming access: nontemporal loads / stores for operands touched once.
// ----------------------------------------------------------------------------
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld_stream(const float4* p) {
    const f32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
    return make_float4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ void st_stream(float4* p, float4 v) {
    const f32x4_t t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<f32x4_t*>(p));
}
__device__ __forceinline__ uint32_t ld_stream(const uint32_t* p) { return __builtin_nontemporal_load(p); }

// Buffer resources: loads at byte offsets >= `bytes` return zero without a
// memory access, so a tile beyond the end of a tensor can be loaded without a
// branch (which would force the compiler to wait for every outstanding load).
// Word 3 is the gfx9 raw-buffer format (32-bit data, no swizzle).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// A buffer offset past every resource built here (each covers < 2 GB): loads
// through it return zero, which makes masked gathers branch-free.
constexpr uint32_t kOOB = 0x80000000u;
// 16-byte nontemporal load through a buffer resource.
__device__ __forceinline__ float4 ld_buf_stream(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    typedef unsigned int u32x4_t __attribute__((__vector_size__(16)));
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 2 /* nt */);
    return make_float4(u2f(v[0]), u2f(v[1]), u2f(v[2]), u2f(v[3]));
}
__device__ __forceinline__ void st_stream(uint32_t* p, uint32_t v) { __builtin_nontemporal_store(v, p); }

// ----------------------------------------------------------------------------
// Broadcast indexing.  Output shape is collapsed to at most kMaxDims dims
// (adjacent dims merge when every operand is contiguous across them); each
// operand has one element stride per dim (0 where it broadcasts).
// ----------------------------------------------------------------------------
constexpr int kMaxDims = 8;
constexpr int kMaxOperands = 4;

// Division by a run-time invariant d >= 1 for 32-bit numerators:
// q = (umulhi(n, m) + n) >> s with s = ceil(log2 d), m = 2^32 (2^s - d) / d + 1.
struct FastDiv {
    uint32_t d, m, s;
    TO_HD uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
        const uint32_t hi = __umulhi(n, m);
#else
        const uint32_t hi = (uint32_t)(((uint64_t)n * m) >> 32);
#endif
        return (uint32_t)(((uint64_t)hi + n) >> s);
    }
};

inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    f.d = d;
    uint32_t s = 0;
    while ((1ull << s) < d) s++;
    f.s = s;
    f.m = (uint32_t)(((1ull << 32) * ((1ull << s) - d)) / d + 1);
    return f;
}

struct BDesc {
    int nd;                                  // collapsed dims (>= 1), innermost last
    uint32_t dim[kMaxDims];
    FastDiv fd[kMaxDims];
    int64_t dim64[kMaxDims];
    int64_t st[kMaxOperands][kMaxDims];      // element strides per operand
};

// Offsets of the element with output linear index i (< 2^32), fast-div path.
// ND is the collapsed rank when known at compile time, 0 for "use d.nd".
template <int NOP, int ND = 0>
TO_HD void bd_offsets32(const BDesc& d, uint32_t i, int64_t (&off)[NOP]) {
    const int nd = ND > 0 ? ND : d.nd;
    for (int k = 0; k < NOP; k++) off[k] = 0;
#pragma unroll
    for (int a = (ND > 0 ? ND : kMaxDims) - 1; a > 0; a--) {
        if (ND == 0 && a >= nd) continue;
        const uint32_t q = d.fd[a].div(i);
        const uint32_t c = i - q * d.dim[a];
        for (int k = 0; k < NOP; k++) off[k] += (int64_t)c * d.st[k][a];
        i = q;
    }
    for (int k = 0; k < NOP; k++) off[k] += (int64_t)i * d.st[k][0];
}

// 64-bit fallback for very large tensors.
template <int NOP> TO_HD void bd_offsets64(const BDesc& d, int64_t i, int64_t (&off)[NOP]) {
    for (int k = 0; k < NOP; k++) off[k] = 0;
    for (int a = d.nd - 1; a > 0; a--) {
        const int64_t q = i / d.dim64[a];
        const int64_t c = i - q * d.dim64[a];
        for (int k = 0; k < NOP; k++) off[k] += c * d.st[k][a];
        i = q;
    }
    for (int k = 0; k < NOP; k++) off[k] += i * d.st[k][0];
}

// One-launch exchanges: a 64-bit word holds (tag, 32-bit payload), written and
// read with relaxed device-scope atomics (single-copy atomic words, coherent
// across the XCDs' L2s).  A word is current exactly when it carries the call's
// tag, so no fence, zeroing or reset of the slots is needed.
__device__ __forceinline__ void xchg_pub(unsigned long long* p, uint32_t tag, uint32_t v) {
    __hip_atomic_store(p, ((unsigned long long)tag << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool xchg_get(const unsigned long long* p, uint32_t tag, uint32_t& v) {
    const unsigned long long w = __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
    v = (uint32_t)w;
    return (uint32_t)(w >> 32) == tag;
}

// ---- wave-wide reductions without LDS --------------------------------------------
// Another lane's value (float or double) by DPP moves (CTRL: a pattern whose
// source lanes all exist, e.g. a quad permutation or a row mirror).
template <int CTRL, class T> __device__ __forceinline__ T dpp_mov(T v) {
    if constexpr (sizeof(T) == 8) {
        const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
        const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)u, CTRL, 0xF, 0xF, false);
        const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(u >> 32), CTRL, 0xF, 0xF, false);
        return __builtin_bit_cast(T, ((unsigned long long)hi << 32) | lo);
    } else {
        return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
    }
}
// The gfx950 permlane swaps: a receives the value of the even partner (row 2k
// of a row pair for W = 16, the low half of the wave for W = 32) and b that of
// the odd partner, in every lane of the pair.
template <int W, class T> __device__ __forceinline__ void permlane_pair(T v, T& a, T& b) {
    if constexpr (sizeof(T) == 8) {
        const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
        const unsigned lo = (unsigned)u, hi = (unsigned)(u >> 32);
        const auto l = W == 16 ? __builtin_amdgcn_permlane16_swap(lo, lo, false, false)
                               : __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
        const auto h = W == 16 ? __builtin_amdgcn_permlane16_swap(hi, hi, false, false)
                               : __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
        a = __builtin_bit_cast(T, ((unsigned long long)h[0] << 32) | l[0]);
        b = __builtin_bit_cast(T, ((unsigned long long)h[1] << 32) | l[1]);
    } else {
        const unsigned u = __builtin_bit_cast(unsigned, v);
        const auto l = W == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                               : __builtin_amdgcn_permlane32_swap(u, u, false, false);
        a = __builtin_bit_cast(T, (unsigned)l[0]);
        b = __builtin_bit_cast(T, (unsigned)l[1]);
    }
}
// The value of lane l - 1 in lane l (DPP wave_shr:1; lane 0 receives 0), all 64
// lanes active: a VALU move instead of an LDS-pipe permute.
__device__ __forceinline__ float lane_prev(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x138, 0xF, 0xF, false));
}

// op over the wave's 64 lanes, the result in every lane (all 64 lanes must be
// active).  Lanes pair up as quad neighbours, quad halves, 8-lane halves
// (row_half_mirror) and 16-lane halves (row_mirror) with DPP moves, then rows
// 0 / 1 and 2 / 3 and the two wave halves with permlane swaps: no LDS traffic.
// The association order is fixed, so a sum over the same values always returns
// the same bits.
template <class T, class OP> __device__ __forceinline__ T wave_allreduce(T v, OP op) {
    v = op(v, dpp_mov<0xB1>(v));     // quad_perm [1, 0, 3, 2]
    v = op(v, dpp_mov<0x4E>(v));     // quad_perm [2, 3, 0, 1]
    v = op(v, dpp_mov<0x141>(v));    // row_half_mirror
    v = op(v, dpp_mov<0x140>(v));    // row_mirror
    T a, b;
    permlane_pair<16>(v, a, b);
    v = op(a, b);
    permlane_pair<32>(v, a, b);
    return op(a, b);
}

}  // namespace tohip
