// qconv.hip — QDQ convolution blocks on int8 MFMA for gfx950.
//
// A QDQ residual block (ONNX: QuantizeLinear -> DequantizeLinear -> Conv whose
// weight is a DequantizeLinear of int8 codes with per-output-channel scales ->
// Relu -> Add(skip), the skip being a tensor or a 1x1 projection Conv of the
// same activation) evaluates, per output channel m and pixel p,
//   conv[m, p] = sum_k ((x_k - zx) sx) (w[m, k] sw[m])
// over the dequantized operands (tensor_ops.c:1036-1114 for the Conv,
// :1018-1034 for DequantizeLinear).  With integer codes the sum factors as
//   conv[m, p] = sx sw[m] S,   S = sum_k w[m, k] (x_k - zx),
// and S is an integer: these kernels accumulate it exactly in int32 on
// v_mfma_i32_32x32x32_i8, scale it once in double and round to f32.  The
// reference rounds each dequantized operand to f32 before it multiplies, so the
// two differ by at most 2^-23 of sum_k |term_k| plus the final rounding: the
// tolerance class of the f32 MFMA convolution (there is no exact mode here).
// Integer sums do not depend on the order of the k steps, so splitting k over
// waves changes no bit.
//
// Layouts, internal to these kernels:
//  * activations channels-last, [N, H, W, C] int8 holding code - 128 for uint8
//    codes (the code itself for int8), so the 16 channels one lane feeds to an
//    MFMA are one 16-byte load and the MFMA's signed operand is the code
//    shifted by `shift` (128 or 0):
//      S = sum_k w[m, k] (x_k - shift) - (zx - shift) sum_k w[m, k],
//    with padded taps read as zx - shift (their dequantized value is 0);
//  * weights [M, KH, KW, C] int8 (k = tap * C + c, zero points 0) with the
//    per-channel code sums that the correction needs.
//
//  * k_quant_nhwc — QuantizeLinear of an f32 NCHW tensor into that layout (the
//    codes are quantize_linear_forward's, bit for bit).
//  * k_qconv_pack — [M, C, KH, KW] int8 weight codes -> [M, KH, KW, C] and the
//    per-tap code sums.
//  * k_qconv — the block: implicit GEMM over k = (tap, 32-channel step), 64
//    output channels x 64 pixels per wave (2x2 MFMA tiles of 32x32, operands
//    loaded straight into registers one step ahead), optionally the 1x1
//    projection into a second accumulator set, then the epilogue
//    [Relu](conv + b) [+ proj | + skip] written as f32 NCHW, or quantized for
//    the next block into its channels-last codes.  KS = 1: a 256-thread block
//    is 4 waves side by side along the pixels; KS = 4: the 4 waves split one
//    tile's k steps and add their integer partials through LDS.
#include <algorithm>
#include <cmath>

#include "quant.h"
#include "runtime.h"

namespace tohip {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

struct QGeom {
    int N, C, H, W, M, KH, KW, OH, OW, pt, pl, sh, sw, dh, dw;
    int P, OHW, csteps;     // N * OH * OW, OH * OW, C / 32
    int steps, psteps;      // main k steps (KH * KW * csteps), projection k steps (csteps or 0)
    FastDiv fd_ohw, fd_ow, fd_cs, fd_kw;
};

struct QEpi {
    const float* xs;        // input DequantizeLinear scale (one element)
    const void* xz;         // its zero point (one element of the code dtype), or null: 0
    int xkind;              // input codes: 1 uint8 (stored code - 128), 2 int8
    const int* wsum;        // [M, KH * KW] weight code sums per tap
    const float* ws;        // [M] weight scales
    const float* bias;      // [M] or null
    const int* psum;        // projection [M] code sums (its one tap)
    const float* ps;        // projection [M] scales
    const float* skip;      // f32 [N, M, OH, OW] residual or null
    int relu;
    const float* qs;        // output quantization (codes out): scale,
    const void* qz;         // zero point (one element of the code dtype), or null: 0
    int qkind;              // output codes: 1 uint8, 2 int8
};

// LDS byte address of a __shared__ object (the offset ds_read takes)
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

__device__ __forceinline__ int code_at(const void* z, int kind) {
    return z ? (kind == 2 ? (int)*(const int8_t*)z : (int)*(const uint8_t*)z) : 0;
}

// Output quantization of one value into the stored byte (code - 128 for
// uint8, the code for int8): quantize_linear_forward's code through the Q
// kernels' fast path, the fp64 expression where that path cannot decide.
struct QOut {
    QParm p;
    int kind;
};

__device__ __forceinline__ uint32_t qout_byte(float v, const QOut& q) {
    bool good = true;
    const float r = qfast(v, q.p, good);
    // v_cvt_pk_u8_f32 clamps to [0, 255]: the uint8 code, or the int8 code + 128
    uint32_t b = __builtin_amdgcn_cvt_pk_u8_f32(r, 0, 0u) & 0xFFu;
    if (!good) {
        const double rr = qval((double)v, (double)q.p.s, q.p.zd);
        b = q.kind == 2 ? (uint32_t)((int)(int8_t)code8<kI8>(rr) + 128) : (uint32_t)code8<kU8>(rr);
    }
    return b ^ 0x80u;
}

__device__ __forceinline__ QOut qout_parm(const float* qs, const void* qz, int kind) {
    QOut q;
    const double zq = (double)code_at(qz, kind);
    q.p = kind == 2 ? qparm<kI8>(qs[0], zq) : qparm<kU8>(qs[0], zq);
    q.kind = kind;
    return q;
}

// ---- QuantizeLinear into channels-last codes --------------------------------
// Block: one image, 64 consecutive pixels x 32 channels.  VEC (H W % 4 == 0):
// thread t reads 4 consecutive pixels (one float4) of channel t / 16 + 16 e, so
// 16 lanes cover a channel's 256 contiguous bytes; otherwise one pixel of
// channels t / 64 + 4 e.  The codes go through LDS ([pixel][channel] bytes) and
// 128 threads write the 64 pixels' 32-byte channel runs as 16-byte stores.
template <bool VEC>
__global__ __launch_bounds__(256) void k_quant_nhwc(const float* __restrict__ X, int8_t* __restrict__ Y,
                                                    const float* __restrict__ qs, const void* __restrict__ qz,
                                                    int kind, int C, int HW) {
    __shared__ uint32_t tile[64][9];          // 64 pixels x 32 bytes (+4: distinct banks per pixel)
    const int t = threadIdx.x;
    const int n = blockIdx.z, c0 = blockIdx.y * 32, px0 = blockIdx.x * 64;
    const QOut q = qout_parm(qs, qz, kind);
    const float* xb = X + ((size_t)n * C + c0) * HW + px0;
    if constexpr (VEC) {
        const int quad = t & 15, cq = t >> 4;
        const bool ok = px0 + 4 * quad < HW;      // HW % 4 == 0: a quad is all in or all out
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int c = cq + 16 * e;
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (ok) v = *reinterpret_cast<const float4*>(xb + (size_t)c * HW + 4 * quad);
            const float f[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
                reinterpret_cast<uint8_t*>(&tile[4 * quad + i][0])[c] = (uint8_t)qout_byte(f[i], q);
        }
    } else {
        const int px = t & 63, cq = t >> 6;
        const bool ok = px0 + px < HW;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int c = cq + 4 * e;
            const float v = ok ? xb[(size_t)c * HW + px] : 0.0f;
            reinterpret_cast<uint8_t*>(&tile[px][0])[c] = (uint8_t)qout_byte(v, q);
        }
    }
    __syncthreads();
    if (t < 128) {
        const int p = t >> 1, part = t & 1;
        if (px0 + p < HW) {
            const uint32_t* s = &tile[p][4 * part];
            uint4 w = make_uint4(s[0], s[1], s[2], s[3]);
            *reinterpret_cast<uint4*>(Y + ((size_t)n * HW + px0 + p) * C + c0 + 16 * part) = w;
        }
    }
}

// C % 64 == 0 and H W % 4 == 0: a block covers 64 pixels x 64 channels; thread t
// loads 4 consecutive pixels (one float4) of channels 4 (t / 16) .. + 3 (16 lanes
// per 256-byte channel row), packs each pixel's 4 codes into one word for LDS,
// and every thread then stores 16 of the 64 pixels' 64-byte channel runs.
__global__ __launch_bounds__(256) void k_quant_nhwc64(const float* __restrict__ X, int8_t* __restrict__ Y,
                                                      const float* __restrict__ qs, const void* __restrict__ qz,
                                                      int kind, int C, int HW) {
    __shared__ uint32_t tile[64][17];         // 64 pixels x 64 bytes (+4: distinct banks per pixel)
    const int t = threadIdx.x;
    const int n = blockIdx.z, c0 = blockIdx.y * 64, px0 = blockIdx.x * 64;
    const QOut q = qout_parm(qs, qz, kind);
    const int quad = t & 15, cg = t >> 4;
    const bool ok = px0 + 4 * quad < HW;          // HW % 4 == 0: a quad is all in or all out
    const float* xb = X + ((size_t)n * C + c0 + 4 * cg) * HW + px0 + 4 * quad;
    float4 v[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
        v[j] = ok ? *reinterpret_cast<const float4*>(xb + (size_t)j * HW) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t w = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float f = i == 0 ? v[j].x : i == 1 ? v[j].y : i == 2 ? v[j].z : v[j].w;
            w |= qout_byte(f, q) << (8 * j);
        }
        tile[4 * quad + i][cg] = w;
    }
    __syncthreads();
    const int p = t >> 2, part = t & 3;
    if (px0 + p < HW) {
        const uint32_t* s = &tile[p][4 * part];
        *reinterpret_cast<uint4*>(Y + ((size_t)n * HW + px0 + p) * C + c0 + 16 * part) =
            make_uint4(s[0], s[1], s[2], s[3]);
    }
}

// ---- MaxPool with the channels-last codes of its output -----------------------
// max_pool_forward (f32, 3x3, stride 2, top / left padding 1, W == 2 OW, OW <=
// 64) and quantize_linear_nhwc_forward of its output in one pass.  Block: a
// strip of kMPRows output rows of 16 channels of one image; wave w pools the
// group's channel w, its input rows loaded up front (one wait for memory per
// wave).  Output row oh reads input rows 2oh-1, 2oh, 2oh+1, each tap in the
// reference's order with a strict > (a NaN never wins, the padding is -inf),
// as the plain MaxPool kernel; lane l holds input columns (2l, 2l+1) and takes
// column 2l-1 from lane l-1.  The f32 result goes to Y (NCHW, cached stores:
// the next layer reads it as its residual), its code to LDS [pixel][channel],
// and the strip's codes leave as one 16-byte store per pixel.
constexpr int kMPRows = 7;
__global__ __launch_bounds__(1024) void k_maxpool_q16(const float* __restrict__ X, float* __restrict__ Y,
                                                     int8_t* __restrict__ Yc, const float* __restrict__ qs,
                                                     const void* __restrict__ qz, int kind, int C, int H, int W,
                                                     int OH, int OW, int strips) {
    __shared__ uint32_t tile[kMPRows * 64][5];    // [pixel][16 channel bytes] (+1 word: distinct banks per pixel)
    uint8_t* t8 = reinterpret_cast<uint8_t*>(&tile[0][0]);
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = threadIdx.x & 63;
    // work index: each XCD (block index mod 8) takes a contiguous run of
    // (image, strip, channel group), channel group fastest: the four blocks
    // that fill one pixel's 64 bytes of codes write through one L2, and
    // neighbouring strips share their edge input row through it
    int strip, c0, n;
    {
        const int groups = C / 16, total = strips * groups * (int)gridDim.y;
        const int L = (int)blockIdx.x + (int)blockIdx.y * (int)gridDim.x;
        const int cls = L & 7, q = total >> 3, rem = total & 7;
        const int w = cls * q + min(cls, rem) + (L >> 3);
        c0 = (w % groups) * 16;
        const int rest = w / groups;
        strip = rest % strips;
        n = rest / strips;
    }
    const int oh0 = strip * kMPRows, nrow = min(kMPRows, OH - oh0);
    const uint32_t plane = (uint32_t)H * W;
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X + ((size_t)n * C + c0) * plane, 16u * plane * 4u);
    const QOut q = qout_parm(qs, qz, kind);
    const float ninf = -__builtin_inff();
    const uint32_t lo = (uint32_t)lane * 8u;
    // (HIP's float2 struct: hipcc folds a bit_cast of an ext_vector element to element 0)
    auto ldrows = [&](int cl, float2 (&rows)[2 * kMPRows + 1]) {
#pragma unroll
        for (int j = 0; j < 2 * kMPRows + 1; j++) {
            const int ih = 2 * oh0 - 1 + j;
            float2 v = make_float2(ninf, ninf);
            if ((unsigned)ih < (unsigned)H && j <= 2 * nrow) {   // uniform
                const uint64_t u = __builtin_bit_cast(
                    uint64_t, __builtin_amdgcn_raw_buffer_load_b64(xr, lo, ((uint32_t)cl * plane + (uint32_t)ih * W) * 4u,
                                                                   2 /* nt */));
                v = make_float2(__builtin_bit_cast(float, (uint32_t)u), __builtin_bit_cast(float, (uint32_t)(u >> 32)));
            }
            rows[j] = v;
        }
    };
    auto row_max = [&](float best, float2 v) {
        const float left = __builtin_bit_cast(
            float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, ninf), __builtin_bit_cast(int, v.y),
                                               0x138 /* wave_shr:1 */, 0xF, 0xF, false));
        best = left > best ? left : best;
        best = v.x > best ? v.x : best;
        best = v.y > best ? v.y : best;
        return best;
    };
    const bool live = lane < OW;
    float2 rows[2 * kMPRows + 1];
    ldrows(wave, rows);
    float* yp = Y + (((size_t)n * C + c0 + wave) * OH + oh0) * OW;
#pragma unroll
    for (int o = 0; o < kMPRows; o++) {
        if (o >= nrow) break;
        const float best = row_max(row_max(row_max(ninf, rows[2 * o]), rows[2 * o + 1]), rows[2 * o + 2]);
        if (live) {
            yp[o * OW + lane] = best;
            t8[(o * OW + lane) * 20 + wave] = (uint8_t)qout_byte(best, q);
        }
    }
    __syncthreads();
    const int npx = nrow * OW;
    int8_t* yc = Yc + (((size_t)n * OH + oh0) * OW) * C + c0;
    for (int p = threadIdx.x; p < npx; p += 1024)
        *reinterpret_cast<uint4*>(yc + (size_t)p * C) = make_uint4(tile[p][0], tile[p][1], tile[p][2], tile[p][3]);
}

// ---- weight packing ------------------------------------------------------------
// One block per output channel: [C, KH, KW] codes -> [KH, KW, C], and the sum
// of each tap's C codes (wave w sums taps w, w + 4, ...).
__global__ __launch_bounds__(256) void k_qconv_pack(const int8_t* __restrict__ W, int8_t* __restrict__ Wk,
                                                    int* __restrict__ wsum, int C, int khw) {
    const int m = blockIdx.x, K = C * khw;
    const int8_t* src = W + (size_t)m * K;
    int8_t* dst = Wk + (size_t)m * K;
    for (int i = threadIdx.x; i < K; i += 256) {
        const int c = i / khw, tap = i - c * khw;
        dst[tap * C + c] = src[i];
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int tap = wave; tap < khw; tap += 4) {
        int s = 0;
        for (int c = lane; c < C; c += 64) s += src[c * khw + tap];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
        if (lane == 0) wsum[(size_t)m * khw + tap] = s;
    }
}

// ---- the block kernel ------------------------------------------------------------
template <int KS, bool PROJ, int OUT>
__global__ __launch_bounds__(256) void k_qconv(const int8_t* __restrict__ X, const int8_t* __restrict__ Wk,
                                               const int8_t* __restrict__ Pk, void* __restrict__ Y, QGeom g, QEpi e,
                                               uint32_t xbytes, uint32_t wbytes, uint32_t pbytes) {
    const int lane = threadIdx.x & 63, col = lane & 31, half = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int m0 = (int)blockIdx.y * 64;
    const int p0 = KS == 1 ? (int)blockIdx.x * 256 + wave * 64 : (int)blockIdx.x * 64;
    const int shift = e.xkind == 1 ? 128 : 0;
    const int zx = code_at(e.xz, e.xkind);
    const int zsh = zx - shift;
    const uint32_t padb = (uint32_t)(zsh & 0xFF) * 0x01010101u;
    const i32x4 padv = {(int)padb, (int)padb, (int)padb, (int)padb};

    // Per-channel terms of the epilogue for the block's 64 channels, in LDS
    // (filled while the k loop runs): the correction (zx - shift) sum_k w and
    // the scale sx sw (exact in double).
    __shared__ double s_cm[64], s_cp[64];
    __shared__ int s_corr[64], s_corrp[64];
    __shared__ float s_bias[64];
    const bool has_bias = e.bias != nullptr, has_skip = e.skip != nullptr;
    if (threadIdx.x < 64) {
        const int m = m0 + (int)threadIdx.x;
        const double xsd = (double)e.xs[0];
        s_cm[threadIdx.x] = xsd * (double)e.ws[m];
        int ws = 0;
        for (int t = 0; t < g.KH * g.KW; t++) ws += e.wsum[m * g.KH * g.KW + t];
        s_corr[threadIdx.x] = zsh * ws;
        s_bias[threadIdx.x] = has_bias ? e.bias[m] : 0.0f;
        if constexpr (PROJ) {
            s_cp[threadIdx.x] = xsd * (double)e.ps[m];
            s_corrp[threadIdx.x] = zsh * e.psum[m];
        }
    }

    // this lane's two pixel columns (j = 0, 1: pixels p0 + 32 j + col)
    int ih0[2], iw0[2], rowb[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int p = p0 + 32 * j + col;
        const int pp = p < g.P ? p : 0;
        const int n = (int)g.fd_ohw.div((uint32_t)pp), r = pp - n * g.OHW;
        const int oh = (int)g.fd_ow.div((uint32_t)r), ow = r - oh * g.OW;
        ih0[j] = p < g.P ? oh * g.sh - g.pt : -(1 << 29);    // a pixel past the end reads only padding
        iw0[j] = ow * g.sw - g.pl;
        rowb[j] = n * g.H;
    }
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X, xbytes);
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(Wk, wbytes);
    const __amdgpu_buffer_rsrc_t pr = buffer_rsrc(PROJ ? Pk : Wk, PROJ ? pbytes : 0u);
    const int K = g.KH * g.KW * g.C;
    const uint32_t aoff = (uint32_t)((m0 + col) * K + half * 16);
    const uint32_t poff = (uint32_t)((m0 + col) * g.C + half * 16);

    i32x16 acc[2][2], accp[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                acc[i][j][r] = 0;
                accp[i][j][r] = 0;
            }

    // Step st: the main conv's (tap, 32-channel step) for st < steps, then the
    // projection's 32-channel steps at the centre pixel (1x1, pads 0).
    auto load = [&](int st, i32x4 (&a)[2], i32x4 (&b)[2]) {
        if (!PROJ || st < g.steps) {
            const int tap = (int)g.fd_cs.div((uint32_t)st);
            const int cs = st - tap * g.csteps;
            const int kh = (int)g.fd_kw.div((uint32_t)tap), kw = tap - kh * g.KW;
            const int dy = kh * g.dh, dx = kw * g.dw;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int ih = ih0[j] + dy, iw = iw0[j] + dx;
                const bool ok = (unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W;
                const uint32_t off = ok ? (uint32_t)((((rowb[j] + ih) * g.W + iw) * g.C) + cs * 32 + half * 16) : kOOB;
                const i32x4 v = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
                b[j] = ok ? v : padv;
            }
            const uint32_t ko = (uint32_t)(tap * g.C + cs * 32);
            a[0] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, aoff + ko, 0, 0));
            a[1] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, aoff + 32 * K + ko, 0, 0));
        } else {
            const int cs = st - g.steps;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int ih = ih0[j] + g.pt, iw = iw0[j] + g.pl;
                const bool ok = (unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W;
                const uint32_t off = ok ? (uint32_t)((((rowb[j] + ih) * g.W + iw) * g.C) + cs * 32 + half * 16) : kOOB;
                b[j] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
            }
            const uint32_t ko = (uint32_t)(cs * 32);
            a[0] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, poff + ko, 0, 0));
            a[1] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, poff + 32 * g.C + ko, 0, 0));
        }
    };
    auto mfma = [&](i32x16 (&c)[2][2], const i32x4 (&a)[2], const i32x4 (&b)[2]) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) c[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], c[i][j], 0, 0, 0);
    };

    // this wave's steps [sbeg, send): the main conv's part into acc, the
    // projection's into accp, each loop loading two steps ahead
    const int total = g.steps + (PROJ ? g.psteps : 0);
    const int sbeg = KS > 1 ? wave * total / KS : 0;
    const int send = KS > 1 ? (wave + 1) * total / KS : total;
    auto run = [&](i32x16 (&c)[2][2], int b0, int b1) {
        if (b0 >= b1) return;
        i32x4 a0[2], x0[2], a1[2], x1[2];
        load(b0, a0, x0);
        if (b0 + 1 < b1) load(b0 + 1, a1, x1);
        for (int st = b0; st < b1; st++) {
            i32x4 a2[2], x2[2];
            if (st + 2 < b1) load(st + 2, a2, x2);
            mfma(c, a0, x0);
#pragma unroll
            for (int i = 0; i < 2; i++) {
                a0[i] = a1[i];
                x0[i] = x1[i];
                a1[i] = a2[i];
                x1[i] = x2[i];
            }
        }
    };
    run(acc, sbeg, min(send, g.steps));
    if constexpr (PROJ) run(accp, max(sbeg, g.steps), send);

    QOut qo;
    if constexpr (OUT == 1) qo = qout_parm(e.qs, e.qz, e.qkind);
    // value of local channel ml: [Relu](conv + b) [+ projection] [+ skip]
    auto value = [&](int A, int Ap, int ml, float sk) {
        float v = (float)((double)(A - s_corr[ml]) * s_cm[ml]);
        if (has_bias) v = v + s_bias[ml];
        if (e.relu) v = v > 0.0f ? v : 0.0f;
        if constexpr (PROJ) v = v + (float)((double)(Ap - s_corrp[ml]) * s_cp[ml]);
        if (has_skip) v = v + sk;
        return v;
    };
    // Tile (i, j): lane holds column p0 + 32 j + col and local rows
    // 32 i + 8 q + 4 half + r (q, r = 0..3) in element 4 q + r.  The skip values
    // of a wave's tiles are all loaded before its first store.
    auto ybase = [&](int j, int& p) {
        p = p0 + 32 * j + col;
        const int pp = p < g.P ? p : 0;
        const int n = (int)g.fd_ohw.div((uint32_t)pp);
        return (size_t)n * g.M * g.OHW + (size_t)(pp - n * g.OHW) + (size_t)m0 * g.OHW;
    };
    auto load_skip = [&](int i, int j, float (&sk)[16]) {
        int p;
        const size_t yb = ybase(j, p);
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int ml = 32 * i + 8 * (k >> 2) + 4 * half + (k & 3);
            sk[k] = (has_skip && p < g.P) ? e.skip[yb + (size_t)ml * g.OHW] : 0.0f;
        }
    };
    auto store = [&](const i32x16& A, const i32x16& Ap, const float (&sk)[16], int i, int j) {
        int p;
        const size_t yb = ybase(j, p);
        if (p >= g.P) return;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int mb = 32 * i + 8 * q + 4 * half;
            uint32_t word = 0;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float v = value(A[4 * q + r], Ap[4 * q + r], mb + r, sk[4 * q + r]);
                if constexpr (OUT == 0) ((float*)Y)[yb + (size_t)(mb + r) * g.OHW] = v;
                else word |= qout_byte(v, qo) << (8 * r);
            }
            if constexpr (OUT == 1)
                *reinterpret_cast<uint32_t*>((int8_t*)Y + (size_t)p * g.M + m0 + mb) = word;
        }
    };

    if constexpr (KS == 1) {
        float sk[2][2][16];
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) load_skip(i, j, sk[i][j]);
        __syncthreads();      // the per-channel table
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) store(acc[i][j], accp[i][j], sk[i][j], i, j);
    } else {
        // integer partials of the 4 waves through LDS; wave w finishes tile
        // (w / 2, w % 2)
        __shared__ int red[4][4][16][64];
        const int bi = wave >> 1, bj = wave & 1;
        float sk[16];
        load_skip(bi, bj, sk);
        i32x16 sum, sump;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) red[wave][2 * i + j][r][lane] = acc[i][j][r];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 16; r++)
            sum[r] = red[0][wave][r][lane] + red[1][wave][r][lane] + red[2][wave][r][lane] + red[3][wave][r][lane];
        if constexpr (PROJ) {
            __syncthreads();
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) red[wave][2 * i + j][r][lane] = accp[i][j][r];
            __syncthreads();
#pragma unroll
            for (int r = 0; r < 16; r++)
                sump[r] = red[0][wave][r][lane] + red[1][wave][r][lane] + red[2][wave][r][lane] + red[3][wave][r][lane];
        } else {
            sump = sum;
        }
        store(sum, sump, sk, bi, bj);
    }
}

// ---- the block kernel through an LDS ring -------------------------------------
// C % 64 == 0.  Block tile 64 channels x 64 pixels, wave w computing the
// 32x32 tile (w / 2, w % 2).  A stage is two k steps of one tap: 64 contiguous
// bytes per weight row and per pixel.  Wave w fetches its group's 32 rows of a
// stage (w = 0, 1: weight rows 32 w..; w = 2, 3: pixels 32 (w - 2)..) with two
// loads in which four lanes read one row's 64 bytes, and writes each 16 bytes
// to where lane (row, k half) of an MFMA reads them back (one contiguous
// 512 bytes per half-wave).  Stages travel through
// three register sets (loaded three iterations ahead of their LDS write) and
// three LDS slots.  A padded tap loads 16 bytes of zx - shift from a table,
// the stored form of the code whose dequantized value is 0.  The k step of
// the next load is kept as running counters (tap row, tap column, channel
// step): k = tap * C + 32 cs advances by 32 per step, so the weight offset is
// 32 st, and no step needs a division.

// 16 bytes of v for each byte value v: the padding loads
struct QPadTable {
    uint32_t w[256][4];
};
constexpr QPadTable make_qpad() {
    QPadTable t{};
    for (int v = 0; v < 256; v++)
        for (int i = 0; i < 4; i++) t.w[v][i] = (uint32_t)v * 0x01010101u;
    return t;
}
// (global, not constant, memory: a load that picks it or X stays a global load)
__device__ __attribute__((aligned(16))) QPadTable kQPad = make_qpad();
constexpr int kQSteps = 2;     // k steps per LDS stage (4: slower, the prologue covers most of a short block)
// LDS stage layout [step u][group][half h][32 rows][16 B] with pitches that put
// the 16 lanes of one 16-byte write pass (4 rows x 4 chunks) on distinct banks:
// half 512 + 64, group 2 halves, step 4 groups + 128 (128 mod 256)
constexpr int kQHalf = 576, kQGroup = 2 * kQHalf, kQStep = 4 * kQGroup + 128, kQSlot = kQSteps * kQStep;

// KG = 2 (grids of at most two blocks per CU): 8 waves per block, waves 4-7 a
// second k group that runs the second half of the stages through a ring of its
// own; its integer partial sums are added to the first group's through LDS
// (exact), and the first group writes the output.  The two groups meet at the
// same barriers (the shorter runs its last stage again without multiplying).
template <bool PROJ, int OUT, int KG>
__global__ __launch_bounds__(256 * KG) __attribute__((amdgpu_waves_per_eu(PROJ && OUT == 0 ? 3 : 4))) void k_qconv_lds(const int8_t* __restrict__ X, const int8_t* __restrict__ Wk,
                                                   const int8_t* __restrict__ Pk, void* __restrict__ Y, QGeom g,
                                                   QEpi e) {
    __shared__ __attribute__((aligned(1024))) int8_t rings[KG * 3 * kQSlot];
    __shared__ double s_cm[64], s_cp[64];
    __shared__ int s_corr[64], s_corrp[64];
    __shared__ float s_bias[64];
    const int lane = threadIdx.x & 63, col = lane & 31, half = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) & 3;
    const int grp = KG == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 8);
    int8_t* const ring = rings + grp * (3 * kQSlot);
    // Tile order: the dispatcher deals consecutive blocks to the 8 XCDs in
    // turn, each with its own L2.  Block L works on tile w, which gives XCD
    // L % 8 a contiguous run of the tiles, ordered (pixel tile, channel tile)
    // with the channel tile fastest, so an XCD's L2 holds its slice of the
    // input while the taps and channel tiles re-read it (a bijection on
    // [0, tiles) for any count).
    int m0, p0;
    {
        const int tiles = (int)gridDim.x, L = (int)blockIdx.x;
        const int cls = L & 7, q = tiles >> 3, rem = tiles & 7;
        const int w = cls * q + min(cls, rem) + (L >> 3);
        const int ntm = g.M >> 6;
        const int tp = w / ntm;
        m0 = (w - tp * ntm) * 64;
        p0 = tp * 64;
    }
    const int khw = g.KH * g.KW;
    const int shift = e.xkind == 1 ? 128 : 0;
    const int zsh = code_at(e.xz, e.xkind) - shift;
    const bool has_bias = e.bias != nullptr, has_skip = e.skip != nullptr;
    if (threadIdx.x < 64) {
        const int m = m0 + (int)threadIdx.x;
        const double xsd = (double)e.xs[0];
        int tot = 0;
        for (int t = 0; t < khw; t++) tot += e.wsum[m * khw + t];
        s_corr[threadIdx.x] = zsh * tot;
        s_cm[threadIdx.x] = xsd * (double)e.ws[m];
        s_bias[threadIdx.x] = has_bias ? e.bias[m] : 0.0f;
        if constexpr (PROJ) {
            s_cp[threadIdx.x] = xsd * (double)e.ps[m];
            s_corrp[threadIdx.x] = zsh * e.psum[m];
        }
    }

    // The loads this lane issues per stage: rows (weight rows for waves 0, 1,
    // pixels for waves 2, 3) rr[j] = 16 j + lane / 4 of the wave's 32, the 16
    // bytes at chunk lane % 4 of the stage's 64 contiguous bytes (step u =
    // chunk / 2, half h = chunk % 2): four lanes read one 64-byte run.
    const bool is_a = wave < 2;
    const int K = khw * g.C;
    const int chunk = lane & 3;
    // row rr[1] = rr[0] + 16: weight rows 16 K bytes on, LDS rows 256 bytes on
    const int8_t* const arow = Wk + (size_t)(m0 + 32 * wave + (lane >> 2)) * K + chunk * 16;
    const int8_t* const prow = PROJ ? Pk + (size_t)(m0 + 32 * wave + (lane >> 2)) * g.C + chunk * 16 : arow;
    const uint32_t loff =                     // LDS byte offset of row rr[0] in a slot
        (uint32_t)((chunk >> 1) * kQStep + wave * kQGroup + (chunk & 1) * kQHalf + (lane >> 2) * 16);
    const int8_t* xrow[2];
    int ih0[2], iw0[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int rr = 16 * j + (lane >> 2);
        ih0[j] = -(1 << 29);
        iw0[j] = 0;
        int rowb = 0;
        const int p = p0 + 32 * (wave - 2) + rr;
        if (!is_a && p < g.P) {
            const int n = (int)g.fd_ohw.div((uint32_t)p), r = p - n * g.OHW;
            const int oh = (int)g.fd_ow.div((uint32_t)r), ow = r - oh * g.OW;
            ih0[j] = oh * g.sh - g.pt;
            iw0[j] = ow * g.sw - g.pl;
            rowb = n * g.H;
        }
        xrow[j] = X + (size_t)rowb * g.W * g.C + chunk * 16;
    }
    const int8_t* const pad = reinterpret_cast<const int8_t*>(&kQPad.w[zsh & 0xFF][0]);
    const int total = g.steps + (PROJ ? g.psteps : 0);
    const int nst_all = (total + kQSteps - 1) / kQSteps;
    // this group's stages [s_beg, s_end) and the loop's trip count nst (the
    // same for both groups)
    const int s_half = (nst_all + KG - 1) / KG;
    const int s_beg = grp * s_half, s_end = min(nst_all, s_beg + s_half), nst = s_half;
    const int step_end = min(total, kQSteps * s_end);
    // Next stage to load: sst, its first channel step cs (even: a stage is two
    // steps of one tap) and tap (kh, kw); past the group's last stage the last
    // is loaded again (its copy is never read).  One global load per row on
    // every path keeps the compiler's count of loads in flight exact, so its
    // waits stay partial.
    int sst = s_beg, cs = 0, kh = 0, kw = 0;
    if (KG > 1 && s_beg > 0) {
        const int st0 = kQSteps * s_beg;
        if (st0 < g.steps) {
            const int tap = st0 / g.csteps;
            cs = st0 - tap * g.csteps;
            kh = tap / g.KW;
            kw = tap - kh * g.KW;
        } else {
            cs = st0 - g.steps;
            kh = g.KH;
        }
    }
    auto gload = [&](i32x4 (&v)[2]) {
        const bool main = !PROJ || 2 * sst < g.steps;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int ih = ih0[j] + (main ? kh * g.dh : g.pt), iw = iw0[j] + (main ? kw * g.dw : g.pl);
            const bool ok = (unsigned)ih < (unsigned)g.H && (unsigned)iw < (unsigned)g.W;
            const int8_t* pb = ok ? xrow[j] + ((size_t)ih * g.W + iw) * g.C + cs * 32 : pad;
            const int8_t* pa = main ? arow + ((size_t)j * 16 * K + (size_t)sst * 64)
                                    : prow + ((size_t)j * 16 * g.C + cs * 32);
            v[j] = *reinterpret_cast<const i32x4*>(is_a ? pa : pb);
        }
        if (sst + 1 < s_end) {
            sst++;
            cs += 2;
            if (cs == g.csteps) {
                cs = 0;
                if (++kw == g.KW) {
                    kw = 0;
                    kh++;
                }
            }
        }
    };
    auto put = [&](int slot, const i32x4 (&v)[2]) {
#pragma unroll
        for (int j = 0; j < 2; j++) *reinterpret_cast<i32x4*>(&ring[slot * kQSlot + loff + 256 * j]) = v[j];
    };

    // skip values of this wave's tile, loaded before the k loop
    const int wm = wave >> 1, wp = wave & 1;
    const int pme = p0 + 32 * wp + col;                 // this lane's output pixel
    float sk[16];
    size_t yb = 0;
    if (pme < g.P) {
        const int pn = (int)g.fd_ohw.div((uint32_t)pme);
        yb = (size_t)pn * g.M * g.OHW + (size_t)(pme - pn * g.OHW) + (size_t)(m0 + 32 * wm) * g.OHW;
    }
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int ml = 8 * (k >> 2) + 4 * half + (k & 3);
        sk[k] = (has_skip && pme < g.P && grp == 0) ? e.skip[yb + (size_t)ml * g.OHW] : 0.0f;
    }

    i32x16 acc, accp;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        acc[r] = 0;
        accp[r] = 0;
    }
    // Stage k (steps kQSteps k ..) is read from LDS slot k % 3 at iteration k;
    // iteration k first writes stage k + 1 into slot (k + 1) % 3 (last read at
    // iteration k - 2, before the previous barrier) from register set
    // (k + 1) % 3, loaded three iterations earlier, and reloads that set with
    // stage k + 4.  The loop is unrolled by three so that every register set
    // and slot index is static (a rotated copy would wait for every load in
    // flight), with loads on every path inside it for the same reason; steps
    // past the last are not multiplied.
    i32x4 R0[2], R1[2], R2[2];
    gload(R0);
    put(0, R0);
    gload(R1);
    gload(R2);
    gload(R0);
    // MFMA operand of lane l in a group: row l % 32, k half l / 32
    const uint32_t rdo = (uint32_t)((lane >> 5) * kQHalf + (lane & 31) * 16);
    auto body = [&](int k, int sr, int sw, i32x4 (&w)[2]) {
        put(sw, w);
        gload(w);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
        for (int u = 0; u < kQSteps; u++) {
            const int stp = kQSteps * (s_beg + k) + u;
            const int8_t* base = &ring[sr * kQSlot + u * kQStep + rdo];
            const i32x4 a = *reinterpret_cast<const i32x4*>(base + wm * kQGroup);
            const i32x4 b = *reinterpret_cast<const i32x4*>(base + (2 + wp) * kQGroup);
            if (stp >= step_end) break;
            if (!PROJ || stp < g.steps) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc, 0, 0, 0);
            else accp = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, accp, 0, 0, 0);
        }
    };
    int k = 0;
    for (; k + 3 <= nst; k += 3) {
        body(k, 0, 1, R1);
        body(k + 1, 1, 2, R2);
        body(k + 2, 2, 0, R0);
    }
    // the last one or two stages (their waits may be whole: no loop follows)
    if (k < nst) body(k, 0, 1, R1);
    if (k + 1 < nst) body(k + 1, 1, 2, R2);

    if constexpr (KG == 2) {
        // the second group's partial sums through the rings' memory
        int* xch = reinterpret_cast<int*>(rings);
        __syncthreads();
        if (grp == 1) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                xch[(wave * 16 + r) * 64 + lane] = acc[r];
                if constexpr (PROJ) xch[((4 + wave) * 16 + r) * 64 + lane] = accp[r];
            }
        }
        __syncthreads();
        if (grp == 1) return;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            acc[r] += xch[(wave * 16 + r) * 64 + lane];
            if constexpr (PROJ) accp[r] += xch[((4 + wave) * 16 + r) * 64 + lane];
        }
    }
    if (pme >= g.P) return;
    QOut qo;
    if constexpr (OUT == 1) qo = qout_parm(e.qs, e.qz, e.qkind);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int mb = 32 * wm + 8 * q + 4 * half;
        uint32_t word = 0;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int ml = mb + r;
            float v = (float)((double)(acc[4 * q + r] - s_corr[ml]) * s_cm[ml]);
            if (has_bias) v = v + s_bias[ml];
            if (e.relu) v = v > 0.0f ? v : 0.0f;
            if constexpr (PROJ) v = v + (float)((double)(accp[4 * q + r] - s_corrp[ml]) * s_cp[ml]);
            if (has_skip) v = v + sk[4 * q + r];
            if constexpr (OUT == 0) ((float*)Y)[yb + (size_t)(8 * q + 4 * half + r) * g.OHW] = v;
            else word |= qout_byte(v, qo) << (8 * r);
        }
        if constexpr (OUT == 1) *reinterpret_cast<uint32_t*>((int8_t*)Y + (size_t)pme * g.M + m0 + mb) = word;
    }
}

template <bool PROJ>
void launch_qconv_lds(int out, const int8_t* x, const int8_t* wk, const int8_t* pk, void* y, const QGeom& g,
                      const QEpi& e, hipStream_t s) {
    const int tiles = ((g.P + 63) / 64) * (g.M / 64);
    const dim3 grid((unsigned)tiles);
    // a grid of at most two blocks per CU: two k groups per block (each tile's
    // chain of stages halves; its blocks still fit on the CUs at once)
    if (tiles <= 2 * num_cus()) {
        if (out == 0) hipLaunchKernelGGL((k_qconv_lds<PROJ, 0, 2>), grid, dim3(512), 0, s, x, wk, pk, y, g, e);
        else hipLaunchKernelGGL((k_qconv_lds<PROJ, 1, 2>), grid, dim3(512), 0, s, x, wk, pk, y, g, e);
        return;
    }
    if (out == 0) hipLaunchKernelGGL((k_qconv_lds<PROJ, 0, 1>), grid, dim3(256), 0, s, x, wk, pk, y, g, e);
    else hipLaunchKernelGGL((k_qconv_lds<PROJ, 1, 1>), grid, dim3(256), 0, s, x, wk, pk, y, g, e);
}

template <int KS, bool PROJ>
void launch_qconv(int out, const int8_t* x, const int8_t* wk, const int8_t* pk, void* y, const QGeom& g, const QEpi& e,
                  uint32_t xb, uint32_t wb, uint32_t pb, hipStream_t s) {
    const dim3 grid((unsigned)((g.P + (KS == 1 ? 255 : 63)) / (KS == 1 ? 256 : 64)), (unsigned)(g.M / 64));
    if (out == 0)
        hipLaunchKernelGGL((k_qconv<KS, PROJ, 0>), grid, dim3(256), 0, s, x, wk, pk, y, g, e, xb, wb, pb);
    else
        hipLaunchKernelGGL((k_qconv<KS, PROJ, 1>), grid, dim3(256), 0, s, x, wk, pk, y, g, e, xb, wb, pb);
}

bool dev_tensor(const Tensor* t, const char* name, const char* what) {
    if (!tensor_sane(t, name)) return false;
    if (!is_dev(classify(t->data))) {
        set_error("%s: %s must be a device tensor", name, what);
        return false;
    }
    return true;
}

bool one_code(const Tensor* z, int kind, const char* name, const char* what) {
    if (!z || !z->data) return true;
    if (!dev_tensor(z, name, what)) return false;
    if (z->size != 1 || (int)z->dtype != (kind == 2 ? kI8 : kU8)) {
        set_error("%s: %s must be one element of the code dtype", name, what);
        return false;
    }
    return true;
}

}  // namespace
}  // namespace tohip

using namespace tohip;

extern "C" void quantize_linear_nhwc_forward(const Tensor* X, const Tensor* Scale, const Tensor* ZeroPoint,
                                             int code_dtype, Tensor* Y) {
    const char* name = "quantize_linear_nhwc_forward";
    tensor_ops_hip_clear_error();
    if (!ensure_device()) return;
    if (!dev_tensor(X, name, "X") || !dev_tensor(Scale, name, "Scale") || !dev_tensor(Y, name, "Y")) return;
    const int kind = code_dtype == kU8 ? 1 : (code_dtype == kI8 ? 2 : 0);
    if (!kind) { set_error("%s: code_dtype must be uint8 or int8", name); return; }
    if (!one_code(ZeroPoint, kind, name, "ZeroPoint")) return;
    if ((int)X->dtype != kF32 || X->ndim != 4 || (int)Scale->dtype != kF32 || Scale->size != 1) {
        set_error("%s: X must be 4-D float32 and Scale one float32", name);
        return;
    }
    const int N = X->shape[0], C = X->shape[1], H = X->shape[2], W = X->shape[3];
    if ((int)Y->dtype != kI8 || Y->ndim != 4 || Y->shape[0] != N || Y->shape[1] != H || Y->shape[2] != W ||
        Y->shape[3] != C) {
        set_error("%s: Y must be int8 [N, H, W, C]", name);
        return;
    }
    if (C % 32) { set_error("%s: C must be a multiple of 32, got %d", name, C); return; }
    if (X->size == 0) return;
    const int HW = H * W;
    const dim3 grid((unsigned)((HW + 63) / 64), (unsigned)(C / 32), (unsigned)N);
    const void* zp = (ZeroPoint && ZeroPoint->data) ? ZeroPoint->data : nullptr;
    if (HW % 4 == 0 && C % 64 == 0 && ((uintptr_t)X->data & 15) == 0)
        hipLaunchKernelGGL(k_quant_nhwc64, dim3((unsigned)((HW + 63) / 64), (unsigned)(C / 64), (unsigned)N),
                           dim3(256), 0, stream(), (const float*)X->data, (int8_t*)Y->data,
                           (const float*)Scale->data, zp, kind, C, HW);
    else if (HW % 4 == 0 && ((uintptr_t)X->data & 15) == 0)
        hipLaunchKernelGGL((k_quant_nhwc<true>), grid, dim3(256), 0, stream(), (const float*)X->data,
                           (int8_t*)Y->data, (const float*)Scale->data, zp, kind, C, HW);
    else
        hipLaunchKernelGGL((k_quant_nhwc<false>), grid, dim3(256), 0, stream(), (const float*)X->data,
                           (int8_t*)Y->data, (const float*)Scale->data, zp, kind, C, HW);
    check_launch(name);
}

extern "C" void max_pool_quantize_nhwc_forward(const Tensor* X, Tensor* Y, PoolParams* params, const Tensor* Scale,
                                               const Tensor* ZeroPoint, int code_dtype, Tensor* Yc) {
    const char* name = "max_pool_quantize_nhwc_forward";
    tensor_ops_hip_clear_error();
    if (!ensure_device()) return;
    if (!dev_tensor(X, name, "X") || !dev_tensor(Y, name, "Y") || !dev_tensor(Scale, name, "Scale") ||
        !dev_tensor(Yc, name, "Yc"))
        return;
    if (!params || !params->pads || !params->strides || !params->dilations || !params->kernel_shape) {
        set_error("%s: NULL params", name);
        return;
    }
    const int kind = code_dtype == kU8 ? 1 : (code_dtype == kI8 ? 2 : 0);
    if (!kind) { set_error("%s: code_dtype must be uint8 or int8", name); return; }
    if (!one_code(ZeroPoint, kind, name, "ZeroPoint")) return;
    if ((int)X->dtype != kF32 || X->ndim != 4 || (int)Y->dtype != kF32 || Y->ndim != 4 || (int)Scale->dtype != kF32 ||
        Scale->size != 1) {
        set_error("%s: X and Y must be 4-D float32 and Scale one float32", name);
        return;
    }
    const int N = X->shape[0], C = X->shape[1], H = X->shape[2], W = X->shape[3], OH = Y->shape[2], OW = Y->shape[3];
    if (Y->shape[0] != N || Y->shape[1] != C) { set_error("%s: Y batch/channels differ from X", name); return; }
    if ((int)Yc->dtype != kI8 || Yc->ndim != 4 || Yc->shape[0] != N || Yc->shape[1] != OH || Yc->shape[2] != OW ||
        Yc->shape[3] != C) {
        set_error("%s: Yc must be int8 [N, OH, OW, C]", name);
        return;
    }
    const int* k = params->kernel_shape;
    const bool fits = k[0] == 3 && k[1] == 3 && params->strides[0] == 2 && params->strides[1] == 2 &&
                      params->dilations[0] == 1 && params->dilations[1] == 1 && params->pads[0] == 1 &&
                      params->pads[1] == 1 && W == 2 * OW && OW <= 64 && OH >= 1 && 2 * OH <= H + 2 && C % 16 == 0 &&
                      ((uintptr_t)X->data & 7) == 0 && (size_t)16 * H * W * 4 < ((size_t)1 << 31) && N <= 65535;
    if (!fits) {
        // the two calls it stands for
        max_pool_forward(X, Y, params);
        if (tensor_ops_hip_last_error()[0]) return;
        quantize_linear_nhwc_forward(Y, Scale, ZeroPoint, code_dtype, Yc);
        return;
    }
    if (X->size == 0) return;
    const int strips = (OH + kMPRows - 1) / kMPRows, blocks = strips * (C / 16);
    const void* zp = (ZeroPoint && ZeroPoint->data) ? ZeroPoint->data : nullptr;
    hipLaunchKernelGGL(k_maxpool_q16, dim3((unsigned)blocks, (unsigned)N), dim3(1024), 0, stream(),
                       (const float*)X->data, (float*)Y->data, (int8_t*)Yc->data, (const float*)Scale->data, zp, kind,
                       C, H, W, OH, OW, strips);
    check_launch(name);
}

extern "C" void qconv_pack_weights(const Tensor* Wq, Tensor* Wk, Tensor* WSum) {
    const char* name = "qconv_pack_weights";
    tensor_ops_hip_clear_error();
    if (!ensure_device()) return;
    if (!dev_tensor(Wq, name, "Wq") || !dev_tensor(Wk, name, "Wk") || !dev_tensor(WSum, name, "WSum")) return;
    if ((int)Wq->dtype != kI8 || Wq->ndim != 4) { set_error("%s: Wq must be int8 [M, C, KH, KW]", name); return; }
    const int M = Wq->shape[0], C = Wq->shape[1], KH = Wq->shape[2], KW = Wq->shape[3];
    if ((int)Wk->dtype != kI8 || Wk->ndim != 4 || Wk->shape[0] != M || Wk->shape[1] != KH || Wk->shape[2] != KW ||
        Wk->shape[3] != C) {
        set_error("%s: Wk must be int8 [M, KH, KW, C]", name);
        return;
    }
    if ((int)WSum->dtype != kI32 || WSum->size != (size_t)M * KH * KW) {
        set_error("%s: WSum must be int32 [M, KH * KW]", name);
        return;
    }
    if (Wq->size == 0) return;
    hipLaunchKernelGGL(k_qconv_pack, dim3((unsigned)M), dim3(256), 0, stream(), (const int8_t*)Wq->data,
                       (int8_t*)Wk->data, (int*)WSum->data, C, KH * KW);
    check_launch(name);
}

extern "C" void qconv_block_forward(const Tensor* X, const QConvBlock* blk, Tensor* Y, ConvParams* params) {
    const char* name = "qconv_block_forward";
    tensor_ops_hip_clear_error();
    if (!blk || !params || !params->pads || !params->strides || !params->dilations) {
        set_error("%s: NULL block or params", name);
        return;
    }
    if (exact_mode()) {
        set_error("%s: the int8 block has no exact mode (run the operator sequence instead)", name);
        return;
    }
    if (!ensure_device()) return;
    const QConvBlock& b = *blk;
    const int xkind = b.x_codes == kU8 ? 1 : (b.x_codes == kI8 ? 2 : 0);
    if (!xkind) { set_error("%s: x_codes must be uint8 or int8", name); return; }
    if (!dev_tensor(X, name, "X") || !dev_tensor(Y, name, "Y") || !dev_tensor(b.x_scale, name, "x_scale") ||
        !dev_tensor(b.w, name, "w") || !dev_tensor(b.w_sum, name, "w_sum") || !dev_tensor(b.w_scale, name, "w_scale"))
        return;
    if (!one_code(b.x_zero, xkind, name, "x_zero")) return;
    if ((int)X->dtype != kI8 || X->ndim != 4 || (int)b.w->dtype != kI8 || b.w->ndim != 4) {
        set_error("%s: X must be int8 [N, H, W, C] and w int8 [M, KH, KW, C]", name);
        return;
    }
    QGeom g;
    g.N = X->shape[0]; g.H = X->shape[1]; g.W = X->shape[2]; g.C = X->shape[3];
    g.M = b.w->shape[0]; g.KH = b.w->shape[1]; g.KW = b.w->shape[2];
    if (b.w->shape[3] != g.C) { set_error("%s: w has %d input channels, X %d", name, b.w->shape[3], g.C); return; }
    if (params->group != 1) { set_error("%s: group must be 1", name); return; }
    g.pt = params->pads[0]; g.pl = params->pads[1];
    g.sh = params->strides[0]; g.sw = params->strides[1];
    g.dh = params->dilations[0]; g.dw = params->dilations[1];
    if (g.sh < 1 || g.sw < 1 || g.dh < 1 || g.dw < 1 || g.pt < 0 || g.pl < 0) {
        set_error("%s: bad strides / dilations / pads", name);
        return;
    }
    g.OH = (g.H + g.pt + params->pads[2] - g.dh * (g.KH - 1) - 1) / g.sh + 1;
    g.OW = (g.W + g.pl + params->pads[3] - g.dw * (g.KW - 1) - 1) / g.sw + 1;
    if (g.C % 32 || g.M % 64 || g.OH < 1 || g.OW < 1) {
        set_error("%s: needs C %% 32 == 0 and M %% 64 == 0 (C %d, M %d) and a non-empty output", name, g.C, g.M);
        return;
    }
    if ((int)b.w_sum->dtype != kI32 || b.w_sum->size != (size_t)g.M * g.KH * g.KW || (int)b.w_scale->dtype != kF32 ||
        b.w_scale->size != (size_t)g.M || (int)b.x_scale->dtype != kF32 || b.x_scale->size != 1) {
        set_error("%s: w_sum int32 [M, KH * KW], w_scale float32 [M] and x_scale one float32 expected", name);
        return;
    }
    const bool has_b = b.bias && b.bias->data;
    if (has_b && (!dev_tensor(b.bias, name, "bias") || (int)b.bias->dtype != kF32 || b.bias->size != (size_t)g.M)) {
        if (!tensor_ops_hip_last_error()[0]) set_error("%s: bias must be float32 [M]", name);
        return;
    }
    const bool proj = b.p && b.p->data;
    if (proj) {
        if (!dev_tensor(b.p, name, "p") || !dev_tensor(b.p_sum, name, "p_sum") || !dev_tensor(b.p_scale, name, "p_scale"))
            return;
        if ((int)b.p->dtype != kI8 || b.p->size != (size_t)g.M * g.C || (int)b.p_sum->dtype != kI32 ||
            b.p_sum->size != (size_t)g.M || (int)b.p_scale->dtype != kF32 || b.p_scale->size != (size_t)g.M) {
            set_error("%s: projection needs p int8 [M, C], p_sum int32 [M], p_scale float32 [M]", name);
            return;
        }
        // the 1x1 / pads-0 projection with the same strides must give the same grid
        if ((g.H - 1) / g.sh + 1 != g.OH || (g.W - 1) / g.sw + 1 != g.OW || g.pt >= g.H || g.pl >= g.W) {
            set_error("%s: the projection's output grid differs from the convolution's", name);
            return;
        }
    }
    const bool has_skip = b.skip && b.skip->data;
    if (has_skip && (!dev_tensor(b.skip, name, "skip") || (int)b.skip->dtype != kF32 ||
                     b.skip->size != (size_t)g.N * g.M * g.OH * g.OW)) {
        if (!tensor_ops_hip_last_error()[0]) set_error("%s: skip must be float32 [N, M, OH, OW]", name);
        return;
    }
    const bool codes_out = b.q_scale && b.q_scale->data;
    int qkind = 0;
    if (codes_out) {
        qkind = b.y_codes == kU8 ? 1 : (b.y_codes == kI8 ? 2 : 0);
        if (!qkind) { set_error("%s: y_codes must be uint8 or int8", name); return; }
        if (!dev_tensor(b.q_scale, name, "q_scale") || !one_code(b.q_zero, qkind, name, "q_zero")) return;
        if ((int)b.q_scale->dtype != kF32 || b.q_scale->size != 1) { set_error("%s: q_scale must be one float32", name); return; }
        if ((int)Y->dtype != kI8 || Y->ndim != 4 || Y->shape[0] != g.N || Y->shape[1] != g.OH || Y->shape[2] != g.OW ||
            Y->shape[3] != g.M) {
            set_error("%s: Y must be int8 [N, OH, OW, M] for code output", name);
            return;
        }
    } else if ((int)Y->dtype != kF32 || Y->ndim != 4 || Y->shape[0] != g.N || Y->shape[1] != g.M || Y->shape[2] != g.OH ||
               Y->shape[3] != g.OW) {
        set_error("%s: Y must be float32 [N, M, OH, OW]", name);
        return;
    }
    const int64_t P = (int64_t)g.N * g.OH * g.OW;
    const int64_t xb = (int64_t)X->size, wb = (int64_t)b.w->size;
    const int64_t yb = P * g.M * (codes_out ? 1 : 4);
    if (xb >= ((int64_t)1 << 31) || wb >= ((int64_t)1 << 31) || yb >= ((int64_t)1 << 31)) {
        set_error("%s: operands beyond 2 GB", name);
        return;
    }
    g.P = (int)P;
    g.OHW = g.OH * g.OW;
    g.csteps = g.C / 32;
    g.steps = g.KH * g.KW * g.csteps;
    g.psteps = proj ? g.csteps : 0;
    g.fd_ohw = make_fastdiv((uint32_t)g.OHW);
    g.fd_ow = make_fastdiv((uint32_t)g.OW);
    g.fd_cs = make_fastdiv((uint32_t)g.csteps);
    g.fd_kw = make_fastdiv((uint32_t)g.KW);
    QEpi e;
    e.xs = (const float*)b.x_scale->data;
    e.xz = (b.x_zero && b.x_zero->data) ? b.x_zero->data : nullptr;
    e.xkind = xkind;
    e.wsum = (const int*)b.w_sum->data;
    e.ws = (const float*)b.w_scale->data;
    e.bias = has_b ? (const float*)b.bias->data : nullptr;
    e.psum = proj ? (const int*)b.p_sum->data : nullptr;
    e.ps = proj ? (const float*)b.p_scale->data : nullptr;
    e.skip = has_skip ? (const float*)b.skip->data : nullptr;
    e.relu = b.relu ? 1 : 0;
    e.qs = codes_out ? (const float*)b.q_scale->data : nullptr;
    e.qz = (codes_out && b.q_zero && b.q_zero->data) ? b.q_zero->data : nullptr;
    e.qkind = qkind;
    if (P == 0) return;
    // one wave per 64x64 tile when there are at least 8 tiles per CU, else the
    // 4 waves of a block split one tile's k steps
    const int64_t tiles = ((P + 63) / 64) * (g.M / 64);
    const bool split = tiles < 8 * (int64_t)num_cus();
    const int8_t* x = (const int8_t*)X->data;
    const int8_t* wk = (const int8_t*)b.w->data;
    const int8_t* pk = proj ? (const int8_t*)b.p->data : nullptr;
    const uint32_t pb = proj ? (uint32_t)b.p->size : 0u;
    const int out = codes_out ? 1 : 0;
    hipStream_t s = stream();
    if (g.C % 64 == 0) {
        if (proj) launch_qconv_lds<true>(out, x, wk, pk, Y->data, g, e, s);
        else launch_qconv_lds<false>(out, x, wk, pk, Y->data, g, e, s);
    } else if (split) {
        if (proj) launch_qconv<4, true>(out, x, wk, pk, Y->data, g, e, (uint32_t)xb, (uint32_t)wb, pb, s);
        else launch_qconv<4, false>(out, x, wk, pk, Y->data, g, e, (uint32_t)xb, (uint32_t)wb, pb, s);
    } else {
        if (proj) launch_qconv<1, true>(out, x, wk, pk, Y->data, g, e, (uint32_t)xb, (uint32_t)wb, pb, s);
        else launch_qconv<1, false>(out, x, wk, pk, Y->data, g, e, (uint32_t)xb, (uint32_t)wb, pb, s);
    }
    check_launch(name);
}
