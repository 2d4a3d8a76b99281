// gemm.hip — Gemm (Y = alpha * A' B' + beta * C) for gfx950.
//
// tensor_ops/tensor_ops.c:1167-1228 accumulates sum_k A'[m,k] B'[k,n] in
// double, sequentially in k, then adds beta * C with the reference's bias
// broadcast rules and writes through the output encoder.  Three kernels:
//
//  * k_gemm_mfma_f32 — v_mfma_f32_32x32x2f32 (fp32 operands, fp32 accumulate),
//    for the layouts and dtypes k_gemm_f32_nt does not take.
//    Operands of any dtype exactly representable in fp32 (f32, f16, bf16,
//    fp8, int4/8/16, uint8) are decoded while staging into LDS.
//    128x128 block tile, 4 waves (2x2), each wave 64x64 = 2x2 MFMA tiles,
//    BK = 16, LDS double buffer.  Tolerance class vs the reference.
//  * k_gemm_f16_nt — f16 x f16 with A [M, K] and B [N, K] (transB = 1):
//    v_mfma_f32_32x32x16_f16, 256x256x64 block tiles over 16 waves (64x64
//    each), operands through raw buffer loads into registers one k-tile
//    ahead, LDS double buffer, XCD-aware tile order.  fp32 accumulate.
//  * k_gemm_f32_nt — f32 A [M, K] with B [N, K] of f32 or int8 / uint8 codes
//    (dequantised while staging): v_mfma_f32_32x32x2f32, 128x256x16 tiles over
//    8 waves, split-K with a deterministic reduction for small grids.
//  * k_gemm_mfma_f16 — the other f16 transposes: 128x128x32 tiles.
//  * k_gemm_exact — fp64, sequential k, no contraction: bit-identical to the
//    reference for every dtype combination.  Used for f64 / int32 / int64
//    operands and when exact mode is on.
// The epilogue is shared: alpha * acc + beta * bias in double, then st_d.
#include <algorithm>

#include "runtime.h"

namespace tohip {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((__vector_size__(16)));
typedef __attribute__((address_space(1))) float gfloat;
typedef __attribute__((address_space(1))) uint16_t gu16;

__device__ __forceinline__ u32x4 ld_buf_b128(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
}
// Zero the halves of an 8-half chunk starting at k whose index is >= K.
__device__ __forceinline__ u32x4 mask_k8(u32x4 v, int k, int K) {
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t lo = (k + 2 * w < K) ? 0x0000FFFFu : 0u, hi = (k + 2 * w + 1 < K) ? 0xFFFF0000u : 0u;
        v[w] &= lo | hi;
    }
    return v;
}

struct Bias {
    const void* p;
    int dt;
    int mode;   // 0 none, 1 scalar, 2 per column (n), 3 per row (m), 4 two-d (H, W broadcast),
                // 5 present but matching neither N nor M: beta * 0.0 is still added
    int H, W;
};

__device__ __forceinline__ double bias_at(const Bias& c, int m, int n) {
    switch (c.mode) {
    case 1: return ld_d_rt(c.dt, c.p, 0);
    case 2: return ld_d_rt(c.dt, c.p, n);
    case 3: return ld_d_rt(c.dt, c.p, m);
    case 4: {
        const int r = c.H == 1 ? 0 : m, q = c.W == 1 ? 0 : n;
        return (r < c.H && q < c.W) ? ld_d_rt(c.dt, c.p, (int64_t)r * c.W + q) : 0.0;
    }
    default: return 0.0;
    }
}

struct GemmArgs {
    const void* A;
    const void* B;
    void* Y;
    int M, N, K;
    int lda, ldb;   // row lengths of A and B as stored (A->shape[1], B->shape[1])
    double alpha, beta;
    Bias c;
    int dty;
};

// Any output dtype / bias dtype: kept out of line so the unrolled MFMA
// epilogues stay small.  It takes scalars, not the argument struct: a
// reference to the kernel's by-value argument would move it to scratch memory
// and make every field a per-lane (divergent) load in the main loop.
__device__ __noinline__ void store_rt_s(void* Y, int dty, int N, double alpha, double beta, const void* cp, int cdt,
                                        int cmode, int cH, int cW, int m, int n, double acc) {
    double r = alpha * acc;
    if (cmode) r += beta * bias_at(Bias{cp, cdt, cmode, cH, cW}, m, n);
    st_d_rt(dty, Y, (int64_t)m * N + n, r);
}
__device__ __forceinline__ void store_rt(const GemmArgs& g, int m, int n, double acc) {
    store_rt_s(g.Y, g.dty, g.N, g.alpha, g.beta, g.c.p, g.c.dt, g.c.mode, g.c.H, g.c.W, m, n, acc);
}

// YDT >= 0: output dtype known at compile time; f32 bias (scalar / per
// column / per row) is handled inline, anything else goes through store_rt.
template <int YDT>
__device__ __forceinline__ void epilogue_store(const GemmArgs& g, int m, int n, double acc) {
    if (m >= g.M || n >= g.N) return;
    if constexpr (YDT >= 0) {
        if (g.c.mode == 0 || (g.c.dt == kF32 && g.c.mode <= 3)) {
            double r = g.alpha * acc;
            if (g.c.mode) {
                const float* c = (const float*)g.c.p;
                r += g.beta * (double)c[g.c.mode == 1 ? 0 : (g.c.mode == 2 ? n : m)];
            }
            st_d<YDT>(g.Y, (int64_t)m * g.N + n, r);
            return;
        }
    }
    store_rt(g, m, n, acc);
}

// ------------------------------------------------------------------- exact ---
constexpr int kET = 16;

__global__ __launch_bounds__(kET * kET) void k_gemm_exact(GemmArgs g, int dta, int dtb, int ta, int tb) {
    __shared__ double As[kET][kET + 1];
    __shared__ double Bs[kET][kET + 1];
    const int tx = threadIdx.x % kET, ty = threadIdx.x / kET;
    const int m = blockIdx.y * kET + ty, n = blockIdx.x * kET + tx;
    double acc = 0.0;
    for (int k0 = 0; k0 < g.K; k0 += kET) {
        {
            const int mm = blockIdx.y * kET + ty, kk = k0 + tx;
            double v = 0.0;
            if (mm < g.M && kk < g.K)
                v = ld_d_rt(dta, g.A, ta ? (int64_t)kk * g.lda + mm : (int64_t)mm * g.lda + kk);
            As[ty][tx] = v;
            const int nn = blockIdx.x * kET + tx, kb = k0 + ty;
            double w = 0.0;
            if (nn < g.N && kb < g.K)
                w = ld_d_rt(dtb, g.B, tb ? (int64_t)nn * g.ldb + kb : (int64_t)kb * g.ldb + nn);
            Bs[ty][tx] = w;
        }
        __syncthreads();
        const int kend = min(kET, g.K - k0);
        for (int kk = 0; kk < kend; kk++) acc += As[ty][kk] * Bs[kk][tx];
        __syncthreads();
    }
    epilogue_store<-1>(g, m, n, acc);
}

// ------------------------------------------------------------------- f32 MFMA ---
constexpr int kBM = 128, kBN = 128, kBK = 16, kThreads = 256;
constexpr int kPad = 4;

// DT >= 0: compile-time dtype; DT < 0: decode with the run-time dtype rdt.
template <int DT> __device__ __forceinline__ float ldf(const void* p, int64_t i, int rdt) {
    if constexpr (DT == kF32) return ((const float*)p)[i];
    else if constexpr (DT >= 0) return (float)ld_d<DT>(p, i);
    else return (float)ld_d_rt(rdt, p, i);
}

// Stage a BK x 128 slice of an operand into LDS laid out [k][row] (row = m or n).
// KMAJOR: operand stored with k contiguous (A with transA=0, B with transB=1).
template <int DT, bool KMAJOR>
__device__ __forceinline__ void stage_f32(float (*dst)[kBM + kPad], const void* src, int ld, int rows, int K,
                                          int row0, int k0, int rdt) {
    const int t = threadIdx.x;
    if constexpr (KMAJOR) {
        // 128 rows x 16 k: thread handles 8 consecutive k of one row (2 threads per row).
        const int r = t >> 1, kq = (t & 1) * 8;
        const int gr = row0 + r;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int gk = k0 + kq + e;
            dst[kq + e][r] = (gr < rows && gk < K) ? ldf<DT>(src, (int64_t)gr * ld + gk, rdt) : 0.0f;
        }
    } else {
        // 16 k x 128 rows, rows contiguous: thread handles 8 consecutive rows of one k.
        const int kk = t >> 4, rq = (t & 15) * 8;
        const int gk = k0 + kk;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int gr = row0 + rq + e;
            dst[kk][rq + e] = (gr < rows && gk < K) ? ldf<DT>(src, (int64_t)gk * ld + gr, rdt) : 0.0f;
        }
    }
}

// Vectorised staging for f32 operands when the leading dimension allows
// 16-byte loads (ld % 4 == 0, base 16-byte aligned).
template <bool KMAJOR>
__device__ __forceinline__ void stage_f32_vec(float (*dst)[kBM + kPad], const float* src, int ld, int rows, int K,
                                              int row0, int k0) {
    const int t = threadIdx.x;
    if constexpr (KMAJOR) {
        const int r = t >> 1, kq = (t & 1) * 8;
        const int gr = row0 + r;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int gk = k0 + kq + 4 * h;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (gr < rows) {
                if (gk + 3 < K) v = *reinterpret_cast<const float4*>(src + (int64_t)gr * ld + gk);
                else {
                    const float* p = src + (int64_t)gr * ld;
                    v.x = gk < K ? p[gk] : 0.f;
                    v.y = gk + 1 < K ? p[gk + 1] : 0.f;
                    v.z = gk + 2 < K ? p[gk + 2] : 0.f;
                }
            }
            dst[kq + 4 * h][r] = v.x;
            dst[kq + 4 * h + 1][r] = v.y;
            dst[kq + 4 * h + 2][r] = v.z;
            dst[kq + 4 * h + 3][r] = v.w;
        }
    } else {
        const int kk = t >> 4, rq = (t & 15) * 8;
        const int gk = k0 + kk;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int gr = row0 + rq + 4 * h;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (gk < K) {
                const float* p = src + (int64_t)gk * ld;
                if (gr + 3 < rows) v = *reinterpret_cast<const float4*>(p + gr);
                else {
                    v.x = gr < rows ? p[gr] : 0.f;
                    v.y = gr + 1 < rows ? p[gr + 1] : 0.f;
                    v.z = gr + 2 < rows ? p[gr + 2] : 0.f;
                }
            }
            *reinterpret_cast<float4*>(&dst[kk][rq + 4 * h]) = v;
        }
    }
}

// DA / DB: kF32, or -1 for operands decoded with the run-time dtypes dta / dtb.
template <int DA, int DB, bool TA, bool TB, bool VEC, int YDT>
__global__ __launch_bounds__(kThreads) void k_gemm_mfma_f32(GemmArgs g, int dta, int dtb) {
    __shared__ float As[2][kBK][kBM + kPad];
    __shared__ float Bs[2][kBK][kBN + kPad];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    auto stage = [&](int buf, int k0) {
        if constexpr (VEC && DA == kF32) stage_f32_vec<!TA>(As[buf], (const float*)g.A, g.lda, g.M, g.K, m0, k0);
        else stage_f32<DA, !TA>(As[buf], g.A, g.lda, g.M, g.K, m0, k0, dta);
        if constexpr (VEC && DB == kF32) stage_f32_vec<TB>(Bs[buf], (const float*)g.B, g.ldb, g.N, g.K, n0, k0);
        else stage_f32<DB, TB>(Bs[buf], g.B, g.ldb, g.N, g.K, n0, k0, dtb);
    };

    const int nk = (g.K + kBK - 1) / kBK;
    stage(0, 0);
    __syncthreads();
    const int lr = lane & 31, lk = lane >> 5;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) stage(cur ^ 1, (kt + 1) * kBK);
#pragma unroll
        for (int ks = 0; ks < kBK; ks += 2) {
            float a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; i++) a[i] = As[cur][ks + lk][wm * 64 + i * 32 + lr];
#pragma unroll
            for (int j = 0; j < 2; j++) b[j] = Bs[cur][ks + lk][wn * 64 + j * 32 + lr];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
    // D[m][n]: n = lane % 32, m = 8 * (r / 4) + 4 * (lane / 32) + r % 4 within the 32x32 tile.
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
                const int n = n0 + wn * 64 + j * 32 + lr;
                epilogue_store<YDT>(g, m, n, (double)acc[i][j][r]);
            }
}

// ------------------------------------------------------------------- f16 MFMA ---
constexpr int kHBK = 32, kHPad = 8;   // row stride 40 halves = 80 bytes

// Stage a 128-row x 32-k slice of an f16 operand into LDS laid out [row][k].
template <bool KMAJOR>
__device__ __forceinline__ void stage_f16(_Float16 (*dst)[kHBK + kHPad], const uint16_t* src, int ld, int rows, int K,
                                          int row0, int k0, bool vec) {
    const int t = threadIdx.x;
    if constexpr (KMAJOR) {
        // 128 rows x 32 k = 512 chunks of 8 halves; 2 chunks per thread.
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int c = t + h * kThreads;
            const int r = c >> 2, kq = (c & 3) * 8;
            const int gr = row0 + r, gk = k0 + kq;
            halfx8 v;
            if (vec && gr < rows && gk + 7 < K) {
                v = *reinterpret_cast<const halfx8*>(src + (int64_t)gr * ld + gk);
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    v[e] = (gr < rows && gk + e < K) ? __builtin_bit_cast(_Float16, src[(int64_t)gr * ld + gk + e])
                                                      : (_Float16)0.0f;
            }
            *reinterpret_cast<halfx8*>(&dst[r][kq]) = v;
        }
    } else {
        // stored [k][row]: 32 k x 128 rows, thread reads 8 consecutive rows of 2 k values.
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int c = t + h * kThreads;
            const int kk = c >> 4, rq = (c & 15) * 8;
            const int gk = k0 + kk;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int gr = row0 + rq + e;
                dst[rq + e][kk] = (gr < rows && gk < K) ? __builtin_bit_cast(_Float16, src[(int64_t)gk * ld + gr])
                                                         : (_Float16)0.0f;
            }
        }
    }
}

template <bool TA, bool TB, int YDT>
__global__ __launch_bounds__(kThreads) void k_gemm_mfma_f16(GemmArgs g, int vec) {
    __shared__ _Float16 As[2][kBM][kHBK + kHPad];
    __shared__ _Float16 Bs[2][kBN][kHBK + kHPad];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    const uint16_t* A = (const uint16_t*)g.A;
    const uint16_t* B = (const uint16_t*)g.B;
    auto stage = [&](int buf, int k0) {
        stage_f16<!TA>(As[buf], A, g.lda, g.M, g.K, m0, k0, vec != 0);
        stage_f16<TB>(Bs[buf], B, g.ldb, g.N, g.K, n0, k0, vec != 0);
    };
    const int nk = (g.K + kHBK - 1) / kHBK;
    stage(0, 0);
    __syncthreads();
    const int lr = lane & 31, lk = (lane >> 5) * 8;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) stage(cur ^ 1, (kt + 1) * kHBK);
#pragma unroll
        for (int ks = 0; ks < kHBK; ks += 16) {
            halfx8 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; i++) a[i] = *reinterpret_cast<const halfx8*>(&As[cur][wm * 64 + i * 32 + lr][ks + lk]);
#pragma unroll
            for (int j = 0; j < 2; j++) b[j] = *reinterpret_cast<const halfx8*>(&Bs[cur][wn * 64 + j * 32 + lr][ks + lk]);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + (lk >> 1) + (r & 3);
                const int n = n0 + wn * 64 + j * 32 + lr;
                epilogue_store<YDT>(g, m, n, (double)acc[i][j][r]);
            }
}

// ------------------------------------------------ f16 MFMA, both operands K-major ---
// A [M, K] and B [N, K] row-major (transA = 0, transB = 1: the layout of the
// ONNX Gemm with transB = 1).  Block tile BM x BN x BK over NT = 64 * WGM * WGN
// threads; wave tile (BM / WGM) x (BN / WGN) of 32x32 MFMA tiles.
// Pipeline per k-tile (below): the next tile's registers go to the other LDS
// buffer, the tile after it is requested, the MFMAs of tile k run from LDS,
// one barrier.  LDS rows are BK + 8 halves (16 bytes of padding), so
// the 16-byte fragment reads of 8 consecutive rows cover all banks once.
// Tile order: consecutive workgroups are spread over the 8 XCDs by the
// dispatcher, so the block index is remapped to give each XCD a contiguous
// run of tiles, and tiles are walked in groups of kGroupM tile rows, so one
// XCD's L2 serves a few A panels and B panels.
constexpr int kGroupM = 4;

__device__ __forceinline__ void tile_of_block(int nbm, int nbn, int& tm, int& tn) {
    const int nb = nbm * nbn;
    int bid = blockIdx.x;
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    const int per_group = kGroupM * nbn;
    const int first_m = (bid / per_group) * kGroupM;
    const int gsz = min(nbm - first_m, kGroupM);
    const int r = bid % per_group;
    tm = first_m + r % gsz;
    tn = r / gsz;
}

// Epilogue of the tiled kernels.  YDT = kF16 / kF32 with no bias or an f32
// bias (scalar, per column, per row) is fully inline and call-free: a call
// would force the accumulators, live across it, into scratch memory.  Every
// other case (YDT = -1) goes through the out-of-line store_rt.  Output goes
// through a global-address-space pointer (a generic pointer compiles to flat
// stores, which also count against the LDS wait counter).
template <int YDT>
__device__ __forceinline__ void epilogue_fast(const GemmArgs& g, int m, int n, double acc) {
    if constexpr (YDT == kF16 || YDT == kF32) {
        double r = g.alpha * acc;
        if (g.c.mode) {
            const gfloat* c = (const gfloat*)g.c.p;
            r += g.beta * (double)c[g.c.mode == 1 ? 0 : (g.c.mode == 2 ? n : m)];
        }
        const int64_t i = (int64_t)m * g.N + n;
        if constexpr (YDT == kF16) ((gu16*)g.Y)[i] = enc_f16((float)r);
        else ((gfloat*)g.Y)[i] = (float)r;
    } else {
        store_rt(g, m, n, acc);
    }
}

// The 16 accumulators a lane holds for one 32x32 MFMA tile: column n, rows
// mb + 8 * (r >> 2) + (r & 3).  Same arithmetic as epilogue_fast, specialised
// on the bias (BIAS 0: none, 1: scalar / per column, loaded and multiplied once
// per column, 3: per row) and on whether the tile lies wholly inside Y (FULL:
// no per-element checks), so the stores need no divergent branches.
// A1: alpha == 1 (1.0 * x is x in double, so skipping the product changes no bit).
template <int YDT, int BIAS, bool FULL, bool A1 = false>
__device__ __forceinline__ void epilogue_col_f(const GemmArgs& g, int mb, int n, const floatx16& a) {
    const gfloat* c = (const gfloat*)g.c.p;
    double cn = 0.0;
    if constexpr (BIAS == 1) cn = g.beta * (double)c[g.c.mode == 1 ? 0 : n];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int m = mb + 8 * (r >> 2) + (r & 3);
        if (!FULL && (m >= g.M || n >= g.N)) continue;
        double v = A1 ? (double)a[r] : g.alpha * (double)a[r];
        if constexpr (BIAS == 1) v += cn;
        if constexpr (BIAS == 3) v += g.beta * (double)c[m];
        const int64_t i = (int64_t)m * g.N + n;
        // nontemporal: Y is written once and not read back here (4096^3 f16:
        // 118.0 -> 116.5 us, same bits)
        if constexpr (YDT == kF16) __builtin_nontemporal_store(enc_f16((float)v), &((gu16*)g.Y)[i]);
        else __builtin_nontemporal_store((float)v, &((gfloat*)g.Y)[i]);
    }
}

template <int YDT, int BIAS>
__device__ __forceinline__ void epilogue_col_b(const GemmArgs& g, bool full, int mb, int n, const floatx16& a) {
    if (full) epilogue_col_f<YDT, BIAS, true>(g, mb, n, a);
    else epilogue_col_f<YDT, BIAS, false>(g, mb, n, a);
}

// mt, nt: the MFMA tile's first row and column (uniform over the wave).
template <int YDT>
__device__ __forceinline__ void epilogue_col(const GemmArgs& g, int mt, int mb, int nt, int n, const floatx16& a) {
    if constexpr (YDT == kF16 || YDT == kF32) {
        const bool full = mt + 32 <= g.M && nt + 32 <= g.N;
        if (g.c.mode == 0) epilogue_col_b<YDT, 0>(g, full, mb, n, a);
        else if (g.c.mode == 3) epilogue_col_b<YDT, 3>(g, full, mb, n, a);
        else epilogue_col_b<YDT, 1>(g, full, mb, n, a);
    } else {
        if (n >= g.N) return;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = mb + 8 * (r >> 2) + (r & 3);
            if (m < g.M) store_rt(g, m, n, (double)a[r]);
        }
    }
}

template <int BM, int BN, int BK, int WGM, int WGN, int YDT, int IGLP = -1>
__global__ __launch_bounds__(64 * WGM * WGN) void k_gemm_f16_nt(GemmArgs g) {
    constexpr int NT = 64 * WGM * WGN;
    constexpr int LDK = BK + 8;
    constexpr int WTM = BM / WGM, WTN = BN / WGN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int CPR = BK / 8;                   // 16-byte chunks per tile row
    constexpr int CA = BM * CPR / NT, CB = BN * CPR / NT;
    static_assert(CA * NT == BM * CPR && CB * NT == BN * CPR, "tile / thread mismatch");
    __shared__ _Float16 lds[2][(BM + BN) * LDK];

    const int nbm = (g.M + BM - 1) / BM, nbn = (g.N + BN - 1) / BN;
    int tm, tn;
    tile_of_block(nbm, nbn, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    // Buffer resources over the operands: rows past M / N read as zero.  The
    // host guarantees (rows + tile) * ld * 2 < 2^31 and ld % 8 == 0.
    const __amdgpu_buffer_rsrc_t ar = buffer_rsrc(g.A, (uint32_t)((int64_t)g.M * g.lda * 2));
    const __amdgpu_buffer_rsrc_t br = buffer_rsrc(g.B, (uint32_t)((int64_t)g.N * g.ldb * 2));

    u32x4 ra[CA], rb[CB];
    auto load_tile = [&](int k0) {
#pragma unroll
        for (int i = 0; i < CA; i++) {
            const int c = t + i * NT;
            ra[i] = ld_buf_b128(ar, (uint32_t)(((m0 + c / CPR) * g.lda + k0 + (c % CPR) * 8) * 2));
        }
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const int c = t + i * NT;
            rb[i] = ld_buf_b128(br, (uint32_t)(((n0 + c / CPR) * g.ldb + k0 + (c % CPR) * 8) * 2));
        }
    };
    // Chunks that straddle K are zeroed here, after the wait for the loads.
    auto mask_tile = [&](int k0) {
#pragma unroll
        for (int i = 0; i < CA; i++) ra[i] = mask_k8(ra[i], k0 + ((t + i * NT) % CPR) * 8, g.K);
#pragma unroll
        for (int i = 0; i < CB; i++) rb[i] = mask_k8(rb[i], k0 + ((t + i * NT) % CPR) * 8, g.K);
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CA; i++) {
            const int c = t + i * NT;
            *reinterpret_cast<u32x4*>(&lds[buf][(c / CPR) * LDK + (c % CPR) * 8]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const int c = t + i * NT;
            *reinterpret_cast<u32x4*>(&lds[buf][(BM + c / CPR) * LDK + (c % CPR) * 8]) = rb[i];
        }
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int lr = lane & 31, lk = (lane >> 5) * 8;
    auto compute = [&](int buf) {
        const _Float16* As = &lds[buf][(wm * WTM + lr) * LDK + lk];
        const _Float16* Bs = &lds[buf][(BM + wn * WTN + lr) * LDK + lk];
#pragma unroll
        for (int ks = 0; ks < BK; ks += 16) {
            halfx8 a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) a[i] = *reinterpret_cast<const halfx8*>(As + i * 32 * LDK + ks);
#pragma unroll
            for (int j = 0; j < TN; j++) b[j] = *reinterpret_cast<const halfx8*>(Bs + j * 32 * LDK + ks);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };

    // Pipeline: tile k + 1 sits in registers while tile k is multiplied.  At
    // the top of iteration k it goes to the other LDS buffer (its loads were
    // issued one whole iteration earlier, so their latency is hidden), then
    // the loads of tile k + 2 are issued into the same registers, then tile
    // k's MFMAs run, then one barrier.  The buffer written in iteration k was
    // last read in iteration k - 1, before that iteration's barrier.
    const int nk = (g.K + BK - 1) / BK;
    load_tile(0);
    if (BK > g.K) mask_tile(0);
    store_tile(0);
    if (nk > 1) load_tile(BK);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) {
            const int k1 = (kt + 1) * BK;
            if (k1 + BK > g.K) mask_tile(k1);
            store_tile(cur ^ 1);
            if (kt + 2 < nk) load_tile(k1 + BK);
        }
        // keep the stores and the next loads ahead of this tile's MFMAs
        __builtin_amdgcn_sched_barrier(0);
        compute(cur);
        if constexpr (IGLP >= 0) __builtin_amdgcn_iglp_opt(IGLP);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
            epilogue_col<YDT>(g, m0 + wm * WTM + i * 32, m0 + wm * WTM + i * 32 + (lk >> 1), n0 + wn * WTN + j * 32,
                              n0 + wn * WTN + j * 32 + lr, acc[i][j]);
}

// f16 NT with K % 64 == 0 (lda, ldb multiples of 8): 256x256x64 block tiles over
// 8 waves of 128x64 (two waves per SIMD), the operands fetched straight into
// LDS by buffer loads (no register staging, no LDS store instructions).
// On MI355X this Gemm runs at its power limit (1.5-1.7 GHz, against 2.4 GHz
// for the f32 Gemm), so what pays is energy per MFMA: the direct loads and the
// larger wave tiles (192 KB of fragment reads per k-tile, not 256 KB) run it
// at a higher clock than the register-staged 16-wave kernel above.
// LDS layout: per operand 32 blocks of 1 KB, block b holding rows 8b..8b+7 of
// 64 halves; one load instruction of a wave fills one block, lane l writing
// slot l & 7 of row l >> 3, and it fetches chunk (l & 7) ^ ((row >> 1) & 7) of
// that row, so chunk c of row r sits in slot c ^ ((r >> 1) & 7): the 16 rows
// that 16 lanes of a fragment read touch cover the 64 banks once.  Rows past M
// or N lie past the buffer resource's range and load as zeros.
// MFMA step s of a k-tile multiplies k = 16 s + 8 h .. + 7 in lane half h, the
// order of k_gemm_f16_nt: the two kernels return the same bits.
// Pipeline per k-tile: loads of tile k + 1 into the idle buffer, MFMAs of tile
// k with each step's fragments read one step ahead, then this wave's loads are
// waited for and one barrier; the next tile's first fragments are read after
// the barrier while the last MFMAs of this tile are in flight.
template <int YDT>
__global__ __launch_bounds__(512, 1) void k_gemm_f16_dl(GemmArgs g) {
    constexpr int BM = 256, BN = 256, BK = 64, NL = 8, PRE = 4;
    __shared__ __attribute__((aligned(1024))) _Float16 lds[2][(BM + BN) * BK];
    const int nbm = (g.M + BM - 1) / BM, nbn = (g.N + BN - 1) / BN;
    int tm, tn;
    tile_of_block(nbm, nbn, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const __amdgpu_buffer_rsrc_t ar = buffer_rsrc(g.A, (uint32_t)((int64_t)g.M * g.lda * 2));
    const __amdgpu_buffer_rsrc_t br = buffer_rsrc(g.B, (uint32_t)((int64_t)g.N * g.ldb * 2));
    // load q of this wave fills block wave + 8 q: q < 4 of A, q >= 4 of B
    uint32_t voff[NL];
#pragma unroll
    for (int q = 0; q < NL; q++) {
        const int r = ((wave + 8 * q) & 31) * 8 + (lane >> 3);
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        voff[q] = q < 4 ? (uint32_t)(((m0 + r) * g.lda + c * 8) * 2) : (uint32_t)(((n0 + r) * g.ldb + c * 8) * 2);
    }
    // the k offset goes in soffset, which the range check leaves out: a row
    // past M / N is out of range through voffset alone
    auto dload = [&](int buf, int k0, int q) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(q < 4 ? ar : br,
                                                 (__attribute__((address_space(3))) void*)&lds[buf][(wave + 8 * q) * 512],
                                                 16, voff[q], k0 * 2, 0, 0);
    };
    const int lr = lane & 31, h = lane >> 5;
    int aoff[4], boff[4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int slot = (2 * s + h) ^ ((lr >> 1) & 7);
        aoff[s] = (wm * 128 + lr) * BK + slot * 8;
        boff[s] = (BM + wn * 64 + lr) * BK + slot * 8;
    }
    halfx8 fa0[4], fb0[2], fa1[4], fb1[2];
    auto fread = [&](int buf, int s, halfx8 (&fa)[4], halfx8 (&fb)[2]) {
#pragma unroll
        for (int i = 0; i < 4; i++) fa[i] = *reinterpret_cast<const halfx8*>(&lds[buf][aoff[s] + i * 32 * BK]);
#pragma unroll
        for (int j = 0; j < 2; j++) fb[j] = *reinterpret_cast<const halfx8*>(&lds[buf][boff[s] + j * 32 * BK]);
    };
    floatx16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    auto mfmas = [&](const halfx8 (&fa)[4], const halfx8 (&fb)[2], int lo, int hi) {
#pragma unroll
        for (int q = lo; q < hi; q++)
            acc[q >> 1][q & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[q >> 1], fb[q & 1], acc[q >> 1][q & 1], 0, 0, 0);
    };
    // group masks of sched_group_barrier: MFMA 0x008, VMEM read 0x020, DS read 0x100
    auto interleave = [&](int nvmem) {
#pragma unroll
        for (int q = 0; q < 8; q++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (q < 6) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            if (q < nvmem) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
    };
    const int nk = g.K / BK;
#pragma unroll
    for (int q = 0; q < NL; q++) dload(0, 0, q);
    __builtin_amdgcn_s_waitcnt(0x3f70);    // vmcnt(0)
    __syncthreads();
    fread(0, 0, fa0, fb0);
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        // past the last tile the last tile is loaded again into the idle buffer
        const int kn = min(kt + 1, nk - 1) * BK;
        fread(cur, 1, fa1, fb1);
#pragma unroll
        for (int q = 0; q < NL; q++) dload(cur ^ 1, kn, q);
        mfmas(fa0, fb0, 0, 8);
        interleave(NL);
        __builtin_amdgcn_sched_barrier(0);
        fread(cur, 2, fa0, fb0);
        mfmas(fa1, fb1, 0, 8);
        interleave(0);
        __builtin_amdgcn_sched_barrier(0);
        fread(cur, 3, fa1, fb1);
        mfmas(fa0, fb0, 0, 8);
        interleave(0);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(fa1, fb1, 0, PRE);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0x3f70);    // vmcnt(0): this wave's blocks of tile k + 1 are in LDS
        __syncthreads();
        fread(cur ^ 1, 0, fa0, fb0);
        mfmas(fa1, fb1, PRE, 8);
#pragma unroll
        for (int q = 0; q < 6; q++) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            if (q < 8 - PRE) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // Written out: as a loop the f16 epilogue is too large to be unrolled, and
    // a rolled loop indexes the accumulators through scratch memory.  A block
    // wholly inside Y with alpha = 1 and no bias or a scalar / per-column one
    // (the ONNX Gemm's usual case) takes one lean variant for all its tiles;
    // 1.0 * x is x, so it returns the general path's bits.
    const int mw = m0 + wm * 128 + 4 * h, nw = n0 + wn * 64 + lr;
    if (g.alpha == 1.0 && m0 + BM <= g.M && n0 + BN <= g.N && (g.c.mode == 1 || g.c.mode == 2)) {
        auto epi = [&](int i, int j, const floatx16& a) { epilogue_col_f<YDT, 1, true, true>(g, mw + i * 32, nw + j * 32, a); };
        epi(0, 0, acc[0][0]); epi(0, 1, acc[0][1]); epi(1, 0, acc[1][0]); epi(1, 1, acc[1][1]);
        epi(2, 0, acc[2][0]); epi(2, 1, acc[2][1]); epi(3, 0, acc[3][0]); epi(3, 1, acc[3][1]);
    } else if (g.alpha == 1.0 && m0 + BM <= g.M && n0 + BN <= g.N && g.c.mode == 0) {
        auto epi = [&](int i, int j, const floatx16& a) { epilogue_col_f<YDT, 0, true, true>(g, mw + i * 32, nw + j * 32, a); };
        epi(0, 0, acc[0][0]); epi(0, 1, acc[0][1]); epi(1, 0, acc[1][0]); epi(1, 1, acc[1][1]);
        epi(2, 0, acc[2][0]); epi(2, 1, acc[2][1]); epi(3, 0, acc[3][0]); epi(3, 1, acc[3][1]);
    } else {
        auto epi = [&](int i, int j, const floatx16& a) {
            epilogue_col<YDT>(g, m0 + wm * 128 + i * 32, mw + i * 32, n0 + wn * 64 + j * 32, nw + j * 32, a);
        };
        epi(0, 0, acc[0][0]); epi(0, 1, acc[0][1]); epi(1, 0, acc[1][0]); epi(1, 1, acc[1][1]);
        epi(2, 0, acc[2][0]); epi(2, 1, acc[2][1]); epi(3, 0, acc[3][0]); epi(3, 1, acc[3][1]);
    }
}

// ------------------------------------------------------------- f32 NT tiled ---
// Weight-only-quantized B: int8 / uint8 codes with a per-tensor or per-row
// (per output column n) scale and zero point.
struct WoqB {
    const float* s;      // scale: 1 element, or N elements (per n)
    const void* z;       // zero point of B's dtype, 1 or N elements, or null (zero)
    int per_n;           // scale / zero point indexed by n
    int zn;              // zero point elements (0, 1 or N)
};

// A [M, K] f32 and B [N, K] (transB = 1) with K % 4 == 0: v_mfma_f32_32x32x2f32
// on BM x BN x BK tiles, operands through raw buffer loads one k-tile ahead into
// registers, LDS double buffer, XCD-aware tile order.
// BQ = 0: B is f32.  BQ = 1 / 2: B holds int8 / uint8 codes, turned into
// (float)(q - zp) * s while staging into LDS.  (q - zp) is an integer of at
// most 9 bits, so the fp32 product is the correctly rounded exact product, the
// value DequantizeLinear writes (tensor_ops.c:1018-1034 computes it in double
// and rounds once): the fused Gemm sees bit for bit the operand the unfused
// DequantizeLinear -> Gemm pair sees, and with the same tile shape it returns
// the same bits.
// MFMA step s of a k-tile multiplies k = h * BK/2 + s in lane half h, so each
// lane reads BK/2 consecutive floats of its row (b128 LDS reads); A and B use
// the same order, so every product pairs equal k.
// SPLIT: blockIdx.y takes k in [y * kchunk, (y + 1) * kchunk) (kchunk a
// multiple of BK) and writes its raw fp32 sums to the workspace g.Y + y * M * N;
// k_splitk_reduce adds the slices in order and applies the epilogue.
template <int BM, int BN, int BK, int WGM, int WGN, int YDT, int BQ, int IGLP = -1, bool SPLIT = false>
__global__ __launch_bounds__(64 * WGM * WGN) void k_gemm_f32_nt(GemmArgs g, WoqB q, int kchunk) {
    constexpr int NT = 64 * WGM * WGN;
    constexpr int LDK = BK + 4;
    constexpr int WTM = BM / WGM, WTN = BN / WGN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int CPR = BK / 4;                   // 4-element chunks per tile row
    constexpr int CA = BM * CPR / NT, CB = BN * CPR / NT;
    constexpr int EB = BQ ? 1 : 4;                // bytes per B element
    static_assert(CA * NT == BM * CPR && CB * NT == BN * CPR && CA >= 1 && CB >= 1, "tile / thread mismatch");
    static_assert(TM >= 1 && TN >= 1 && BK % 8 == 0, "wave tile");
    __shared__ float lds[2][(BM + BN) * LDK];

    const int nbm = (g.M + BM - 1) / BM, nbn = (g.N + BN - 1) / BN;
    int tm, tn;
    tile_of_block(nbm, nbn, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    // Rows past M / N read as zero; the host guarantees (rows + tile) * ld * size < 2^31.
    const __amdgpu_buffer_rsrc_t ar = buffer_rsrc(g.A, (uint32_t)((int64_t)g.M * g.lda * 4));
    const __amdgpu_buffer_rsrc_t br = buffer_rsrc(g.B, (uint32_t)((int64_t)g.N * g.ldb * EB));

    // Per-row dequantisation constants of the B chunks this thread stages
    // (a thread's chunk rows do not change across k-tiles).
    float bs[BQ ? CB : 1];
    int bz[BQ ? CB : 1];
    if constexpr (BQ) {
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const int n = min(n0 + (t + i * NT) / CPR, g.N - 1);
            bs[i] = q.s[q.per_n ? n : 0];
            const int zi = q.zn > 1 ? n : 0;
            bz[i] = q.zn == 0 ? 0 : (BQ == 1 ? (int)((const int8_t*)q.z)[zi] : (int)((const uint8_t*)q.z)[zi]);
        }
    }

    u32x4 ra[CA];
    uint32_t rq[BQ ? CB : 1];
    u32x4 rb[BQ ? 1 : CB];
    auto load_tile = [&](int k0) {
#pragma unroll
        for (int i = 0; i < CA; i++) {
            const int c = t + i * NT;
            const int k = k0 + (c % CPR) * 4;
            ra[i] = ld_buf_b128(ar, k < g.K ? (uint32_t)(((m0 + c / CPR) * g.lda + k) * 4) : kOOB);
        }
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const int c = t + i * NT;
            const int k = k0 + (c % CPR) * 4;
            const uint32_t off = k < g.K ? (uint32_t)(((n0 + c / CPR) * g.ldb + k) * EB) : kOOB;
            if constexpr (BQ) rq[i] = __builtin_amdgcn_raw_buffer_load_b32(br, off, 0, 0);
            else rb[i] = ld_buf_b128(br, off);
        }
    };
    auto store_tile = [&](int buf, int k0) {
#pragma unroll
        for (int i = 0; i < CA; i++) {
            const int c = t + i * NT;
            *reinterpret_cast<u32x4*>(&lds[buf][(c / CPR) * LDK + (c % CPR) * 4]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const int c = t + i * NT;
            float* dst = &lds[buf][(BM + c / CPR) * LDK + (c % CPR) * 4];
            if constexpr (BQ) {
                // Past K the A operand is zero, but (0 - zp) * s need not be: zero it.
                const bool ok = k0 + (c % CPR) * 4 < g.K;
                const uint32_t w = rq[i];
                float4 v;
                float* pv = reinterpret_cast<float*>(&v);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int code = BQ == 1 ? (int)(int8_t)(w >> (8 * e)) : (int)((w >> (8 * e)) & 255u);
                    pv[e] = ok ? (float)(code - bz[i]) * bs[i] : 0.0f;
                }
                *reinterpret_cast<float4*>(dst) = v;
            } else {
                *reinterpret_cast<u32x4*>(dst) = rb[i];
            }
        }
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int lr = lane & 31, lh = (lane >> 5) * (BK / 2);
    auto compute = [&](int buf) {
        const float* As = &lds[buf][(wm * WTM + lr) * LDK + lh];
        const float* Bs = &lds[buf][(BM + wn * WTN + lr) * LDK + lh];
#pragma unroll
        for (int s4 = 0; s4 < BK / 2; s4 += 4) {
            float4 a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) a[i] = *reinterpret_cast<const float4*>(As + i * 32 * LDK + s4);
#pragma unroll
            for (int j = 0; j < TN; j++) b[j] = *reinterpret_cast<const float4*>(Bs + j * 32 * LDK + s4);
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(reinterpret_cast<const float*>(&a[i])[e],
                                                                         reinterpret_cast<const float*>(&b[j])[e],
                                                                         acc[i][j], 0, 0, 0);
        }
    };

    // Tiles never straddle a split boundary, so masking against K stays exact.
    const int kbeg = SPLIT ? (int)blockIdx.y * kchunk : 0;
    const int kend = SPLIT ? min(g.K, kbeg + kchunk) : g.K;
    const int nk = (kend - kbeg + BK - 1) / BK;
    load_tile(kbeg);
    store_tile(0, kbeg);
    __syncthreads();
    int kt = 0;
    for (; kt + 1 < nk; kt++) {
        const int cur = kt & 1;
        const int k1 = kbeg + (kt + 1) * BK;
        load_tile(k1);
        compute(cur);
        if constexpr (IGLP >= 0) __builtin_amdgcn_iglp_opt(IGLP);
        store_tile(cur ^ 1, k1);
        __syncthreads();
    }
    compute(kt & 1);
    gfloat* part = (gfloat*)g.Y + (SPLIT ? (int64_t)blockIdx.y * g.M * g.N : 0);
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int n = n0 + wn * WTN + j * 32 + lr;
                if (m < g.M && n < g.N) {
                    if constexpr (SPLIT) part[(int64_t)m * g.N + n] = acc[i][j][r];
                    else epilogue_fast<YDT>(g, m, n, (double)acc[i][j][r]);
                }
            }
}

// Sums the split-K slices of element (m, n) in slice order (in double) and
// applies the Gemm epilogue.  One element per thread, coalesced; M * N < 2^31
// (the caller's reach check bounds it).
template <int YDT>
__global__ __launch_bounds__(256) void k_splitk_reduce(GemmArgs g, const float* __restrict__ part, int nsplit,
                                                       FastDiv fd_n) {
    const int mn = g.M * g.N;
    const int i = (int)blockIdx.x * 256 + (int)threadIdx.x;
    if (i >= mn) return;
    double acc = 0.0;
    for (int sp = 0; sp < nsplit; sp++) acc += (double)part[(int64_t)sp * mn + i];
    const int m = (int)fd_n.div((uint32_t)i);
    epilogue_fast<YDT>(g, m, i - m * g.N, acc);
}

// -------------------------------------------------------------------- dispatch ---
inline bool f32_exact_dtype(int dt) {
    return dt == kF32 || dt == kF16 || dt == kBF16 || dt == kE4M3 || dt == kE5M2 || dt == kI4 || dt == kI8 ||
           dt == kU8 || dt == kI16;
}

template <int DA, int DB, bool TA, bool TB, bool VEC>
void launch_f32_y(const GemmArgs& g, int dta, int dtb, dim3 grid, hipStream_t s) {
    if (g.dty == kF32)
        hipLaunchKernelGGL((k_gemm_mfma_f32<DA, DB, TA, TB, VEC, kF32>), grid, dim3(kThreads), 0, s, g, dta, dtb);
    else
        hipLaunchKernelGGL((k_gemm_mfma_f32<DA, DB, TA, TB, VEC, -1>), grid, dim3(kThreads), 0, s, g, dta, dtb);
}

template <int DA, int DB, bool VEC>
void launch_f32_t(const GemmArgs& g, int dta, int dtb, int ta, int tb, dim3 grid, hipStream_t s) {
    if (!ta && tb) launch_f32_y<DA, DB, false, true, VEC>(g, dta, dtb, grid, s);
    else if (!ta && !tb) launch_f32_y<DA, DB, false, false, VEC>(g, dta, dtb, grid, s);
    else if (ta && tb) launch_f32_y<DA, DB, true, true, VEC>(g, dta, dtb, grid, s);
    else launch_f32_y<DA, DB, true, false, VEC>(g, dta, dtb, grid, s);
}

template <bool TA, bool TB>
void launch_f16_y(const GemmArgs& g, dim3 grid, int vec, hipStream_t s) {
    if (g.dty == kF16) hipLaunchKernelGGL((k_gemm_mfma_f16<TA, TB, kF16>), grid, dim3(kThreads), 0, s, g, vec);
    else if (g.dty == kF32) hipLaunchKernelGGL((k_gemm_mfma_f16<TA, TB, kF32>), grid, dim3(kThreads), 0, s, g, vec);
    else hipLaunchKernelGGL((k_gemm_mfma_f16<TA, TB, -1>), grid, dim3(kThreads), 0, s, g, vec);
}

// f16 x f16 with both operands K-major (A [M, K], B [N, K]) and 16-byte
// aligned rows: the tiled kernel.  256x256 tiles (16 waves of 64x64) when the
// grid still covers the 256 CUs, else 128x128 tiles (4 waves of 64x64).
// Sweeps on MI355X: 16 waves of 64x64 beat 8 waves of 128x64 or 64x128 and a
// two-group ping-pong of 8 waves at 4096^3.
// Returns false when the operands exceed the 2 GB reach of a buffer resource.
template <int BM, int BN, int BK, int WGM, int WGN, int IGLP>
void launch_f16_nt_cfg(const GemmArgs& g, hipStream_t s) {
    const int nb = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
    const bool fast_bias = g.c.mode == 0 || (g.c.dt == kF32 && g.c.mode <= 3);
    const dim3 grid(nb), block(64 * WGM * WGN);
    if (fast_bias && g.dty == kF16)
        hipLaunchKernelGGL((k_gemm_f16_nt<BM, BN, BK, WGM, WGN, kF16, IGLP>), grid, block, 0, s, g);
    else if (fast_bias && g.dty == kF32)
        hipLaunchKernelGGL((k_gemm_f16_nt<BM, BN, BK, WGM, WGN, kF32, IGLP>), grid, block, 0, s, g);
    else
        hipLaunchKernelGGL((k_gemm_f16_nt<BM, BN, BK, WGM, WGN, -1, IGLP>), grid, block, 0, s, g);
}

bool launch_f16_nt(const GemmArgs& g, hipStream_t s) {
    const int64_t reach = (int64_t)1 << 31;
    if ((int64_t)(g.M + 256) * g.lda * 2 >= reach || (int64_t)(g.N + 256) * g.ldb * 2 >= reach) return false;
    const int64_t big_tiles = (int64_t)((g.M + 255) / 256) * ((g.N + 255) / 256);
    const bool fast_bias = g.c.mode == 0 || (g.c.dt == kF32 && g.c.mode <= 3);
    if (big_tiles >= 192 && g.K > 0 && g.K % 64 == 0 && fast_bias && (g.dty == kF16 || g.dty == kF32)) {
        // 4096^3 on MI355X: 132.9 -> 124.0 us against the 16-wave kernel on one box
        const dim3 grid((unsigned)big_tiles), block(512);
        if (g.dty == kF16) hipLaunchKernelGGL((k_gemm_f16_dl<kF16>), grid, block, 0, s, g);
        else hipLaunchKernelGGL((k_gemm_f16_dl<kF32>), grid, block, 0, s, g);
    } else if (big_tiles >= 192) launch_f16_nt_cfg<256, 256, 64, 4, 4, 1>(g, s);
    else launch_f16_nt_cfg<128, 128, 64, 2, 2, 1>(g, s);
    return true;
}

// f32 A [M, K] with B [N, K] (f32 codes or int8 / uint8 codes dequantised on
// the fly): the tiled kernel.  128x256 tiles over 8 waves (64x64 each) when
// they cover the CUs; otherwise 128x64 tiles with k split into up to 16
// slices (each at least 64 deep) so that about 512 blocks run, the slices
// summed by k_splitk_reduce.  The plan depends on M, N and K only, so the
// fused weight-only-quantized Gemm and the unfused DequantizeLinear -> Gemm
// pair run the same schedule and return the same bits.
// Returns 1 when launched, 0 when the operands do not fit the kernel (caller
// falls back), -1 on an allocation failure (error set).
int nt_split_plan(int M, int N, int K, bool& big) {
    const int64_t big_tiles = (int64_t)((M + 127) / 128) * ((N + 255) / 256);
    big = big_tiles >= 192;
    if (big) return 1;
    const int64_t tiles = (int64_t)((M + 127) / 128) * ((N + 63) / 64);
    int64_t sp = std::min<int64_t>((512 + tiles - 1) / tiles, K / 64);
    return (int)std::max<int64_t>(1, std::min<int64_t>(sp, 16));
}

template <int BM, int BN, int BK, int WGM, int WGN, int BQ, bool SPLIT>
void launch_nt_kernel(const GemmArgs& g, const WoqB& q, int kchunk, int nsplit, int ydt, hipStream_t s) {
    const dim3 grid(((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN), nsplit), block(64 * WGM * WGN);
    if (SPLIT || ydt == kF32)
        hipLaunchKernelGGL((k_gemm_f32_nt<BM, BN, BK, WGM, WGN, kF32, BQ, -1, SPLIT>), grid, block, 0, s, g, q, kchunk);
    else if (ydt == kF16)
        hipLaunchKernelGGL((k_gemm_f32_nt<BM, BN, BK, WGM, WGN, kF16, BQ, -1, SPLIT>), grid, block, 0, s, g, q, kchunk);
    else
        hipLaunchKernelGGL((k_gemm_f32_nt<BM, BN, BK, WGM, WGN, -1, BQ, -1, SPLIT>), grid, block, 0, s, g, q, kchunk);
}

// probs (f32 [M, N], or null): with a k split, the reduction also takes the
// rows' softmax into probs (returns 2); otherwise the caller runs the softmax.
template <int BQ>
int launch_f32_nt(const GemmArgs& g, const WoqB& q, hipStream_t s, float* probs = nullptr) {
    const int64_t reach = (int64_t)1 << 31;
    const int eb = BQ ? 1 : 4;
    if ((int64_t)(g.M + 256) * g.lda * 4 >= reach || (int64_t)(g.N + 256) * g.ldb * eb >= reach) return 0;
    const bool fast_bias = g.c.mode == 0 || (g.c.dt == kF32 && g.c.mode <= 3);
    const int ydt = fast_bias && (g.dty == kF32 || g.dty == kF16) ? g.dty : -1;
    bool big = false;
    int split = nt_split_plan(g.M, g.N, g.K, big);
    // (no k split under graph capture: the slices' workspace would have to outlive the call)
    if (split > 1 && stream_capturing(s)) split = 1;
    if (big) {
        launch_nt_kernel<128, 256, 16, 2, 4, BQ, false>(g, q, 0, 1, ydt, s);
        return 1;
    }
    if (split <= 1) {
        launch_nt_kernel<128, 64, 16, 2, 2, BQ, false>(g, q, 0, 1, ydt, s);
        return 1;
    }
    const int kchunk = ((g.K + split - 1) / split + 15) / 16 * 16;
    const int nsplit = (g.K + kchunk - 1) / kchunk;
    const int64_t mn = (int64_t)g.M * g.N;
    float* part = (float*)pool_alloc((size_t)nsplit * mn * sizeof(float));
    if (!part) return -1;
    GemmArgs gp = g;
    gp.Y = part;
    launch_nt_kernel<128, 64, 16, 2, 2, BQ, true>(gp, q, kchunk, nsplit, kF32, s);
    if (probs && ydt == kF32 &&
        launch_splitk_softmax(part, nsplit, g.M, g.N, g.alpha, g.beta, (const float*)g.c.p, g.c.mode, (float*)g.Y,
                              probs, s)) {
        pool_free(part);
        return 2;
    }
    const dim3 rgrid((unsigned)((mn + 255) / 256));
    const FastDiv fd_n = make_fastdiv((uint32_t)g.N);
    if (ydt == kF32)
        hipLaunchKernelGGL((k_splitk_reduce<kF32>), rgrid, dim3(256), 0, s, g, (const float*)part, nsplit, fd_n);
    else if (ydt == kF16)
        hipLaunchKernelGGL((k_splitk_reduce<kF16>), rgrid, dim3(256), 0, s, g, (const float*)part, nsplit, fd_n);
    else
        hipLaunchKernelGGL((k_splitk_reduce<-1>), rgrid, dim3(256), 0, s, g, (const float*)part, nsplit, fd_n);
    pool_free(part);   // stream-ordered reuse: later work on this stream runs after the reduction
    return 1;
}

// f32 x f32 uses typed (optionally vectorised) staging; every other pair of
// fp32-exact dtypes is decoded with a run-time switch while staging.
bool launch_f32_mfma(const GemmArgs& g, int dta, int dtb, int ta, int tb, hipStream_t s) {
    const dim3 grid((g.N + kBN - 1) / kBN, (g.M + kBM - 1) / kBM);
    if (dta == kF32 && dtb == kF32) {
        const bool vec = ((g.lda % 4) == 0) && ((g.ldb % 4) == 0) && (((uintptr_t)g.A & 15) == 0) &&
                         (((uintptr_t)g.B & 15) == 0);
        if (vec) launch_f32_t<kF32, kF32, true>(g, dta, dtb, ta, tb, grid, s);
        else launch_f32_t<kF32, kF32, false>(g, dta, dtb, ta, tb, grid, s);
    } else {
        launch_f32_t<-1, -1, false>(g, dta, dtb, ta, tb, grid, s);
    }
    return true;
}

}  // namespace
}  // namespace tohip

using namespace tohip;

namespace {
// gemm_forward; with probs (a device f32 [M, N] buffer) the rows' softmax of Y is
// written there as well when the split reduction can take it (*softmax_done).
void gemm_impl(const char* name, const Tensor* A, const Tensor* B, const Tensor* C, Tensor* Y, float alpha,
               float beta, int transA, int transB, float* probs, bool* softmax_done) {
    if (!tensor_sane(A, name) || !tensor_sane(B, name) || !tensor_sane(Y, name)) return;
    if (A->ndim < 2 || B->ndim < 2) { set_error("%s: A and B must be 2-D", name); return; }
    const int M = transA ? A->shape[1] : A->shape[0];
    const int K = transA ? A->shape[0] : A->shape[1];
    const int N = transB ? B->shape[0] : B->shape[1];
    const int KB = transB ? B->shape[1] : B->shape[0];
    if (K != KB) { set_error("%s: inner dimensions differ (%d vs %d)", name, K, KB); return; }
    if ((size_t)M * (size_t)N > Y->size) { set_error("%s: Y holds %zu elements, needs %d x %d", name, Y->size, M, N); return; }
    const bool has_c = C && C->data;
    if (has_c && !tensor_sane(C, name)) return;
    if (!ensure_device()) return;

    GemmArgs g;
    g.M = M; g.N = N; g.K = K;
    g.lda = A->shape[1]; g.ldb = B->shape[1];
    g.alpha = (double)alpha; g.beta = (double)beta;
    g.dty = (int)Y->dtype;
    g.c = Bias{nullptr, has_c ? (int)C->dtype : 0, 0, 0, 0};
    if (has_c) {
        // tensor_ops.c:1197-1220
        if (C->size == 1) g.c.mode = 1;
        else if (C->ndim == 1) g.c.mode = (C->shape[0] == N) ? 2 : (C->shape[0] == M ? 3 : 5);
        else if (C->ndim >= 2) { g.c.mode = 4; g.c.H = C->shape[C->ndim - 2]; g.c.W = C->shape[C->ndim - 1]; }
        // The reference's Python passes a 1-D bias reshaped to (1, N) or (M, 1)
        // (nn/Operators.py:638-645); those index exactly like the per-column /
        // per-row modes, which the MFMA epilogues handle inline.
        if (g.c.mode == 4 && C->size == (size_t)g.c.H * g.c.W) {
            if (g.c.H == 1 && g.c.W == N) g.c.mode = 2;
            else if (g.c.H == M && g.c.W == 1) g.c.mode = 3;
        }
    }
    Staging st;
    g.A = st.in(A);
    g.B = st.in(B);
    if (has_c) g.c.p = st.in(C);
    g.Y = st.out(Y, (size_t)M * N * dt_bytes((int)Y->dtype));
    if (!g.A || !g.B || !g.Y || (has_c && !g.c.p)) { st.finish(); return; }
    if (!has_c) g.c.mode = 0;
    hipStream_t s = stream();
    const int dta = (int)A->dtype, dtb = (int)B->dtype;
    if ((size_t)M * N > 0) {
        bool done = false;
        if (!exact_mode() && K > 0) {
            if (dta == kF16 && dtb == kF16) {
                const dim3 grid((N + kBN - 1) / kBN, (M + kBM - 1) / kBM);
                const int vec = ((g.lda % 8) == 0 && (g.ldb % 8) == 0 && ((uintptr_t)g.A & 15) == 0 &&
                                 ((uintptr_t)g.B & 15) == 0) ? 1 : 0;
                if (!transA && transB && vec && launch_f16_nt(g, s)) {
                } else if (!transA && transB) launch_f16_y<false, true>(g, grid, vec, s);
                else if (!transA && !transB) launch_f16_y<false, false>(g, grid, vec, s);
                else if (transA && transB) launch_f16_y<true, true>(g, grid, vec, s);
                else launch_f16_y<true, false>(g, grid, vec, s);
                done = true;
            } else if (f32_exact_dtype(dta) && f32_exact_dtype(dtb)) {
                const bool nt = dta == kF32 && dtb == kF32 && !transA && transB && (g.lda % 4) == 0 &&
                                (g.ldb % 4) == 0 && ((uintptr_t)g.A & 15) == 0 && ((uintptr_t)g.B & 15) == 0;
                const int r = nt ? launch_f32_nt<0>(g, WoqB{nullptr, nullptr, 0, 0}, s, probs) : 0;
                if (r < 0) { st.finish(); return; }
                if (r == 2 && softmax_done) *softmax_done = true;
                done = r >= 1 || launch_f32_mfma(g, dta, dtb, transA, transB, s);
            }
        }
        if (!done) {
            const dim3 grid((N + kET - 1) / kET, (M + kET - 1) / kET);
            hipLaunchKernelGGL(k_gemm_exact, grid, dim3(kET * kET), 0, s, g, dta, dtb, transA, transB);
        }
        if (!check_launch(name)) { st.finish(); return; }
    }
    st.finish();
}
}  // namespace

extern "C" void gemm_forward(const Tensor* A, const Tensor* B, const Tensor* C, Tensor* Y, float alpha, float beta,
                             int transA, int transB) {
    gemm_impl("gemm_forward", A, B, C, Y, alpha, beta, transA, transB, nullptr, nullptr);
}

extern "C" void gemm_softmax_forward(const Tensor* A, const Tensor* B, const Tensor* C, Tensor* Y, Tensor* P,
                                     float alpha, float beta, int transA, int transB) {
    const char* name = "gemm_softmax_forward";
    if (!tensor_sane(Y, name) || !tensor_sane(P, name)) return;
    if (P->size != Y->size || Y->ndim < 2) { set_error("%s: P must have Y's size and Y two dimensions", name); return; }
    const bool fuse = (int)Y->dtype == kF32 && (int)P->dtype == kF32 && is_dev(classify(Y->data)) &&
                      is_dev(classify(P->data));
    bool done = false;
    gemm_impl(name, A, B, C, Y, alpha, beta, transA, transB, fuse ? (float*)P->data : nullptr, &done);
    if (tensor_ops_hip_last_error()[0] || done) return;
    softmax_forward(Y, P, Y->ndim - 1);
}

namespace {
// The unfused pair, for the cases the fused kernel does not cover.
void dequantize_then_gemm(const Tensor* A, const Tensor* Bq, const Tensor* Scale, const Tensor* ZeroPoint, int axis,
                          const Tensor* C, Tensor* Y, float alpha, float beta, int transA, int transB) {
    int shp[2] = {Bq->shape[0], Bq->shape[1]};
    Tensor* Bd = create_tensor_device_empty(shp, 2, DTYPE_FLOAT32);
    if (!Bd) return;
    tensor_ops_hip_clear_error();
    dequantize_linear_axis_forward(Bq, Scale, ZeroPoint, Bd, axis);
    if (tensor_ops_hip_last_error()[0] == 0) gemm_forward(A, Bd, C, Y, alpha, beta, transA, transB);
    free_tensor(Bd);
}
}  // namespace

// Weight-only-quantized Gemm: the DequantizeLinear -> Gemm pair of a quantized
// ONNX graph (tensor_ops.c:1018-1034 then :1167-1228) in one pass.  The fused
// kernel covers f32 A [M, K] (transA = 0) with B [N, K] (transB = 1) of int8 /
// uint8 codes, an f32 Scale of 1 or N elements (axis 0) and a ZeroPoint of B's
// dtype; everything else runs the two operators in sequence, which is also
// what the fused kernel returns, bit for bit.
extern "C" void dequantize_gemm_forward(const Tensor* A, const Tensor* Bq, const Tensor* Scale,
                                        const Tensor* ZeroPoint, int axis, const Tensor* C, Tensor* Y, float alpha,
                                        float beta, int transA, int transB) {
    const char* name = "dequantize_gemm_forward";
    if (!tensor_sane(A, name) || !tensor_sane(Bq, name) || !tensor_sane(Scale, name) || !tensor_sane(Y, name)) return;
    const bool has_z = ZeroPoint && ZeroPoint->data;
    if (has_z && !tensor_sane(ZeroPoint, name)) return;
    if (A->ndim != 2 || Bq->ndim != 2) { set_error("%s: A and B must be 2-D", name); return; }
    if (axis < 0) axis += 2;
    if (axis < 0 || axis > 1) { set_error("%s: axis out of range", name); return; }
    const size_t nax = (size_t)Bq->shape[axis];
    if (Scale->size != 1 && Scale->size != nax) {
        set_error("%s: Scale must have 1 or B.shape[axis] elements", name);
        return;
    }
    if (has_z && ZeroPoint->size != 1 && ZeroPoint->size != nax) {
        set_error("%s: ZeroPoint must have 1 or B.shape[axis] elements", name);
        return;
    }
    const int M = transA ? A->shape[1] : A->shape[0];
    const int K = transA ? A->shape[0] : A->shape[1];
    const int N = transB ? Bq->shape[0] : Bq->shape[1];
    const int KB = transB ? Bq->shape[1] : Bq->shape[0];
    if (K != KB) { set_error("%s: inner dimensions differ (%d vs %d)", name, K, KB); return; }
    if ((size_t)M * (size_t)N > Y->size) { set_error("%s: Y holds %zu elements, needs %d x %d", name, Y->size, M, N); return; }
    const bool has_c = C && C->data;
    if (has_c && !tensor_sane(C, name)) return;
    if (!ensure_device()) return;

    const int dtb = (int)Bq->dtype;
    const int64_t reach = (int64_t)1 << 31;
    const bool fused = !exact_mode() && A->dtype == kF32 && (dtb == kI8 || dtb == kU8) && Scale->dtype == kF32 &&
                       (!has_z || (int)ZeroPoint->dtype == dtb) && !transA && transB &&
                       (axis == 0 || (Scale->size == 1 && (!has_z || ZeroPoint->size == 1))) && (K % 4) == 0 &&
                       M > 0 && N > 0 && ((uintptr_t)A->data & 15) == 0 && ((uintptr_t)Bq->data & 3) == 0 &&
                       (int64_t)(M + 256) * K * 4 < reach && (int64_t)(N + 256) * K < reach;
    if (!fused) {
        dequantize_then_gemm(A, Bq, Scale, has_z ? ZeroPoint : nullptr, axis, C, Y, alpha, beta, transA, transB);
        return;
    }

    GemmArgs g;
    g.M = M; g.N = N; g.K = K;
    g.lda = K; g.ldb = K;
    g.alpha = (double)alpha; g.beta = (double)beta;
    g.dty = (int)Y->dtype;
    g.c = Bias{nullptr, has_c ? (int)C->dtype : 0, 0, 0, 0};
    if (has_c) {
        if (C->size == 1) g.c.mode = 1;
        else if (C->ndim == 1) g.c.mode = (C->shape[0] == N) ? 2 : (C->shape[0] == M ? 3 : 5);
        else { g.c.mode = 4; g.c.H = C->shape[C->ndim - 2]; g.c.W = C->shape[C->ndim - 1]; }
        if (g.c.mode == 4 && C->size == (size_t)g.c.H * g.c.W) {
            if (g.c.H == 1 && g.c.W == N) g.c.mode = 2;
            else if (g.c.H == M && g.c.W == 1) g.c.mode = 3;
        }
    }
    Staging st;
    g.A = st.in(A);
    g.B = st.in(Bq);
    const void* sp = st.in(Scale);
    const void* zp = has_z ? st.in(ZeroPoint) : nullptr;
    if (has_c) g.c.p = st.in(C);
    g.Y = st.out(Y, (size_t)M * N * dt_bytes((int)Y->dtype));
    if (!g.A || !g.B || !sp || (has_z && !zp) || !g.Y || (has_c && !g.c.p)) { st.finish(); return; }
    if (!has_c) g.c.mode = 0;
    const WoqB q{(const float*)sp, zp, Scale->size > 1 ? 1 : 0, has_z ? (int)ZeroPoint->size : 0};
    const int r = dtb == kI8 ? launch_f32_nt<1>(g, q, stream()) : launch_f32_nt<2>(g, q, stream());
    if (r > 0) check_launch(name);
    st.finish();
}
