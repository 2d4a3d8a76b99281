// conv.hip — Conv2d (NCHW) for gfx950.
//
// tensor_ops/tensor_ops.c:1036-1114: for each output (n, m, oh, ow), a double
// sum over (ic, kh, kw) of X * W with zero padding (padded taps contribute
// 0.0 * w), then + bias[m], written through the output encoder.  Output
// extent comes from Y's shape; pads[0] / pads[1] are top / left.
//
//  * k_conv_tiled — f32 x f32: implicit GEMM with register prefetch, buffer
//    loads and an LDS double buffer; three gathers (MODE 0 per-element
//    (c, kh, kw), MODE 1 1x1 float4, MODE 2 tap-blocked channels with
//    b128 LDS reads), split-K for small grids, fused Relu / residual
//    epilogue (described at the kernel and at launch_conv_tiled_xq).
//  * k_conv_mfma_f32 — other fp32-exact dtypes (decoded while staging):
//    implicit GEMM on v_mfma_f32_32x32x2f32.  Per group:
//    M = out channels, N = batch * OH * OW pixels, K = Cin/g * KH * KW.  The
//    block tile is 64 channels x 256 pixels (4 waves side by side, each
//    64 x 64 = 2x2 MFMA tiles), BK = 16.  Each thread owns one pixel column
//    of the im2col tile, so the gather along the pixel dimension is
//    coalesced; the (c, kh, kw) decode of k is uniform across the block.
//    fp32 accumulate: tolerance class vs the reference.
//  * k_conv_exact — fp64, reference summation order, bit-identical.
#include <algorithm>
#include <cmath>

#include "quant.h"
#include "runtime.h"

namespace tohip {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

struct ConvGeom {
    int N, C, H, W;      // input
    int M, KH, KW;       // weights [M, C/g, KH, KW]
    int OH, OW;          // output (from Y)
    int pt, pl, sh, sw, dh, dw, group;
    int Cg, Mg, Kg;      // per-group channels in / out, Cg * KH * KW
};

__global__ __launch_bounds__(256) void k_conv_exact(const void* __restrict__ X, int dtx, const void* __restrict__ Wt,
                                                    int dtw, const void* __restrict__ Bv, int dtb, void* __restrict__ Y,
                                                    int dty, ConvGeom g, int64_t total) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < total; o += stride) {
        const int ow = (int)(o % g.OW);
        int64_t t = o / g.OW;
        const int oh = (int)(t % g.OH);
        t /= g.OH;
        const int m = (int)(t % g.M);
        const int n = (int)(t / g.M);
        const int grp = m / g.Mg;
        double acc = 0.0;
        for (int c = 0; c < g.Cg; c++) {
            const int ic = grp * g.Cg + c;
            for (int kh = 0; kh < g.KH; kh++) {
                const int ih = oh * g.sh + kh * g.dh - g.pt;
                for (int kw = 0; kw < g.KW; kw++) {
                    const int iw = ow * g.sw + kw * g.dw - g.pl;
                    double xv = 0.0;
                    if (ih >= 0 && ih < g.H && iw >= 0 && iw < g.W)
                        xv = ld_d_rt(dtx, X, (((int64_t)n * g.C + ic) * g.H + ih) * g.W + iw);
                    const double wv = ld_d_rt(dtw, Wt, (((int64_t)m * g.Cg + c) * g.KH + kh) * g.KW + kw);
                    acc += xv * wv;
                }
            }
        }
        const double bias = Bv ? ld_d_rt(dtb, Bv, m) : 0.0;
        st_d_rt(dty, Y, o, acc + bias);
    }
}

constexpr int kCM = 64, kCN = 256, kCK = 16, kCPad = 4;

// DT >= 0: compile-time dtype; DT < 0: decode with the run-time dtype rdt.
template <int DT> __device__ __forceinline__ float ldf(const void* p, int64_t i, int rdt) {
    if constexpr (DT == kF32) return ((const float*)p)[i];
    else if constexpr (DT >= 0) return (float)ld_d<DT>(p, i);
    else return (float)ld_d_rt(rdt, p, i);
}

// Output / bias of uncommon dtypes, kept out of line.
__device__ __noinline__ void conv_store_rt(void* Y, int dty, int64_t yi, const void* Bv, int dtb, int m, float acc) {
    const double bias = Bv ? ld_d_rt(dtb, Bv, m) : 0.0;
    st_d_rt(dty, Y, yi, (double)acc + bias);
}

template <int DX, int DW, int YDT>
__global__ __launch_bounds__(256) void k_conv_mfma_f32(const void* __restrict__ X, const void* __restrict__ Wt,
                                                       const void* __restrict__ Bv, int dtb, void* __restrict__ Y,
                                                       int dty, ConvGeom g, int dtx, int dtw) {
    __shared__ float As[2][kCK][kCM + kCPad];
    __shared__ float Bs[2][kCK][kCN + kCPad];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = blockIdx.z;
    const int m0 = blockIdx.y * kCM;                 // within the group
    const int p0 = blockIdx.x * kCN;
    const int OHW = g.OH * g.OW;
    const int P = g.N * OHW;
    const int KHW = g.KH * g.KW;

    // This thread's im2col column.
    const int p = p0 + threadIdx.x;
    const bool pv = p < P;
    const int pn = pv ? p / OHW : 0;
    const int pr = pv ? p - pn * OHW : 0;
    const int poh = pr / g.OW, pow_ = pr - poh * g.OW;
    const int ih0 = poh * g.sh - g.pt, iw0 = pow_ * g.sw - g.pl;
    const int64_t xbase = ((int64_t)pn * g.C + (int64_t)grp * g.Cg) * g.H * g.W;
    const int64_t wbase = ((int64_t)grp * g.Mg) * g.Kg;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    auto stage = [&](int buf, int k0) {
        // Weights: 64 rows (m) x 16 k; thread -> (m = t / 4, 4 consecutive k).
        {
            const int mm = threadIdx.x >> 2, kq = (threadIdx.x & 3) * 4;
            const int gm = m0 + mm;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int gk = k0 + kq + e;
                As[buf][kq + e][mm] = (gm < g.Mg && gk < g.Kg) ? ldf<DW>(Wt, wbase + (int64_t)gm * g.Kg + gk, dtw) : 0.0f;
            }
        }
        // im2col: 16 k x 256 pixels; thread -> its pixel, all 16 k.
        int k = k0;
        int c = k / KHW;
        int rem = k - c * KHW;
        int kh = rem / g.KW, kw = rem - kh * g.KW;
#pragma unroll
        for (int e = 0; e < kCK; e++) {
            float v = 0.0f;
            if (pv && k < g.Kg) {
                const int ih = ih0 + kh * g.dh, iw = iw0 + kw * g.dw;
                if (ih >= 0 && ih < g.H && iw >= 0 && iw < g.W)
                    v = ldf<DX>(X, xbase + ((int64_t)c * g.H + ih) * g.W + iw, dtx);
            }
            Bs[buf][e][threadIdx.x] = v;
            k++;
            if (++kw == g.KW) { kw = 0; if (++kh == g.KH) { kh = 0; c++; } }
        }
    };

    const int nk = (g.Kg + kCK - 1) / kCK;
    stage(0, 0);
    __syncthreads();
    const int lr = lane & 31, lk = lane >> 5;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) stage(cur ^ 1, (kt + 1) * kCK);
#pragma unroll
        for (int ks = 0; ks < kCK; ks += 2) {
            float a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; i++) a[i] = As[cur][ks + lk][i * 32 + lr];
#pragma unroll
            for (int j = 0; j < 2; j++) b[j] = Bs[cur][ks + lk][wave * 64 + j * 32 + lr];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int q = p0 + wave * 64 + j * 32 + lr;
        if (q >= P) continue;
        const int qn = q / OHW, qr = q - qn * OHW;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int mloc = m0 + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
                if (mloc >= g.Mg) continue;
                const int m = grp * g.Mg + mloc;
                const int64_t yi = ((int64_t)qn * g.M + m) * OHW + qr;
                if constexpr (YDT >= 0) {
                    if (!Bv || dtb == kF32) {
                        const double bias = Bv ? (double)((const float*)Bv)[m] : 0.0;
                        st_d<YDT>(Y, yi, (double)acc[i][j][r] + bias);
                        continue;
                    }
                }
                conv_store_rt(Y, dty, yi, Bv, dtb, m, acc[i][j][r]);
            }
    }
}

// ---------------------------------------------------------------- tiled f32 ---
// f32 input and weights.  Implicit GEMM per group: A = weights [Mg, Kg]
// (k = (c, kh, kw), contiguous), B = im2col [Kg, P] gathered on the fly,
// P = N * OH * OW.  Block tile BM channels x BP pixels x BK, NT = 64 * WGM * WGN
// threads, wave tile (BM / WGM) x (BP / WGN) of 32x32 v_mfma_f32_32x32x2f32.
// The next k-tile is loaded into registers (raw buffer loads; a padding tap or
// a k past Kg gets an out-of-range offset and reads zero, so the gather has no
// branches) while the MFMAs run on the current LDS buffer; one barrier per
// k-tile.  MODE 1 is the 1x1 / stride 1 / no padding case with HW % 4 == 0:
// im2col is the input itself, read as float4 along the pixels.
// Epilogue (f32 output, f32 or no bias): acc + bias in fp32, which equals the
// reference's double sum rounded to float (two floats: 53 >= 2 * 24 + 2).
struct ConvTiled {
    int C, H, W, M, KH, KW, OH, OW;
    int pt, pl, sh, sw, dh, dw;
    int Cg, Mg, Kg, HW, OHW, P;
    FastDiv fd_ohw, fd_ow, fd_khw, fd_kw, fd_cg;
};

typedef __attribute__((address_space(1))) float gfloat;

// Fused epilogue of conv2d_fused_forward (f32 output): y = conv + bias, then
// Relu (v > 0 ? v : 0, as relu_forward), then + skip (an f32 tensor of Y's
// shape, as add_forward).  Each step rounds to f32 exactly as the standalone
// operator does, so the result equals the three calls bit for bit.
struct ConvEpi {
    const float* skip;
    int relu;
    FakeQuant fq;   // applied last (kind 0: none)
};
__device__ __forceinline__ float relu_f(float v) { return v > 0.0f ? v : 0.0f; }

// Quantized input of dequantize_conv2d_fused_forward: X holds uint8 (XQ = 1) or
// int8 (XQ = 2) codes with a per-tensor scale and zero point; the gather forms
// (float)(q - z) * s, which is the value DequantizeLinear writes (q - z has at
// most 9 bits, so the fp32 product is the correctly rounded exact product, as
// the reference's double product rounded once).  Padding taps stay 0.
struct ConvXQ {
    const float* s;      // scale (one element)
    const void* z;       // zero point of the codes' dtype (one element), or null for 0
};
template <int XQ> __device__ __forceinline__ float xq_value(uint32_t code, float s, int z) {
    const int c = XQ == 2 ? (int)(int8_t)(uint8_t)code : (int)(code & 0xFFu);
    return (float)(c - z) * s;
}

// SPLIT: gridDim.z = slices * groups, a block's z = slice * groups + group
// (from its work index, below); slice s covers k in
// [s * kchunk, (s + 1) * kchunk) (kchunk a multiple of BK) and stores its raw
// fp32 sums, without bias, to Y + s * N * M * OH * OW (Y is then the f32
// workspace); k_conv_splitk_reduce adds the slices in order with the bias.
// XQ: 0 f32 input; 1 / 2 uint8 / int8 codes dequantised in the gather (ConvXQ).
// MODE 0: k = (c, kh, kw) as the weights store it, one gathered element per
// (pixel, k) with its own padding test.  MODE 1: 1x1 stride-1 layers, four
// pixels per float4.  MODE 2 (Cg a multiple of BK): k runs in (channel block
// of BK, kh, kw, channel) order, so a k-tile holds BK channels of one tap; the
// padding test and the pixel's address are computed once per tile and each channel is one load
// with a wave-uniform scalar offset (c * H * W).  Its LDS tiles keep k
// contiguous ([row][k]), and lane half h feeds MFMA step s with k = h*BK/2 + s,
// so each operand is read as 16-byte vectors covering four steps.  DEPTH 2
// (MODE 2 only) keeps a second loaded tile in registers.  DEPTH 3 (MODE 2
// only) is the store-first pipeline: at the top of k-tile k the registers of
// tile k + 1 (loaded one whole k-tile earlier) go to the idle LDS buffer and the
// loads of tile k + 2 are issued, interleaved with the MFMAs; each 4-step
// sub-step's fragments are read one sub-step ahead; the barrier sits between
// the two halves of the last sub-step, and the next tile's first fragments are
// read right after it, under the second half's MFMAs.  Same k order and MFMA
// sequence as DEPTH 1 / 2, so the same bits.
template <int BM, int BP, int BK, int WGM, int WGN, int MODE, int YDT, bool SPLIT = false, int XQ = 0, int DEPTH = 1>
__global__ __launch_bounds__(64 * WGM * WGN) void k_conv_tiled(const float* __restrict__ X, const float* __restrict__ Wt,
                                                               const float* __restrict__ Bv, void* __restrict__ Y,
                                                               int dty, int dtb, ConvTiled g, uint32_t xbytes,
                                                               uint32_t wbytes, uint32_t ybytes, ConvEpi epi,
                                                               ConvXQ xq, int kchunk = 0, int groups = 1) {
    constexpr uint32_t XES = XQ ? 1u : 4u;        // bytes per input element
    float xs = 1.0f;
    int xz = 0;
    if constexpr (XQ != 0) {
        xs = xq.s[0];
        xz = xq.z ? (XQ == 2 ? (int)((const int8_t*)xq.z)[0] : (int)((const uint8_t*)xq.z)[0]) : 0;
    }
    constexpr int NT = 64 * WGM * WGN;
    constexpr int WTM = BM / WGM, WTP = BP / WGN, TM = WTM / 32, TP = WTP / 32;
    constexpr int EA = BM * BK / NT;              // weights per thread per k-tile (consecutive k)
    constexpr int EB = BK * BP / NT;              // im2col values per thread per k-tile
    static_assert(EA >= 1 && BK % EA == 0 && EB >= 1, "tile / thread mismatch");
    constexpr bool TAP = MODE == 2;
    static_assert(!TAP || BK % 8 == 0, "MODE 2 reads four k per lane half and vector");
    static_assert(DEPTH == 1 || (TAP && (DEPTH == 2 || DEPTH == 3)), "DEPTH 2 / 3 are MODE 2 options");
    // MODE 0 / 1: [k][row]; MODE 2: [row][k] (rows of BK + 4 floats: 16-byte
    // reads and writes of consecutive rows fall in distinct bank groups)
    __shared__ float As[2][TAP ? BM : BK][TAP ? BK + 4 : BM + 4];
    __shared__ float Bs[2][TAP ? BP : BK][TAP ? BK + 4 : BP + 4];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    // Tile order: the dispatcher deals consecutive workgroups (linear index L
    // over x, y, z) to the 8 XCDs in turn, each with its own L2, so L becomes a
    // work index w that gives XCD class L % 8 a contiguous run of the whole
    // grid, ordered (z, pixel tile, channel tile) with the channel tile
    // fastest: the channel tiles of one pixel tile share their input through
    // one L2, and an XCD's run spans one or two k-slices of a split layer, so
    // it fetches only those slices' weights (per-z runs had every XCD fetch
    // every slice's weights).  A bijection on [0, blocks) for any count.
    int grp, slice, m0, p0;
    {
        const int ntm = (int)gridDim.y, tiles = (int)gridDim.x * ntm, total = tiles * (int)gridDim.z;
        const int L = (int)blockIdx.x + ((int)blockIdx.y + (int)blockIdx.z * ntm) * (int)gridDim.x;
        const int cls = L & 7, q = total >> 3, rem = total & 7;
        const int w = cls * q + min(cls, rem) + (L >> 3);
        const int z = w / tiles, tid = w - z * tiles;
        grp = SPLIT ? z % groups : z;
        slice = SPLIT ? z / groups : 0;
        const int tp = tid / ntm;
        m0 = (tid - tp * ntm) * BM;
        p0 = tp * BP;
    }
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X, xbytes);
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(Wt, wbytes);

    // weights: thread -> row am, EA consecutive k from ak
    const int am = t / (BK / EA), ak = (t % (BK / EA)) * EA;
    const int wrow = grp * g.Mg + m0 + am;
    const bool am_ok = m0 + am < g.Mg;

    // im2col: MODE 0 -> one pixel, KPT consecutive k; MODE 1 -> 4 pixels, KPT k.
    // In MODE 0 a thread's k range (kg) is the same across its wave (PCOLS is
    // a multiple of 64), so the (c, kh, kw) decode runs on scalar registers and
    // a gathered element costs two adds, two compares and a select.
    constexpr int PPT = MODE == 1 ? 4 : 1;
    constexpr int KPT = EB / PPT;
    constexpr int PCOLS = BP / PPT;
    static_assert(MODE == 1 || PCOLS % 64 == 0, "a wave must share its k range");
    static_assert(KPT >= 1 && KPT * PPT == EB, "every thread loads at least one k per tile");
    const int pc = (t % PCOLS) * PPT;
    const int kg = MODE != 1 ? __builtin_amdgcn_readfirstlane((t / PCOLS) * KPT) : (t / PCOLS) * KPT;
    const int p = p0 + pc;
    int ih0 = -(1 << 29), iw0 = 0, pix = 0;
    if (p < g.P) {
        const int n = (int)g.fd_ohw.div((uint32_t)p), r = p - n * g.OHW;
        const int oh = (int)g.fd_ow.div((uint32_t)r), ow = r - oh * g.OW;
        ih0 = oh * g.sh - g.pt;
        iw0 = ow * g.sw - g.pl;
        // element offset of tap (c = 0, kh = 0, kw = 0); in bounds only for valid taps
        pix = (n * g.C + grp * g.Cg) * g.HW + (MODE == 1 ? r : ih0 * g.W + iw0);
    }

    // Tiles never straddle a slice boundary, so masking against kend stays exact.
    const int kbeg = SPLIT ? slice * kchunk : 0;
    const int kend = SPLIT ? min(g.Kg, kbeg + kchunk) : g.Kg;
    const int nk = (kend - kbeg + BK - 1) / BK;
    float ra[EA];
    float rb[EB];
    auto load_tile = [&](int k0) {
#pragma unroll
        for (int e = 0; e < EA; e++) {
            const int k = k0 + ak + e;
            const uint32_t off = (am_ok && k < kend) ? (uint32_t)(wrow * g.Kg + k) * 4u : kOOB;
            ra[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wr, off, 0, 0));
        }
        if constexpr (MODE == 1) {
#pragma unroll
            for (int e = 0; e < KPT; e++) {
                const int k = k0 + kg + e;
                const bool ok = ih0 >= 0 && k < kend;
                const uint32_t off = ok ? (uint32_t)(pix + k * g.HW) * XES : kOOB;
                if constexpr (XQ) {
                    // four codes of four consecutive pixels in one word
                    const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(xr, off, 0, 0);
#pragma unroll
                    for (int q = 0; q < 4; q++) rb[e * 4 + q] = ok ? xq_value<XQ>(w >> (8 * q), xs, xz) : 0.0f;
                } else {
                    typedef unsigned int u32x4 __attribute__((__vector_size__(16)));
                    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        // element copied to a scalar first: hipcc 7.2 folds
                        // __builtin_bit_cast of a vector subscript to element 0
                        const uint32_t u = v[q];
                        rb[e * 4 + q] = __builtin_bit_cast(float, u);
                    }
                }
            }
        } else {
            int k = k0 + kg;
            int c = (int)g.fd_khw.div((uint32_t)k);
            const int rem = k - c * (g.KH * g.KW);
            int kh = (int)g.fd_kw.div((uint32_t)rem);
            int kw = rem - kh * g.KW;
#pragma unroll
            for (int e = 0; e < KPT; e++) {
                const int sdh = kh * g.dh, sdw = kw * g.dw;
                const int koff = c * g.HW + sdh * g.W + sdw;
                const bool ok = k < kend && (unsigned)(ih0 + sdh) < (unsigned)g.H && (unsigned)(iw0 + sdw) < (unsigned)g.W;
                const uint32_t off = ok ? (uint32_t)(pix + koff) * XES : kOOB;
                if constexpr (XQ) rb[e] = ok ? xq_value<XQ>(__builtin_amdgcn_raw_buffer_load_b8(xr, off, 0, 0), xs, xz) : 0.0f;
                else rb[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, off, 0, 0));
                k++;
                if (++kw == g.KW) { kw = 0; if (++kh == g.KH) { kh = 0; c++; } }
            }
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int e = 0; e < EA; e++) As[buf][ak + e][am] = ra[e];
        if constexpr (MODE == 1) {
#pragma unroll
            for (int e = 0; e < KPT; e++)
                *reinterpret_cast<float4*>(&Bs[buf][kg + e][pc]) = make_float4(rb[4 * e], rb[4 * e + 1], rb[4 * e + 2],
                                                                                rb[4 * e + 3]);
        } else {
#pragma unroll
            for (int e = 0; e < KPT; e++) Bs[buf][kg + e][pc] = rb[e];
        }
    };

    floatx16 acc[TM][TP];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TP; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int lr = lane & 31, lk = lane >> 5;
    auto compute = [&](int buf) {
#pragma unroll
        for (int ks = 0; ks < BK; ks += 2) {
            float a[TM], b[TP];
#pragma unroll
            for (int i = 0; i < TM; i++) a[i] = As[buf][ks + lk][wm * WTM + i * 32 + lr];
#pragma unroll
            for (int j = 0; j < TP; j++) b[j] = Bs[buf][ks + lk][wn * WTP + j * 32 + lr];
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TP; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };

    // MODE 0: the next tile's gather is interleaved with this tile's MFMA
    // steps (KPT / (BK / 2) elements after each k-pair), so the wave issues its
    // address arithmetic while the matrix core works.
    struct Gather { int k, c, kh, kw; };
    auto gather_start = [&](int k0) {
        Gather q;
        q.k = k0 + kg;
        q.c = (int)g.fd_khw.div((uint32_t)q.k);
        const int rem = q.k - q.c * (g.KH * g.KW);
        q.kh = (int)g.fd_kw.div((uint32_t)rem);
        q.kw = rem - q.kh * g.KW;
        return q;
    };
    // kend bounds the loads: k at or past the end of this block's k range
    // reads zero through the out-of-range offset.
    auto gather_one = [&](Gather& q, float (&dst)[EB], int e) {
        const int sdh = q.kh * g.dh, sdw = q.kw * g.dw;
        const int koff = q.c * g.HW + sdh * g.W + sdw;
        const bool ok = q.k < kend && (unsigned)(ih0 + sdh) < (unsigned)g.H && (unsigned)(iw0 + sdw) < (unsigned)g.W;
        const uint32_t off = ok ? (uint32_t)(pix + koff) * XES : kOOB;
        if constexpr (XQ) dst[e] = ok ? xq_value<XQ>(__builtin_amdgcn_raw_buffer_load_b8(xr, off, 0, 0), xs, xz) : 0.0f;
        else dst[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, off, 0, 0));
        q.k++;
        if (++q.kw == g.KW) { q.kw = 0; if (++q.kh == g.KH) { q.kh = 0; q.c++; } }
    };
    auto load_weights = [&](int k0, float (&dst)[EA]) {
#pragma unroll
        for (int e = 0; e < EA; e++) {
            const int k = k0 + ak + e;
            const uint32_t off = (am_ok && k < kend) ? (uint32_t)(wrow * g.Kg + k) * 4u : kOOB;
            dst[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wr, off, 0, 0));
        }
    };
    auto compute_and_gather = [&](int buf, int k1, float (&da)[EA], float (&db)[EB]) {
        constexpr int PER = (KPT + BK / 2 - 1) / (BK / 2);
        Gather q = gather_start(k1);
        load_weights(k1, da);
#pragma unroll
        for (int ks = 0; ks < BK; ks += 2) {
            float a[TM], b[TP];
#pragma unroll
            for (int i = 0; i < TM; i++) a[i] = As[buf][ks + lk][wm * WTM + i * 32 + lr];
#pragma unroll
            for (int j = 0; j < TP; j++) b[j] = Bs[buf][ks + lk][wn * WTP + j * 32 + lr];
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TP; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int e = (ks / 2) * PER; e < (ks / 2 + 1) * PER; e++)
                if (e < KPT) gather_one(q, db, e);
        }
    };

    // MODE 2 tile k0 / BK = cb * KH*KW + tap: channels [cb*BK, cb*BK + BK) of
    // tap (kh, kw), so the KH*KW tiles of a channel block run back to back
    // over the same input rows.  Weights W[m][c][tap], input
    // X[n][c][ih0 + kh*dh][iw0 + kw*dw].
    // Lanes of rows past Mg get the out-of-range base; adding a tile offset
    // (< 2^31) keeps it out of range.
    const uint32_t wtap = am_ok ? (uint32_t)(wrow * g.Kg + ak * (g.KH * g.KW)) * 4u : kOOB;
    auto tap_load = [&](int k0, float (&da)[EA], float (&db)[EB]) {
        k0 = min(k0, kend - 1) / BK * BK;     // DEPTH 2 prefetch past the end: reload the last tile (unused)
        const int khw = g.KH * g.KW;
        const int kt0 = k0 / BK;
        const int cb = (int)g.fd_khw.div((uint32_t)kt0);
        const int tap = kt0 - cb * khw;
        const int c0 = cb * BK;
        const int kh = (int)g.fd_kw.div((uint32_t)tap), kw = tap - kh * g.KW;
#pragma unroll
        for (int e = 0; e < EA; e++) {
            const uint32_t wuni = (uint32_t)((c0 + e) * khw + tap) * 4u;   // wave-uniform
            da[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wr, wtap + wuni, 0, 0));
        }
        const int sdh = kh * g.dh, sdw = kw * g.dw;
        const bool ok = (unsigned)(ih0 + sdh) < (unsigned)g.H && (unsigned)(iw0 + sdw) < (unsigned)g.W;
        const uint32_t voff = ok ? (uint32_t)(pix + sdh * g.W + sdw) * XES : kOOB;
#pragma unroll
        for (int e = 0; e < KPT; e++) {
            const uint32_t soff = (uint32_t)((c0 + kg + e) * g.HW) * XES;   // wave-uniform
            if constexpr (XQ)
                db[e] = ok ? xq_value<XQ>(__builtin_amdgcn_raw_buffer_load_b8(xr, voff, soff, 0), xs, xz) : 0.0f;
            else
                db[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, voff, soff, 0));
        }
        // keep the loads ahead of the MFMA steps that follow (DEPTH 3
        // interleaves them with the MFMAs instead)
        if constexpr (DEPTH != 3) __builtin_amdgcn_sched_barrier(0);
    };
    auto tap_store = [&](int buf, const float (&sa)[EA], const float (&sb)[EB]) {
#pragma unroll
        for (int e = 0; e < EA; e++) As[buf][am][ak + e] = sa[e];
        if constexpr (KPT % 4 == 0) {
#pragma unroll
            for (int e = 0; e < KPT; e += 4)
                *reinterpret_cast<float4*>(&Bs[buf][pc][kg + e]) = make_float4(sb[e], sb[e + 1], sb[e + 2], sb[e + 3]);
        } else {
#pragma unroll
            for (int e = 0; e < KPT; e++) Bs[buf][pc][kg + e] = sb[e];
        }
    };
    auto tap_compute = [&](int buf) {
#pragma unroll
        for (int j = 0; j < BK / 8; j++) {
            typedef float f32x4 __attribute__((ext_vector_type(4)));
            f32x4 a4[TM], b4[TP];
#pragma unroll
            for (int i = 0; i < TM; i++)
                a4[i] = *reinterpret_cast<const f32x4*>(&As[buf][wm * WTM + i * 32 + lr][lk * (BK / 2) + 4 * j]);
#pragma unroll
            for (int jj = 0; jj < TP; jj++)
                b4[jj] = *reinterpret_cast<const f32x4*>(&Bs[buf][wn * WTP + jj * 32 + lr][lk * (BK / 2) + 4 * j]);
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int jj = 0; jj < TP; jj++)
                        acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[i][q], b4[jj][q], acc[i][jj], 0, 0, 0);
        }
    };

    int kt = 0;
    if constexpr (TAP && DEPTH == 3) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        constexpr int NS = BK / 8;                  // 4-step sub-steps per k-tile
        constexpr int NM = 4 * TM * TP;             // MFMAs per sub-step
        constexpr int NLD = EA + KPT, NWR = EA + KPT / 4, NRD = TM + TP;
        constexpr int PRE = 2;                      // steps of the last sub-step ahead of the barrier
        f32x4 fa[2][TM], fb[2][TP];
        auto fread = [&](int buf, int j, int f) {
#pragma unroll
            for (int i = 0; i < TM; i++)
                fa[f][i] = *reinterpret_cast<const f32x4*>(&As[buf][wm * WTM + i * 32 + lr][lk * (BK / 2) + 4 * j]);
#pragma unroll
            for (int jj = 0; jj < TP; jj++)
                fb[f][jj] = *reinterpret_cast<const f32x4*>(&Bs[buf][wn * WTP + jj * 32 + lr][lk * (BK / 2) + 4 * j]);
        };
        auto mf = [&](int f, int qlo, int qhi) {
#pragma unroll
            for (int q = qlo; q < qhi; q++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int jj = 0; jj < TP; jj++)
                        acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[f][i][q], fb[f][jj][q], acc[i][jj], 0, 0, 0);
        };
        tap_load(kbeg, ra, rb);
        tap_store(0, ra, rb);
        tap_load(kbeg + BK, ra, rb);                // past the end: the last tile again (unused)
        __syncthreads();
        fread(0, 0, 0);
        for (; kt < nk; kt++) {
            const int cur = kt & 1;
#pragma unroll
            for (int s = 0; s < NS - 1; s++) {
                fread(cur, s + 1, (s + 1) & 1);
                if (s == 0) {
                    tap_store(cur ^ 1, ra, rb);     // tile k + 1 (past the end: an unused copy)
                    tap_load(kbeg + (kt + 2) * BK, ra, rb);
                }
                mf(s & 1, 0, 4);
                // sched_group_barrier masks: MFMA 0x008, DS read 0x100, DS write
                // 0x200, VMEM read 0x020
#pragma unroll
                for (int q = 0; q < NM; q++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if (q < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    if (s == 0) {
                        __builtin_amdgcn_sched_group_barrier(0x200, (NWR + NM - 1) / NM, 0);
                        __builtin_amdgcn_sched_group_barrier(0x020, (NLD + NM - 1) / NM, 0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            mf((NS - 1) & 1, 0, PRE);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
            fread(cur ^ 1, 0, 0);
            mf((NS - 1) & 1, PRE, 4);
            __builtin_amdgcn_sched_barrier(0);
        }
    } else if constexpr (TAP) {
        // Two tiles per trip with fixed LDS buffers: tile kt (even) sits in
        // buffer 0 at the top of each trip.  DEPTH 2 keeps tile kt + 1 in a
        // second register set, loaded one trip earlier.
        float ra2[EA], rb2[EB];
        tap_load(kbeg, ra, rb);
        tap_store(0, ra, rb);
        if constexpr (DEPTH == 2) tap_load(kbeg + BK, ra2, rb2);
        __syncthreads();
        for (; kt + 2 < nk; kt += 2) {
            if constexpr (DEPTH == 2) {
                tap_load(kbeg + (kt + 2) * BK, ra, rb);
                tap_compute(0);
                tap_store(1, ra2, rb2);
                __syncthreads();
                tap_load(kbeg + (kt + 3) * BK, ra2, rb2);
                tap_compute(1);
                tap_store(0, ra, rb);
                __syncthreads();
            } else {
                tap_load(kbeg + (kt + 1) * BK, ra, rb);
                tap_compute(0);
                tap_store(1, ra, rb);
                __syncthreads();
                tap_load(kbeg + (kt + 2) * BK, ra, rb);
                tap_compute(1);
                tap_store(0, ra, rb);
                __syncthreads();
            }
        }
        if (kt + 1 < nk) {
            if constexpr (DEPTH != 2) tap_load(kbeg + (kt + 1) * BK, ra2, rb2);
            tap_compute(0);
            tap_store(1, ra2, rb2);
            __syncthreads();
            tap_compute(1);
        } else {
            tap_compute(0);
        }
    } else {
        load_tile(kbeg);
        store_tile(0);
        __syncthreads();
        for (; kt + 1 < nk; kt++) {
            if constexpr (MODE == 0) {
                compute_and_gather(kt & 1, kbeg + (kt + 1) * BK, ra, rb);
            } else {
                load_tile(kbeg + (kt + 1) * BK);
                compute(kt & 1);
            }
            store_tile((kt & 1) ^ 1);
            __syncthreads();
        }
        compute(kt & 1);
    }

    // Output row m of the 32x32 tile (i, j), register r: m = mw + i*32 + 8*(r/4) + (r%4) + 4*lk,
    // pixel q = qw + j*32 + lr.
    const int mw = m0 + wm * WTM;
    if constexpr (SPLIT) {
        gfloat* part = (gfloat*)Y + (int64_t)slice * g.P * g.M;
#pragma unroll
        for (int j = 0; j < TP; j++) {
            const int q = p0 + wn * WTP + j * 32 + lr;
            if (q >= g.P) continue;
            const int qn = (int)g.fd_ohw.div((uint32_t)q), qr = q - qn * g.OHW;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int mloc = mw + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
                    if (mloc < g.Mg) part[((int64_t)qn * g.M + grp * g.Mg + mloc) * g.OHW + qr] = acc[i][j][r];
                }
        }
        return;
    }
    if (YDT == kF32 && mw + WTM <= g.Mg) {
        // Raw buffer stores: per-lane byte offset of (m = mw + 4*lk, pixel q) plus
        // a uniform offset for the tile row, so the 16 x TM x TP stores need no
        // address arithmetic.
        const __amdgpu_buffer_rsrc_t yr = buffer_rsrc(Y, ybytes);
        const __amdgpu_buffer_rsrc_t zr = buffer_rsrc(epi.skip, epi.skip ? ybytes : 0u);
        FQParm fqp;
        if (epi.fq.kind) fqp = fq_parm(epi.fq);
        float bv[TM][16];
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                bv[i][r] = Bv ? ((const gfloat*)Bv)[grp * g.Mg + mw + i * 32 + 8 * (r >> 2) + (r & 3) + 4 * lk] : 0.0f;
        if constexpr (TAP) {
            // Pixels past P get the out-of-range offset: their loads read zero
            // and their stores are dropped.  The skip values of each 32x32
            // tile are loaded before its first store, so those loads are not
            // ordered behind the stores (Y and Skip may alias as far as the
            // compiler knows).
#pragma unroll
            for (int j = 0; j < TP; j++) {
                const int q = p0 + wn * WTP + j * 32 + lr;
                const int qn = (int)g.fd_ohw.div((uint32_t)q), qr = q - qn * g.OHW;
                const uint32_t vo =
                    q < g.P ? (uint32_t)((qn * g.M + grp * g.Mg + mw + 4 * lk) * g.OHW + qr) * 4u : kOOB;
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    float sk[16];
                    if (epi.skip) {
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const uint32_t so = (uint32_t)((i * 32 + 8 * (r >> 2) + (r & 3)) * g.OHW) * 4u;
                            sk[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(zr, vo, so, 0));
                        }
                    }
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const uint32_t so = (uint32_t)((i * 32 + 8 * (r >> 2) + (r & 3)) * g.OHW) * 4u;
                        float v = acc[i][j][r] + bv[i][r];
                        if (epi.relu) v = relu_f(v);
                        if (epi.skip) v += sk[r];
                        if (epi.fq.kind) v = fq_apply(v, fqp);
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), yr, vo, so, 0);
                    }
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < TP; j++) {
                const int q = p0 + wn * WTP + j * 32 + lr;
                if (q < g.P) {
                    const int qn = (int)g.fd_ohw.div((uint32_t)q), qr = q - qn * g.OHW;
                    const uint32_t vo = (uint32_t)((qn * g.M + grp * g.Mg + mw + 4 * lk) * g.OHW + qr) * 4u;
#pragma unroll
                    for (int i = 0; i < TM; i++)
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const uint32_t so = (uint32_t)((i * 32 + 8 * (r >> 2) + (r & 3)) * g.OHW) * 4u;
                            // + 0.0f without a bias, as the reference adds bias_val = 0.0 (-0 -> +0)
                            float v = acc[i][j][r] + bv[i][r];
                            if (epi.relu) v = relu_f(v);
                            if (epi.skip)
                                v += __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(zr, vo, so, 0));
                            if (epi.fq.kind) v = fq_apply(v, fqp);
                            // MODE 1: nontemporal (config-4 1x1 46.5 -> 43.5 us).  The MODE 2
                            // and stem epilogues keep cached stores: with nontemporal ones the
                            // config-5 graph, whose next layer re-reads each output, ran 1.6%
                            // slower (0.740 -> 0.752 ms) for 1-2% on the standalone layers.
                            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), yr, vo, so,
                                                                  MODE == 1 ? 2 /* nt */ : 0);
                        }
                }
            }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < TP; j++) {
        const int q = p0 + wn * WTP + j * 32 + lr;
        if (q >= g.P) continue;
        const int qn = (int)g.fd_ohw.div((uint32_t)q), qr = q - qn * g.OHW;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int mloc = mw + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
                if (mloc >= g.Mg) continue;
                const int m = grp * g.Mg + mloc;
                const int64_t yi = ((int64_t)qn * g.M + m) * g.OHW + qr;
                if constexpr (YDT == kF32) {
                    float v = acc[i][j][r] + (Bv ? ((const gfloat*)Bv)[m] : 0.0f);
                    if (epi.relu) v = relu_f(v);
                    if (epi.skip) v += ((const gfloat*)epi.skip)[yi];
                    if (epi.fq.kind) v = fq_apply(v, fq_parm(epi.fq));
                    ((gfloat*)Y)[yi] = v;
                } else {
                    conv_store_rt(Y, dty, yi, Bv, dtb, m, acc[i][j][r]);
                }
            }
    }
}

// Few-channel convolution (the 7x7 / stride-2 stem over 3 channels): a block
// computes 64 output channels x 256 consecutive output pixels of one image with
// the whole k range resident in LDS, loaded once: the weights as [channel][k]
// and, for each input channel, the input rows the pixels touch with the zero
// halo of the padding.  k runs in the reference's (c, kh, kw) order and is
// unrolled at compile time, so each MFMA operand is one LDS read at a per-lane
// base plus an immediate offset: no address arithmetic, bounds tests or
// barriers inside the k loop.  v_mfma_f32_32x32x1f32 takes one k per step for
// two 32x32 blocks (lanes 0-31 and 32-63), which here are the same 32 output
// channels over two 32-pixel groups: a 32x64 wave tile per instruction, and no
// padded k slots (a padded slot would multiply a zero weight by a real, possibly
// non-finite, input).  Output register r of lane l: block r / 16, channel
// 8*((r%16)/4) + r%4 + 4*(l/32), pixel l%32 of that block's group.  ONE_M (one
// channel tile): the weights go to LDS once per block and each kh row's
// operands are read while the row before it is multiplied; DEFER (ONE_M
// without a residual): a tile's outputs are stored during the next tile's
// multiply.
constexpr int kStemRows = 13, kStemCols = 232;   // LDS patch per input channel: rows x columns
template <int C, int KH, int KW, int S, bool ONE_M, bool DEFER>
__global__ __launch_bounds__(512, 4) void k_conv_stem(const float* __restrict__ X, const float* __restrict__ Wt,
                                                   const float* __restrict__ Bv, float* __restrict__ Y, ConvTiled g,
                                                   int tiles_per_img, int ntm, int tiles, uint32_t xbytes,
                                                   uint32_t wbytes, uint32_t ybytes, ConvEpi epi) {
    typedef float floatx32 __attribute__((ext_vector_type(32)));
    constexpr int BM = 64, BP = 256, WGN = 4, K = C * KH * KW, KA = K + (K % 2 == 0 ? 1 : 2);   // odd row pitch
    constexpr int PRM = kStemRows, PCM = kStemCols, PATCH = C * PRM * PCM;
    __shared__ float As[BM * KA];
    __shared__ float Ps[PATCH];
    __shared__ float Bs[BM];
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6), lr = lane & 31,
              lk = lane >> 5;
    const int wm = wave / WGN, wn = wave % WGN, pw = wn * 64;
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X, xbytes);
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(Wt, wbytes);
    const __amdgpu_buffer_rsrc_t yr = buffer_rsrc(Y, ybytes);
    const __amdgpu_buffer_rsrc_t zr = buffer_rsrc(epi.skip, epi.skip ? ybytes : 0u);

    // Persistent blocks: block b takes tile slots b, b + G, b + 2G, ... (G =
    // gridDim.x, a multiple of 8, so one XCD); a slot maps to a tile with the
    // k_conv_tiled order (each XCD class a contiguous run, channel tile fastest).
    struct Tile { int m0, n, q0, ih_lo; };
    auto tile_of = [&](int slot) {
        const int cls = slot & 7, q = tiles >> 3, rem = tiles & 7;
        const int tid = cls * q + min(cls, rem) + (slot >> 3);
        const int tp = tid / ntm;
        Tile T;
        T.m0 = (tid - tp * ntm) * BM;
        T.n = tp / tiles_per_img;
        T.q0 = (tp - T.n * tiles_per_img) * BP;
        T.ih_lo = (int)g.fd_ow.div((uint32_t)T.q0) * S - g.pt;
        return T;
    };
    // A tile's operands: weights [m][k] (rows past Mg read zero) and the input
    // patch [c][row][col] (row r <-> input row ih_lo + r, col <-> column col - pl).
    // Wave w moves rows w, w + 8, ... (a wave-uniform row index: its address
    // math is scalar), lanes move columns lane, lane + 64, ...: a thread keeps
    // only the loaded values across the multiply.
    constexpr int NW = 8, WROWS = BM / NW, WCOLJ = (K + 63) / 64;
    constexpr int PROWS = C * PRM, PRW = (PROWS + NW - 1) / NW, PCOLJ = (PCM + 63) / 64;
    float wv[WROWS][WCOLJ], pv[PRW][PCOLJ], bv = 0.0f;
    auto load_w = [&](const Tile& T) {
        if (t < BM) bv = (Bv && T.m0 + t < g.Mg) ? Bv[T.m0 + t] : 0.0f;
#pragma unroll
        for (int i = 0; i < WROWS; i++) {
            const int m = wave + i * NW;
            const bool mok = T.m0 + m < g.Mg;
#pragma unroll
            for (int j = 0; j < WCOLJ; j++) {
                const int k = lane + 64 * j;
                const uint32_t off = (mok && k < K) ? (uint32_t)((T.m0 + m) * K + k) * 4u : kOOB;
                wv[i][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wr, off, 0, 0));
            }
        }
    };
    auto load_p = [&](const Tile& T) {
#pragma unroll
        for (int i = 0; i < PRW; i++) {
            const int row = wave + i * NW;
            const int c = row / PRM, ih = T.ih_lo + (row - c * PRM);
            const bool rok = row < PROWS && (unsigned)ih < (unsigned)g.H;
#pragma unroll
            for (int j = 0; j < PCOLJ; j++) {
                const int col = lane + 64 * j, iw = col - g.pl;
                const bool ok = rok && col < PCM && (unsigned)iw < (unsigned)g.W;
                const uint32_t off = ok ? (uint32_t)(((T.n * C + c) * g.H + ih) * g.W + iw) * 4u : kOOB;
                pv[i][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, off, 0, 0));
            }
        }
    };
    auto store_w = [&]() {
        if (t < BM) Bs[t] = bv;
#pragma unroll
        for (int i = 0; i < WROWS; i++)
#pragma unroll
            for (int j = 0; j < WCOLJ; j++) {
                const int k = lane + 64 * j;
                if (k < K) As[(wave + i * NW) * KA + k] = wv[i][j];
            }
    };
    auto store_p = [&]() {
#pragma unroll
        for (int i = 0; i < PRW; i++)
#pragma unroll
            for (int j = 0; j < PCOLJ; j++) {
                const int row = wave + i * NW, col = lane + 64 * j;
                if (row < PROWS && col < PCM) Ps[row * PCM + col] = pv[i][j];
            }
    };

    int slot = blockIdx.x;
    if (slot >= tiles) return;
    Tile T = tile_of(slot);
    load_w(T);
    load_p(T);
    store_w();
    store_p();
    __syncthreads();
    const float* pa = &As[(wm * 32 + lr) * KA];
    // DEFER (one channel tile, no residual): a tile's 32 outputs per lane stay in
    // registers and are stored during the next tile's first kh rows, so the
    // stores (64 KB per tile, issued by every block at once otherwise) overlap
    // the MFMAs; the next tile's patch loads are issued half way through the
    // multiply, after those registers are free.
    static_assert(!DEFER || ONE_M, "DEFER needs the one-channel-tile form");
    float outv[32];
    uint32_t obase[2] = {kOOB, kOOB};
    int omlim = 0;
    bool have_out = false;
    auto store_out = [&](int idx) {
        const int b = idx >> 4, r = idx & 15, cr = 8 * (r >> 2) + (r & 3);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, outv[idx]), yr,
                                              cr < omlim ? obase[b] : kOOB, cr * g.OHW * 4, 0);
    };
    float bias_r[16];
    if constexpr (ONE_M && !DEFER) {
#pragma unroll
        for (int r = 0; r < 16; r++) bias_r[r] = Bs[wm * 32 + 8 * (r >> 2) + (r & 3) + 4 * lk];
    }
    while (true) {
        // the next tile's operands go to registers while this one is multiplied
        // (with one channel tile, ONE_M, the weights stay in LDS from the start)
        const int next = slot + (int)gridDim.x;
        Tile Tn = T;
        if (next < tiles) {
            Tn = tile_of(next);
            if (!ONE_M) load_w(Tn);
            if (!DEFER) load_p(Tn);
        }
        const int q = min(T.q0 + pw + lk * 32 + lr, g.OHW - 1);
        const int oh = (int)g.fd_ow.div((uint32_t)q), ow = q - oh * g.OW;
        const float* pb = &Ps[(oh * S - g.pt - T.ih_lo) * PCM + ow * S];
        floatx32 acc;
#pragma unroll
        for (int r = 0; r < 32; r++) acc[r] = 0.0f;
        // k = (c, kh, kw).  Without the next tile's weights in registers (ONE_M),
        // unrolled: each row of KW taps' operands is read from LDS while the row
        // before it is multiplied.  Otherwise one rolled trip per input channel
        // (bounded read-ahead, so the next tile's operands fit beside it).
        if constexpr (!ONE_M) {
#pragma nounroll
            for (int c = 0; c < C; c++) {
                const float* ac = pa + c * KH * KW;
                const float* bc = pb + c * PRM * PCM;
#pragma unroll
                for (int kh = 0; kh < KH; kh++)
#pragma unroll
                    for (int kw = 0; kw < KW; kw++)
                        acc = __builtin_amdgcn_mfma_f32_32x32x1f32(ac[kh * KW + kw], bc[kh * PCM + kw], acc, 0, 0, 0);
            }
        } else {
        float ra[2][KW], rb[2][KW];
#pragma unroll
        for (int kw = 0; kw < KW; kw++) {
            ra[0][kw] = pa[kw];
            rb[0][kw] = pb[kw];
        }
#pragma unroll
        for (int row = 0; row < C * KH; row++) {
            const int cur = row & 1;
            if constexpr (DEFER) {
                if (row == (C * KH) / 2 && next < tiles) load_p(Tn);
                if (row < 8 && have_out) {
#pragma unroll
                    for (int u = 0; u < 4; u++) store_out(4 * row + u);
                }
            }
            if (row + 1 < C * KH) {
                const int c1 = (row + 1) / KH, kh1 = (row + 1) % KH;
#pragma unroll
                for (int kw = 0; kw < KW; kw++) {
                    ra[cur ^ 1][kw] = pa[c1 * KH * KW + kh1 * KW + kw];
                    rb[cur ^ 1][kw] = pb[c1 * PRM * PCM + kh1 * PCM + kw];
                }
            }
            // keep the scheduler from sinking those reads next to their MFMAs
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kw = 0; kw < KW; kw++)
                acc = __builtin_amdgcn_mfma_f32_32x32x1f32(ra[cur][kw], rb[cur][kw], acc, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        }

        // epilogue (f32 output): bias, Relu, residual; pixels past the image and
        // channels past Mg take the out-of-range offset (loads zero, stores
        // dropped); residual values loaded four at a time ahead of their stores.
        // With one channel tile the bias values sit in registers, and a lane's 16
        // channels of a pixel differ by a wave-uniform offset (the scalar offset
        // operand), so each output costs the bias add, the Relu and its store.
        if constexpr (DEFER) {
            const int chan = wm * 32 + 4 * lk;
            omlim = g.Mg - chan;
#pragma unroll
            for (int b = 0; b < 2; b++) {
                const int qq = T.q0 + pw + b * 32 + lr;
                obase[b] = qq < g.OHW ? (uint32_t)(((T.n * g.M + chan) * g.OHW + qq) * 4) : kOOB;
            }
#pragma unroll
            for (int i = 0; i < 32; i++) {
                const int r = i & 15;
                // + 0.0f without a bias, as the reference adds bias_val = 0.0 (-0 -> +0)
                float v = acc[i] + Bs[wm * 32 + 8 * (r >> 2) + (r & 3) + 4 * lk];
                if (epi.relu) v = relu_f(v);
                outv[i] = v;
            }
            have_out = true;
        } else if constexpr (ONE_M) {
            const int chan = wm * 32 + 4 * lk, mlim = g.Mg - chan;
#pragma unroll
            for (int b = 0; b < 2; b++) {
                const int qq = T.q0 + pw + b * 32 + lr;
                const uint32_t base = qq < g.OHW ? (uint32_t)(((T.n * g.M + chan) * g.OHW + qq) * 4) : kOOB;
#pragma unroll
                for (int r0 = 0; r0 < 16; r0 += 4) {
                    float sk[4];
                    if (epi.skip) {
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            const int cr = 8 * ((r0 + u) >> 2) + ((r0 + u) & 3);
                            sk[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                                  zr, cr < mlim ? base : kOOB, cr * g.OHW * 4, 0));
                        }
                    }
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int cr = 8 * ((r0 + u) >> 2) + ((r0 + u) & 3);
                        // + 0.0f without a bias, as the reference adds bias_val = 0.0 (-0 -> +0)
                        float v = acc[b * 16 + r0 + u] + bias_r[r0 + u];
                        if (epi.relu) v = relu_f(v);
                        if (epi.skip) v += sk[u];
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), yr,
                                                              cr < mlim ? base : kOOB, cr * g.OHW * 4, 0);
                    }
                }
            }
        } else {
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int qq = T.q0 + pw + b * 32 + lr;
            const bool qok = qq < g.OHW;
#pragma unroll
            for (int r0 = 0; r0 < 16; r0 += 4) {
                float sk[4];
                if (epi.skip) {
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int m = T.m0 + wm * 32 + 8 * ((r0 + u) >> 2) + ((r0 + u) & 3) + 4 * lk;
                        const uint32_t vo = (qok && m < g.Mg) ? (uint32_t)(((T.n * g.M + m) * g.OHW + qq) * 4) : kOOB;
                        sk[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(zr, vo, 0, 0));
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int r = r0 + u;
                    const int m = T.m0 + wm * 32 + 8 * (r >> 2) + (r & 3) + 4 * lk;
                    const uint32_t vo = (qok && m < g.Mg) ? (uint32_t)(((T.n * g.M + m) * g.OHW + qq) * 4) : kOOB;
                    // + 0.0f without a bias, as the reference adds bias_val = 0.0 (-0 -> +0)
                    float v = acc[b * 16 + r] + Bs[wm * 32 + 8 * (r >> 2) + (r & 3) + 4 * lk];
                    if (epi.relu) v = relu_f(v);
                    if (epi.skip) v += sk[u];
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), yr, vo, 0, 0);
                }
            }
        }
        }
        if (next >= tiles) break;
        __syncthreads();   // every wave is done reading this tile's operands
        if (!ONE_M) store_w();
        store_p();
        __syncthreads();
        slot = next;
        T = Tn;
    }
    if constexpr (DEFER) {
#pragma unroll
        for (int i = 0; i < 32; i++) store_out(i);
    }
}

// The few-channel plan: 3 input channels, 7x7, stride 2, no dilation, one
// group, and a patch that fits (256 consecutive output pixels touch at most
// kStemRows input rows of at most kStemCols columns).
inline bool stem_plan(const ConvTiled& g, int group) {
    if (group != 1 || g.Cg != 3 || g.KH != 7 || g.KW != 7 || g.sh != 2 || g.sw != 2 || g.dh != 1 || g.dw != 1) return false;
    const int rows_out = std::min((256 + g.OW - 1) / g.OW + 1, g.OH);
    const int PR = (rows_out - 1) * 2 + 7, PC = (g.OW - 1) * 2 + 7 + 1;   // + 1: the last column read stays in the row
    return PR <= kStemRows && PC <= kStemCols;
}

template <int C, int KH, int KW, int S>
void launch_conv_stem(const float* x, const float* w, const float* b, float* y, const ConvTiled& g, uint32_t xbytes,
                      uint32_t wbytes, uint32_t ybytes, ConvEpi epi, hipStream_t s) {
    const int tiles_per_img = (g.OHW + 255) / 256, N = g.P / g.OHW, ntm = (g.Mg + 63) / 64;
    const int tiles = N * tiles_per_img * ntm;
    // persistent grid: two blocks per CU (the LDS footprint allows two), a multiple of 8
    const int grid = std::min(2 * num_cus(), (tiles + 7) / 8 * 8);
    if (ntm == 1 && !epi.skip)
        hipLaunchKernelGGL((k_conv_stem<C, KH, KW, S, true, true>), dim3((unsigned)grid), dim3(512), 0, s, x, w, b, y,
                           g, tiles_per_img, ntm, tiles, xbytes, wbytes, ybytes, epi);
    else if (ntm == 1)
        hipLaunchKernelGGL((k_conv_stem<C, KH, KW, S, true, false>), dim3((unsigned)grid), dim3(512), 0, s, x, w, b,
                           y, g, tiles_per_img, ntm, tiles, xbytes, wbytes, ybytes, epi);
    else
        hipLaunchKernelGGL((k_conv_stem<C, KH, KW, S, false, false>), dim3((unsigned)grid), dim3(512), 0, s, x, w, b,
                           y, g, tiles_per_img, ntm, tiles, xbytes, wbytes, ybytes, epi);
}

// XQ != 0 (quantized input) runs with an f32 output and an f32 or no bias only.
template <int BM, int BP, int BK, int WGM, int WGN, int MODE, int XQ = 0, int DEPTH = 1>
void launch_conv_tiled_cfg(const float* x, const float* w, const void* b, int dtb, void* y, int dty, const ConvTiled& g,
                           int group, uint32_t xbytes, uint32_t wbytes, uint32_t ybytes, ConvEpi epi, ConvXQ xq,
                           hipStream_t s) {
    if (MODE == 2 && g.Cg % BK) { set_error("conv: tap-blocked plan needs Cg %% %d == 0", BK); return; }
    const dim3 grid((g.P + BP - 1) / BP, (g.Mg + BM - 1) / BM, group), block(64 * WGM * WGN);
    if (XQ || (dty == kF32 && (!b || dtb == kF32)))
        hipLaunchKernelGGL((k_conv_tiled<BM, BP, BK, WGM, WGN, MODE, kF32, false, XQ, DEPTH>), grid, block, 0, s, x, w,
                           (const float*)b, y, dty, dtb, g, xbytes, wbytes, ybytes, epi, xq, 0, 1);
    else
        hipLaunchKernelGGL((k_conv_tiled<BM, BP, BK, WGM, WGN, MODE, -1, false, 0, DEPTH>), grid, block, 0, s, x, w,
                           (const float*)b, y,
                           dty, dtb, g, xbytes, wbytes, ybytes, ConvEpi{nullptr, 0}, xq, 0, 1);
}

// Sum of the split-K slices of each output element, in slice order (double),
// plus the bias, rounded once to f32.
// One element per thread (coalesced); total < 2^31 (the caller's reach check).
__global__ __launch_bounds__(256) void k_conv_splitk_reduce(const float* __restrict__ part, const float* __restrict__ Bv,
                                                            float* __restrict__ Y, int total, FastDiv fd_ohw,
                                                            FastDiv fd_m, int nsplit, ConvEpi epi) {
    const int i = (int)blockIdx.x * 256 + (int)threadIdx.x;
    if (i >= total) return;
    double acc = 0.0;
    for (int s = 0; s < nsplit; s++) acc += (double)part[(int64_t)s * total + i];
    if (Bv) {
        const uint32_t r = fd_ohw.div((uint32_t)i);
        acc += (double)Bv[r - fd_m.div(r) * fd_m.d];
    }
    float v = (float)acc;
    if (epi.relu) v = relu_f(v);
    if (epi.skip) v += epi.skip[i];
    if (epi.fq.kind) v = fq_apply(v, fq_parm(epi.fq));
    Y[i] = v;
}

// Four consecutive outputs per thread with 16-byte loads and stores (total,
// Y and the skip tensor 16-byte aligned); per element the same slice order,
// fp64 sum, bias, relu and skip as k_conv_splitk_reduce.
__global__ __launch_bounds__(256) void k_conv_splitk_reduce4(const float* __restrict__ part, const float* __restrict__ Bv,
                                                             float* __restrict__ Y, int total, FastDiv fd_ohw,
                                                             FastDiv fd_m, int nsplit, ConvEpi epi) {
    const int i = ((int)blockIdx.x * 256 + (int)threadIdx.x) * 4;
    if (i >= total) return;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int s = 0; s < nsplit; s++) {
        const float4 p = *(const float4*)(part + (int64_t)s * total + i);
        acc[0] += (double)p.x; acc[1] += (double)p.y; acc[2] += (double)p.z; acc[3] += (double)p.w;
    }
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        double a = acc[j];
        if (Bv) {
            const uint32_t r = fd_ohw.div((uint32_t)(i + j));
            a += (double)Bv[r - fd_m.div(r) * fd_m.d];
        }
        v[j] = (float)a;
        if (epi.relu) v[j] = relu_f(v[j]);
    }
    if (epi.skip) {
        const float4 k = *(const float4*)(epi.skip + i);
        v[0] += k.x; v[1] += k.y; v[2] += k.z; v[3] += k.w;
    }
    if (epi.fq.kind) {
        const FQParm fqp = fq_parm(epi.fq);
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = fq_apply(v[j], fqp);
    }
    *(float4*)(Y + i) = make_float4(v[0], v[1], v[2], v[3]);
}

template <int BM, int BP, int BK, int WGM, int WGN, int MODE, int XQ = 0, int DEPTH = 1>
bool launch_conv_split_cfg(const float* x, const float* w, const float* b, float* y, const ConvTiled& g, int group,
                           uint32_t xbytes, uint32_t wbytes, int nsplit_req, ConvEpi epi, ConvXQ xq, hipStream_t s) {
    if (MODE == 2 && g.Cg % BK) { set_error("conv: tap-blocked plan needs Cg %% %d == 0", BK); return true; }
    const int kchunk = ((g.Kg + nsplit_req - 1) / nsplit_req + BK - 1) / BK * BK;
    const int nsplit = (g.Kg + kchunk - 1) / kchunk;
    const int64_t total = (int64_t)g.P * g.M;
    float* part = (float*)pool_alloc((size_t)nsplit * total * sizeof(float));
    if (!part) return false;
    const dim3 grid((g.P + BP - 1) / BP, (g.Mg + BM - 1) / BM, group * nsplit), block(64 * WGM * WGN);
    hipLaunchKernelGGL((k_conv_tiled<BM, BP, BK, WGM, WGN, MODE, kF32, true, XQ, DEPTH>), grid, block, 0, s, x, w, b, part,
                       kF32, kF32, g, xbytes, wbytes, 0u, ConvEpi{nullptr, 0}, xq, kchunk, group);
    const bool vec4 = total % 4 == 0 && ((uintptr_t)y & 15) == 0 && ((uintptr_t)epi.skip & 15) == 0;
    if (vec4)
        hipLaunchKernelGGL(k_conv_splitk_reduce4, dim3((unsigned)((total / 4 + 255) / 256)), dim3(256), 0, s, part, b,
                           y, (int)total, make_fastdiv((uint32_t)g.OHW), make_fastdiv((uint32_t)g.M), nsplit, epi);
    else
        hipLaunchKernelGGL(k_conv_splitk_reduce, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, part, b, y,
                           (int)total, make_fastdiv((uint32_t)g.OHW), make_fastdiv((uint32_t)g.M), nsplit, epi);
    pool_free(part);   // stream-ordered reuse: later work on this stream runs after the reduction
    return true;
}

// Returns false (caller falls back) when a tensor is beyond the 2 GB reach of
// 32-bit buffer offsets.
template <int XQ>
// *fq_applied (when given) tells whether the kernels applied epi.fq: the stem
// plan leaves it to the caller.
bool launch_conv_tiled_xq(const void* x, const void* w, const void* b, int dtb, void* y, int dty, const ConvGeom& cg,
                          ConvEpi epi, ConvXQ xq, hipStream_t s, bool* fq_applied = nullptr) {
    if (fq_applied) *fq_applied = epi.fq.kind != 0;
    const int64_t xb = (int64_t)cg.N * cg.C * cg.H * cg.W * (XQ ? 1 : 4), wb = (int64_t)cg.M * cg.Kg * 4;
    const int64_t P = (int64_t)cg.N * cg.OH * cg.OW;
    const int64_t yb = P * cg.M * 4;
    if (xb >= ((int64_t)1 << 31) || wb >= ((int64_t)1 << 31) || yb >= ((int64_t)1 << 31)) return false;
    ConvTiled g;
    g.C = cg.C; g.H = cg.H; g.W = cg.W; g.M = cg.M; g.KH = cg.KH; g.KW = cg.KW; g.OH = cg.OH; g.OW = cg.OW;
    g.pt = cg.pt; g.pl = cg.pl; g.sh = cg.sh; g.sw = cg.sw; g.dh = cg.dh; g.dw = cg.dw;
    g.Cg = cg.Cg; g.Mg = cg.Mg; g.Kg = cg.Kg; g.HW = cg.H * cg.W; g.OHW = cg.OH * cg.OW; g.P = (int)P;
    g.fd_ohw = make_fastdiv((uint32_t)g.OHW);
    g.fd_ow = make_fastdiv((uint32_t)g.OW);
    g.fd_khw = make_fastdiv((uint32_t)(g.KH * g.KW));
    g.fd_kw = make_fastdiv((uint32_t)g.KW);
    g.fd_cg = make_fastdiv((uint32_t)g.Cg);
    const bool direct = g.KH == 1 && g.KW == 1 && g.sh == 1 && g.sw == 1 && g.pt == 0 && g.pl == 0 &&
                        g.OH == g.H && g.OW == g.W && g.HW % 4 == 0 && (((uintptr_t)x) & (XQ ? 3 : 15)) == 0;
    const float* xf = (const float*)x;
    const float* wf = (const float*)w;
    // MODE 0 block shapes: 64 channels x 256 pixels with 8 or 16 waves (wave
    // tiles 32x64 / 32x32); BK = 8 when K is short (the 7x7x3 stem: less
    // padding, more tiles in flight).
    const uint32_t ux = (uint32_t)xb, uw = (uint32_t)wb, uy = (uint32_t)yb;
    // The 3-channel 7x7 / stride-2 stem: its whole k range in LDS (k_conv_stem).
    // Quantized inputs never get here for it (conv_xq_fast sends them through
    // DequantizeLinear and this plan, which keeps the two paths' bits equal).
    if constexpr (XQ == 0) {
        if (stem_plan(g, cg.group) && dty == kF32 && (!b || dtb == kF32)) {
            launch_conv_stem<3, 7, 7, 2>(xf, wf, (const float*)b, (float*)y, g, ux, uw, uy, epi, s);
            if (fq_applied) *fq_applied = false;
            return true;
        }
    }
    // Plan: MODE 1 for 1x1 stride-1 layers; MODE 2 (BK = 16, so Cg % 16 == 0
    // keeps every k-tile inside one tap) for
    //   * 1x1 strided layers: 128x128 tiles (16 waves of 32x32, two register
    //     sets) when >= 256 output channels still give >= 192 blocks, else 64x128;
    //   * >= 128 output pixels per image: 128x256 (16 waves of 64x32, two
    //     register sets) for >= 128 output channels, else 64x256 (8 waves of
    //     32x64) or 64x128 (8 waves of 32x32, two register sets) by balance;
    //   * smaller images with >= 128 output channels: 128x256 tiles would span
    //     five or more images and miss L1 on the tap-blocked order, 128x128
    //     tiles (16 waves of 32x32, two register sets) keep it (block 4 of
    //     config 5: 109 -> 92 us at split 5);
    // MODE 0 otherwise (the 3-channel stem, few output channels on small
    // images).  Swept on MI355X over the config-4 / config-5 layers.
    // Tiles do equal work, so a grid of t tiles keeps the CUs busy for a share
    // (t / CUs) / ceil(t / CUs) of the time (fewer tiles than CUs: t / CUs).
    auto balance = [](int64_t t) {
        const double r = (double)t / (double)num_cus();
        return r / std::ceil(r);
    };
    enum { kNone, kT64x128, kT128x128, kT64x256, kT128x256 };
    const int khw = g.KH * g.KW;
    int plan = kNone;
    if (!direct && g.Cg % 16 == 0) {
        if (khw == 1)
            plan = (g.Mg >= 256 && ((P + 127) / 128) * ((g.Mg + 127) / 128) * cg.group >= 192) ? kT128x128 : kT64x128;
        else if (g.OHW >= 128)
            plan = g.Mg >= 128 ? kT128x256 : kT64x256;
        else if (g.Mg >= 128)
            plan = kT128x128;
        // 64x128 tiles (two register sets) when they fill the CUs better than
        // 64x256 ones (config-5 block 1: 784 -> 1568 tiles, 0.77 -> 0.87; 163 -> 159 us)
        if (plan == kT64x256 &&
            balance(((P + 127) / 128) * ((g.Mg + 63) / 64) * cg.group) >
                1.05 * balance(((P + 255) / 256) * ((g.Mg + 63) / 64) * cg.group))
            plan = kT64x128;
    }
    // 64-row tiles when 128-row ones leave CUs idle and the 64-row grid alone
    // covers >= 3/4 of them: no k split, so no slices to write and reduce
    // (config-5 block 3: 98 128x256 tiles -> 196 64x256 tiles, 97.4 -> 92.8 us
    // with the slice reduction counted; block 2, 196 -> 392 tiles, unchanged)
    bool no_split = false;
    if (plan == kT128x256 && ((P + 255) / 256) * ((g.Mg + 127) / 128) * cg.group < num_cus() &&
        4 * ((P + 255) / 256) * ((g.Mg + 63) / 64) * cg.group >= 3 * (int64_t)num_cus()) {
        plan = kT64x256;
        no_split = true;
    }
    const int bm = (plan == kT128x128 || plan == kT128x256) ? 128 : 64;
    const int bp = (plan == kT64x128 || plan == kT128x128) ? 128 : 256;
    const int64_t blocks = ((P + bp - 1) / bp) * ((g.Mg + bm - 1) / bm) * cg.group;
    // Split-k slice count for grids smaller than the CU count: each slice
    // >= 128 deep, at most 8; the count whose block total balances best over
    // the CUs (fewer slices on near ties: each slice adds a write and a read of
    // the output), and only if that beats the unsplit grid by 5%.
    // Config-5 block 4: 100 tiles -> 5 slices (0.98 of the CUs busy, not 0.39).
    int split = 1;
    // (not under graph capture: the slices' workspace would have to outlive the call)
    if (blocks < num_cus() && !no_split && !stream_capturing(s)) {
        const int smax = (int)std::min<int64_t>(g.Kg / 128, 8);
        const double base = balance(blocks);
        double best = base;
        for (int sp = 2; sp <= smax; sp++) {
            const double bal = balance(blocks * sp);
            if (bal > best * 1.02) { best = bal; split = sp; }
        }
        if (best < base * 1.05) split = 1;
    }
    if (split > 1 && dty == kF32 && (!b || dtb == kF32) && yb * split < ((int64_t)1 << 31)) {
        // (an XQ launch always has an f32 output and an f32 or no bias)
        const float* bf = (const float*)b;
        float* yf = (float*)y;
        if (direct)
            return launch_conv_split_cfg<64, 256, 16, 2, 4, 1, XQ>(xf, wf, bf, yf, g, cg.group, ux, uw, split, epi, xq, s);
        if (plan == kT64x128)
            return launch_conv_split_cfg<64, 128, 16, 2, 4, 2, XQ, 2>(xf, wf, bf, yf, g, cg.group, ux, uw, split, epi, xq,
                                                                      s);
        if (plan == kT128x128)
            return launch_conv_split_cfg<128, 128, 16, 4, 4, 2, XQ, 2>(xf, wf, bf, yf, g, cg.group, ux, uw, split, epi,
                                                                       xq, s);
        if (plan == kT128x256)
            return launch_conv_split_cfg<128, 256, 16, 2, 8, 2, XQ, 2>(xf, wf, bf, yf, g, cg.group, ux, uw, split, epi,
                                                                       xq, s);
        if (plan == kT64x256)
            return launch_conv_split_cfg<64, 256, 16, 2, 4, 2, XQ>(xf, wf, bf, yf, g, cg.group, ux, uw, split, epi, xq, s);
        if (g.Kg <= 256)
            return launch_conv_split_cfg<64, 256, 8, 2, 4, 0, XQ>(xf, wf, bf, yf, g, cg.group, ux, uw, split, epi, xq, s);
        return launch_conv_split_cfg<64, 256, 16, 2, 8, 0, XQ>(xf, wf, bf, yf, g, cg.group, ux, uw, split, epi, xq, s);
    }
    if (direct && g.Kg <= 64)
        // shallow 1x1 layers: BK 8 (the config-4 1x1, K = 64: 42.8 -> 42.1 us over six A/B
        // pairs, same bits; K >= 128 ran 3-13% slower with BK 8)
        launch_conv_tiled_cfg<64, 256, 8, 2, 4, 1, XQ>(xf, wf, b, dtb, y, dty, g, cg.group, ux, uw, uy, epi, xq, s);
    else if (direct)
        launch_conv_tiled_cfg<64, 256, 16, 2, 4, 1, XQ>(xf, wf, b, dtb, y, dty, g, cg.group, ux, uw, uy, epi, xq, s);
    else if (plan == kT64x128)
        launch_conv_tiled_cfg<64, 128, 16, 2, 4, 2, XQ, 2>(xf, wf, b, dtb, y, dty, g, cg.group, ux, uw, uy, epi, xq, s);
    else if (plan == kT128x128)
        launch_conv_tiled_cfg<128, 128, 16, 4, 4, 2, XQ, 2>(xf, wf, b, dtb, y, dty, g, cg.group, ux, uw, uy, epi, xq, s);
    else if (plan == kT128x256)
        // store-first pipeline (DEPTH 3): config-5 block 2 89.3 -> 86.8 us (best of 3, same bits)
        launch_conv_tiled_cfg<128, 256, 16, 2, 8, 2, XQ, 3>(xf, wf, b, dtb, y, dty, g, cg.group, ux, uw, uy, epi, xq, s);
    else if (plan == kT64x256)
        // store-first pipeline (DEPTH 3): the config-4 3x3 layer 85.7 -> 84.3 us (best of 3, same bits)
        launch_conv_tiled_cfg<64, 256, 16, 2, 4, 2, XQ, 3>(xf, wf, b, dtb, y, dty, g, cg.group, ux, uw, uy, epi, xq, s);
    else if (g.Kg <= 256)
        launch_conv_tiled_cfg<64, 256, 8, 2, 4, 0, XQ>(xf, wf, b, dtb, y, dty, g, cg.group, ux, uw, uy, epi, xq, s);
    else if (balance(((P + 127) / 128) * ((g.Mg + 63) / 64) * cg.group) > 1.05 * balance(blocks))
        // 64x128 tiles (8 waves) when they fill the CUs better than 64x256 ones
        // (config-5-like 56x56 layers of 64 channels: 784 -> 1568 tiles, 0.77 -> 0.88)
        launch_conv_tiled_cfg<64, 128, 16, 2, 4, 0, XQ>(xf, wf, b, dtb, y, dty, g, cg.group, ux, uw, uy, epi, xq, s);
    else
        launch_conv_tiled_cfg<64, 256, 16, 2, 8, 0, XQ>(xf, wf, b, dtb, y, dty, g, cg.group, ux, uw, uy, epi, xq, s);
    return true;
}

bool launch_conv_tiled(const void* x, const void* w, const void* b, int dtb, void* y, int dty, const ConvGeom& cg,
                       ConvEpi epi, hipStream_t s, bool* fq_applied = nullptr) {
    return launch_conv_tiled_xq<0>(x, w, b, dtb, y, dty, cg, epi, ConvXQ{nullptr, nullptr}, s, fq_applied);
}

inline bool f32_exact_dtype(int dt) {
    return dt == kF32 || dt == kF16 || dt == kBF16 || dt == kE4M3 || dt == kE5M2 || dt == kI4 || dt == kI8 ||
           dt == kU8 || dt == kI16;
}

template <int DX, int DW>
void launch_conv_mfma(const void* x, int dtx, const void* w, int dtw, const void* b, int dtb, void* y, int dty,
                      const ConvGeom& g, hipStream_t s) {
    const int P = g.N * g.OH * g.OW;
    const dim3 grid((P + kCN - 1) / kCN, (g.Mg + kCM - 1) / kCM, g.group);
    if (dty == kF32)
        hipLaunchKernelGGL((k_conv_mfma_f32<DX, DW, kF32>), grid, dim3(256), 0, s, x, w, b, dtb, y, dty, g, dtx, dtw);
    else
        hipLaunchKernelGGL((k_conv_mfma_f32<DX, DW, -1>), grid, dim3(256), 0, s, x, w, b, dtb, y, dty, g, dtx, dtw);
}

}  // namespace
}  // namespace tohip

using namespace tohip;

namespace {
// Shared by conv2d_forward and conv2d_fused_forward.  Returns false when the
// fused epilogue (skip / relu) could not be applied in the kernel: the caller
// then applies it with the standalone operators.
// xq_kind 1 / 2: X holds uint8 / int8 codes dequantised in the kernel with the
// one-element scale xs and zero point xz (xz may be null); the caller has
// checked that this is the tiled f32 path (f32 W / Y, f32 or no bias).
// fq_kind 1 / 2: fake quantization with uint8 / int8 codes after the skip add,
// parameters fq_t = {q scale, q zero point, d scale, d zero point} (one-element
// f32 scales, zero points of the code dtype); *fq_done tells whether the kernel
// applied it, which it does only where it also applied relu and skip.
bool conv_entry(const char* name, const Tensor* X, const Tensor* W, const Tensor* B, Tensor* Y, ConvParams* params,
                const void* skip, int relu, int xq_kind = 0, const Tensor* xs = nullptr, const Tensor* xz = nullptr,
                int fq_kind = 0, const Tensor* const* fq_t = nullptr, bool* fq_done = nullptr) {
    if (fq_done) *fq_done = false;
    if (!tensor_sane(X, name) || !tensor_sane(W, name) || !tensor_sane(Y, name)) return true;
    if (!params || !params->pads || !params->strides || !params->dilations) { set_error("%s: NULL params", name); return true; }
    if (X->ndim != 4 || W->ndim != 4 || Y->ndim != 4) { set_error("%s: X, W and Y must be 4-D", name); return true; }
    ConvGeom g;
    g.N = X->shape[0]; g.C = X->shape[1]; g.H = X->shape[2]; g.W = X->shape[3];
    g.M = W->shape[0]; g.KH = W->shape[2]; g.KW = W->shape[3];
    g.OH = Y->shape[2]; g.OW = Y->shape[3];
    g.pt = params->pads[0]; g.pl = params->pads[1];
    g.sh = params->strides[0]; g.sw = params->strides[1];
    g.dh = params->dilations[0]; g.dw = params->dilations[1];
    g.group = params->group;
    if (g.group < 1 || g.C % g.group || g.M % g.group) { set_error("%s: bad group %d", name, g.group); return true; }
    g.Cg = g.C / g.group; g.Mg = g.M / g.group;
    if (W->shape[1] != g.Cg) { set_error("%s: W.shape[1]=%d but C/group=%d", name, W->shape[1], g.Cg); return true; }
    if (Y->shape[0] != g.N || Y->shape[1] != g.M) { set_error("%s: Y shape does not match N, M", name); return true; }
    g.Kg = g.Cg * g.KH * g.KW;
    const bool has_b = B && B->data;
    if (has_b && (!tensor_sane(B, name) || B->size < (size_t)g.M)) { set_error("%s: bias needs M elements", name); return true; }
    if (!ensure_device()) return true;
    const int64_t total = (int64_t)g.N * g.M * g.OH * g.OW;
    Staging st;
    const void* x = st.in(X);
    const void* w = st.in(W);
    const void* b = has_b ? st.in(B) : nullptr;
    void* y = st.out(Y, (size_t)total * dt_bytes((int)Y->dtype));
    const void* z = skip ? st.in((const Tensor*)skip) : nullptr;
    const void* xsd = xq_kind ? st.in(xs) : nullptr;
    const void* xzd = (xq_kind && xz) ? st.in(xz) : nullptr;
    const void* fqd[4] = {nullptr, nullptr, nullptr, nullptr};
    if (fq_kind)
        for (int k = 0; k < 4; k++) fqd[k] = st.in(fq_t[k]);
    if (!x || !w || !y || (has_b && !b) || (skip && !z) || (xq_kind && !xsd) || (xq_kind && xz && !xzd) ||
        (fq_kind && (!fqd[0] || !fqd[1] || !fqd[2] || !fqd[3]))) {
        st.finish();
        return true;
    }
    const FakeQuant fq{(const float*)fqd[0], fqd[1], (const float*)fqd[2], fqd[3], fq_kind};
    bool fused = !skip && !relu;   // epilogue applied in the kernel (or none requested)
    hipStream_t s = stream();
    const int dtx = (int)X->dtype, dtw = (int)W->dtype, dty = (int)Y->dtype, dtb = has_b ? (int)B->dtype : kF32;
    if (total > 0) {
        const bool big = (int64_t)g.N * g.OH * g.OW > 0x7FFFFFFF;
        bool done = false;
        if (xq_kind) {
            const ConvEpi epi{(const float*)z, relu, fq};
            const ConvXQ xq{(const float*)xsd, xzd};
            bool fq_applied = false;
            const bool ok = xq_kind == 1 ? launch_conv_tiled_xq<1>(x, w, b, dtb, y, dty, g, epi, xq, s, &fq_applied)
                                         : launch_conv_tiled_xq<2>(x, w, b, dtb, y, dty, g, epi, xq, s, &fq_applied);
            if (!ok) set_error("%s: operands beyond the quantized-input kernel's reach", name);
            fused = true;
            if (fq_done) *fq_done = ok && fq_applied;
            done = true;
        } else if (!exact_mode() && !big && g.Kg > 0 && f32_exact_dtype(dtx) && f32_exact_dtype(dtw)) {
            if (dtx == kF32 && dtw == kF32) {
                const bool epi_ok = dty == kF32 && (!has_b || dtb == kF32);
                const ConvEpi epi{epi_ok ? (const float*)z : nullptr, epi_ok ? relu : 0,
                                  epi_ok ? fq : FakeQuant{nullptr, nullptr, nullptr, nullptr, 0}};
                bool fq_applied = false;
                if (launch_conv_tiled(x, w, b, dtb, y, dty, g, epi, s, &fq_applied)) {
                    fused = fused || epi_ok;
                    if (fq_done) *fq_done = fq_applied;
                }
                else launch_conv_mfma<kF32, kF32>(x, dtx, w, dtw, b, dtb, y, dty, g, s);
            } else {
                launch_conv_mfma<-1, -1>(x, dtx, w, dtw, b, dtb, y, dty, g, s);
            }
            done = true;
        }
        if (!done)
            hipLaunchKernelGGL(k_conv_exact, dim3(grid_for((size_t)total, 256)), dim3(256), 0, s, x, dtx, w, dtw, b, dtb,
                               y, dty, g, total);
        if (!check_launch(name)) { st.finish(); return true; }
    }
    st.finish();
    return fused || total == 0;
}
}  // namespace

extern "C" void conv2d_forward(const Tensor* X, const Tensor* W, const Tensor* B, Tensor* Y, ConvParams* params) {
    conv_entry("conv2d_forward", X, W, B, Y, params, nullptr, 0);
}

// Conv -> Relu -> Add(., Skip) in one pass (the ResNet block's epilogue);
// see tensor_ops.h.  The kernel epilogue covers f32 X / W / Y with an f32 or no
// bias and an f32 Skip of Y's size; otherwise the standalone operators run after
// the convolution, which is also what the fused epilogue equals.
extern "C" void conv2d_fused_forward(const Tensor* X, const Tensor* W, const Tensor* B, const Tensor* Skip, int relu,
                                     Tensor* Y, ConvParams* params) {
    const char* name = "conv2d_fused_forward";
    const bool has_skip = Skip && Skip->data;
    if (has_skip && !tensor_sane(Skip, name)) return;
    if (!Y) { set_error("%s: NULL output", name); return; }
    const bool skip_in_kernel = has_skip && Skip->dtype == kF32 && Skip->size == Y->size;
    tensor_ops_hip_clear_error();
    const bool fused = conv_entry(name, X, W, B, Y, params, skip_in_kernel ? Skip : nullptr, relu ? 1 : 0);
    if (tensor_ops_hip_last_error()[0]) return;
    if (!fused && relu) relu_forward(Y, Y);
    if ((!fused || !skip_in_kernel) && has_skip && !tensor_ops_hip_last_error()[0]) add_forward(Y, Skip, Y);
}

// Conv -> Relu -> Add(., Skip) -> QuantizeLinear -> DequantizeLinear in one
// pass; see tensor_ops.h.  The kernel epilogue covers what conv2d_fused_forward's
// does, with uint8 / int8 codes and one-element f32 scales and zero points of
// the code dtype; otherwise the fused convolution runs and then
// quantize_dequantize_linear_forward in place on Y, which is also what the
// epilogue equals.
extern "C" void conv2d_fused_qdq_forward(const Tensor* X, const Tensor* W, const Tensor* B, const Tensor* Skip,
                                         int relu, const Tensor* QScale, const Tensor* QZeroPoint,
                                         const Tensor* DScale, const Tensor* DZeroPoint, int code_dtype, Tensor* Y,
                                         ConvParams* params) {
    const char* name = "conv2d_fused_qdq_forward";
    const bool has_skip = Skip && Skip->data;
    if (has_skip && !tensor_sane(Skip, name)) return;
    if (!tensor_sane(QScale, name) || !tensor_sane(QZeroPoint, name) || !tensor_sane(DScale, name) ||
        !tensor_sane(DZeroPoint, name) || !tensor_sane(Y, name))
        return;
    const bool skip_in_kernel = has_skip && Skip->dtype == kF32 && Skip->size == Y->size;
    const int kind = code_dtype == kU8 ? 1 : (code_dtype == kI8 ? 2 : 0);
    const bool fq_ok = kind && Y->dtype == kF32 && (!has_skip || skip_in_kernel) && QScale->dtype == kF32 &&
                       DScale->dtype == kF32 && QScale->size == 1 && DScale->size == 1 && QZeroPoint->size == 1 &&
                       DZeroPoint->size == 1 && (int)QZeroPoint->dtype == code_dtype &&
                       (int)DZeroPoint->dtype == code_dtype;
    const Tensor* fq_t[4] = {QScale, QZeroPoint, DScale, DZeroPoint};
    tensor_ops_hip_clear_error();
    bool fq_done = false;
    const bool fused = conv_entry(name, X, W, B, Y, params, skip_in_kernel ? Skip : nullptr, relu ? 1 : 0, 0, nullptr,
                                  nullptr, fq_ok ? kind : 0, fq_t, &fq_done);
    if (tensor_ops_hip_last_error()[0]) return;
    if (!fused && relu) relu_forward(Y, Y);
    if ((!fused || !skip_in_kernel) && has_skip && !tensor_ops_hip_last_error()[0]) add_forward(Y, Skip, Y);
    if (!fq_done && !tensor_ops_hip_last_error()[0])
        quantize_dequantize_linear_forward(Y, QScale, QZeroPoint, DScale, DZeroPoint, Y, code_dtype);
}

namespace {
bool conv_xq_fast(const Tensor* Xq, const Tensor* XScale, const Tensor* XZero, const Tensor* W, const Tensor* B,
                  const Tensor* Skip, const Tensor* Y, const ConvParams* params) {
    const int dx = (int)Xq->dtype;
    // 3-channel 7x7 stride-2 layers take the f32 stem plan: run them as the pair
    if (W->ndim == 4 && W->shape[1] == 3 && W->shape[2] == 7 && W->shape[3] == 7 && params && params->strides &&
        params->strides[0] == 2 && params->strides[1] == 2)
        return false;
    if (exact_mode() || (dx != kU8 && dx != kI8) || XScale->dtype != kF32 || XScale->size != 1) return false;
    if (XZero && XZero->data && ((int)XZero->dtype != dx || XZero->size != 1)) return false;
    if (W->dtype != kF32 || Y->dtype != kF32 || (B && B->data && B->dtype != kF32)) return false;
    if (Skip && Skip->data && (Skip->dtype != kF32 || Skip->size != Y->size)) return false;
    if (Xq->ndim != 4 || W->ndim != 4 || Y->ndim != 4) return false;
    return (int64_t)Xq->shape[0] * Xq->shape[1] * Xq->shape[2] * Xq->shape[3] < ((int64_t)1 << 31);
}
}  // namespace

// DequantizeLinear -> Conv -> Relu -> Add(., Skip): the QDQ convolution of a
// quantized ResNet block in one pass; see tensor_ops.h.  The kernel covers
// uint8 / int8 codes with a one-element f32 scale and zero point, f32 weights,
// output and skip; otherwise the standalone operators run in sequence, which
// is also what the fused kernel returns.
extern "C" void dequantize_conv2d_fused_forward(const Tensor* Xq, const Tensor* XScale, const Tensor* XZero,
                                                const Tensor* W, const Tensor* B, const Tensor* Skip, int relu,
                                                Tensor* Y, ConvParams* params) {
    const char* name = "dequantize_conv2d_fused_forward";
    if (!tensor_sane(Xq, name) || !tensor_sane(XScale, name) || !tensor_sane(W, name) || !tensor_sane(Y, name)) return;
    const bool has_z = XZero && XZero->data;
    if (has_z && !tensor_sane(XZero, name)) return;
    if (Xq->ndim != 4) { set_error("%s: X must be 4-D (NCHW), got rank %d", name, Xq->ndim); return; }
    if (!ensure_device()) return;
    if (conv_xq_fast(Xq, XScale, has_z ? XZero : nullptr, W, B, Skip, Y, params)) {
        tensor_ops_hip_clear_error();
        conv_entry(name, Xq, W, B, Y, params, (Skip && Skip->data) ? Skip : nullptr, relu ? 1 : 0,
                   Xq->dtype == kU8 ? 1 : 2, XScale, has_z ? XZero : nullptr);
        return;
    }
    // the unfused sequence: DequantizeLinear into an f32 tensor, then the convolution
    int shp[4];
    for (int i = 0; i < 4; i++) shp[i] = Xq->shape[i];
    Tensor* Xd = create_tensor_device_empty(shp, 4, DTYPE_FLOAT32);
    if (!Xd) return;
    tensor_ops_hip_clear_error();
    if (has_z) {
        dequantize_linear_forward(Xq, XScale, XZero, Xd);
    } else {
        int one = 1;
        Tensor* z0 = create_tensor(&one, 1, DTYPE_UINT8);
        if (z0) {
            dequantize_linear_forward(Xq, XScale, z0, Xd);
            free_tensor(z0);
        }
    }
    if (tensor_ops_hip_last_error()[0] == 0) conv2d_fused_forward(Xd, W, B, Skip, relu, Y, params);
    free_tensor(Xd);
}
