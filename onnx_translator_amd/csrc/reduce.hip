// reduce.hip — Softmax, MaxPool and GlobalAveragePool for gfx950.
//
// Softmax (tensor_ops/tensor_ops.c:1231-1270): the tensor is viewed as
// [outer, L, inner] around the axis; per (outer, inner) column the reference
// takes the max over the axis (from -DBL_MAX), sums exp(v - max) in double and
// writes exp(v - max) / sum.  Kernels here:
//   * many rows (inner == 1): one 1024-thread block per row, the row held in
//     registers, wave64 shuffle + LDS reductions, read once / written once;
//   * few long rows (inner == 1, e.g. [64, 32000]): each row is split over G
//     blocks so the fp64 exp / divide work covers the chip: pass 1 writes each
//     block's (max m_b, sum_b exp(v - m_b)); pass 2 folds them into the row's
//     max M and sum S = sum_b s_b * exp(m_b - M) (fixed order) and writes
//     exp(v - m_b) * (exp(m_b - M) / S); the one-launch form keeps exp(v - m_b)
//     in registers from its partial pass, so each value is exponentiated once;
//   * inner > 1: one thread per column, coalesced along the inner dimension.
// Max, sums and the final scaling are in double (the sums are trees instead of the
// reference's sequential loop); exp is sm_exp below (fp64 range reduction,
// fp32 core) and the divide is a multiply by 1 / sum, so outputs agree with
// the reference to ~1e-7 relative: a tolerance class (rtol 1e-5).
//
// GlobalAveragePool (tensor_ops.c:2844-2868): exact sequential plane sums,
// one thread per plane over LDS-staged tiles.
//
// MaxPool (tensor_ops.c:1116-1165): -inf start, in-bounds taps only, strict >
// in the reference's (kh, kw) order — NaN never wins, an all-padding window
// gives -inf, the first of +-0 wins.  General windows: one wave per output
// row, one lane per output column.  The ResNet 3x3 / stride 2 / pad 1 f32
// window has a block-per-plane strip kernel that loads each input row once.
#include <atomic>
#include <cfloat>

#include "quant.h"
#include "runtime.h"

namespace tohip {
namespace {

// exp(x) for x <= 0 (x = v - max), NaN propagated.  Range reduction in fp64
// (t = x * log2 e, n = rint(t), f = t - n exactly, |f| <= 1/2), the core 2^f
// on the fp32 exp2 unit (v_exp_f32: no range handling is needed for |f| <= 1/2),
// scaled back with ldexp in fp64: ~1e-7 relative to the reference's libm exp
// in double, at a fraction of the cost of a full fp64 exp (which made this
// operator ALU-bound).  Branch-free: t below -1100 (-inf included) is clamped
// there, where ldexp underflows to +0 as exp() does (anything below 2^-1075
// rounds to 0); a NaN fails the compare, passes through rint, the subtraction
// and the exp unchanged and comes out NaN.
__device__ __forceinline__ double sm_exp(double x) {
    double t = x * 1.4426950408889634;
    t = t < -1100.0 ? -1100.0 : t;
    const double n = __builtin_rint(t);
    const float r = __builtin_amdgcn_exp2f((float)(t - n));
    return __builtin_ldexp((double)r, (int)n);
}

constexpr int kRowThreads = 1024;
constexpr int kWaves = kRowThreads / 64;

// Max (strict >) or sum over the wave's 64 lanes, the same result in every
// lane (wave_allreduce: DPP moves and permlane swaps, all 64 lanes active).
template <bool MAX> __device__ __forceinline__ double wave_reduce(double v) {
    return wave_allreduce(v, [](double x, double y) { return MAX ? (y > x ? y : x) : x + y; });
}
__device__ __forceinline__ double wave_max(double v) { return wave_reduce<true>(v); }
__device__ __forceinline__ double wave_sum(double v) { return wave_reduce<false>(v); }

// Block-wide reduction across the NW waves of a block (NW * 64 threads).
template <bool MAX, int NW> __device__ __forceinline__ double block_reduce(double v, double* lds) {
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

template <int DT> __device__ __forceinline__ double ldx(const void* p, int64_t i, int rdt) {
    if constexpr (DT >= 0) return ld_d<DT>(p, i);
    else return ld_d_rt(rdt, p, i);
}
template <int DT> __device__ __forceinline__ void stx(void* p, int64_t i, double v, int rdt) {
    if constexpr (DT >= 0) st_d<DT>(p, i, v);
    else st_d_rt(rdt, p, i, v);
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
    mx = block_reduce<true, kWaves>(mx, lds);
    double sum = 0.0;
#pragma unroll
    for (int t = 0; t < IPT; t++) {
        const int j = threadIdx.x + t * kRowThreads;
        v[t] = j < L ? sm_exp(v[t] - mx) : 0.0;
        sum += v[t];
    }
    sum = block_reduce<false, kWaves>(sum, lds);
    const double rs = 1.0 / sum;     // tolerance class: reciprocal instead of a divide per element
#pragma unroll
    for (int t = 0; t < IPT; t++) {
        const int j = threadIdx.x + t * kRowThreads;
        if (j < L) st_d<DOUT>(Y, (int64_t)(base + j), v[t] * rs);
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
    mx = block_reduce<true, kWaves>(mx, lds);
    double sum = 0.0;
    for (int64_t j = threadIdx.x; j < L; j += kRowThreads) sum += sm_exp(ld_d_rt(dtx, X, base + j) - mx);
    sum = block_reduce<false, kWaves>(sum, lds);
    for (int64_t j = threadIdx.x; j < L; j += kRowThreads)
        st_d_rt(dty, Y, base + j, sm_exp(ld_d_rt(dtx, X, base + j) - mx) / sum);
}

// Split rows: pass 1.  Block b of a row holds its chunk (up to IPT * 256
// elements) in registers, reduces its max m_b and then s_b = sum exp(v - m_b)
// (no second read of X), and writes part[row * G + b] = m_b and
// part[rows * G + row * G + b] = s_b.  IPT = 0: loop over the chunk instead.
constexpr int kSplitThreads = 256;
constexpr int kSplitWaves = kSplitThreads / 64;

// The IPT values of this thread in the block's chunk [j0, j1) of a row
// (element j0 + threadIdx.x + t * 256 for t < IPT; 0 past j1).  f32 goes
// through a buffer resource over the chunk, so the loads are unconditional and
// issue back to back (lanes past the end read 0 without touching memory).
template <int DIN, int IPT>
__device__ __forceinline__ void load_chunk(double (&v)[IPT], const void* __restrict__ X, int dtx, int64_t base,
                                           int64_t j0, int64_t j1) {
    if constexpr (DIN == kF32) {
        const int64_t n = j1 > j0 ? j1 - j0 : 0;
        const __amdgpu_buffer_rsrc_t xr = buffer_rsrc((const float*)X + base + j0, (uint32_t)(n * 4));
#pragma unroll
        for (int t = 0; t < IPT; t++)
            v[t] = (double)__builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                         xr, (uint32_t)((threadIdx.x + t * kSplitThreads) * 4), 0, 0));
    } else {
#pragma unroll
        for (int t = 0; t < IPT; t++) {
            const int64_t j = j0 + threadIdx.x + t * kSplitThreads;
            v[t] = j < j1 ? ldx<DIN>(X, base + j, dtx) : 0.0;
        }
    }
}

// Writes o[t] to element j0 + threadIdx.x + t * 256 of the row for the lanes
// inside the chunk of n elements.  f32 output goes through a buffer resource
// over the chunk: the stores are unconditional and the hardware drops the
// lanes past its end.  They are nontemporal (cache policy nt): the output is
// not read back by this launch, and streaming it past the caches measured
// 8.3 -> 6.8 us on [64, 32000].
template <int DOUT, int IPT>
__device__ __forceinline__ void store_chunk(void* __restrict__ Y, int dty, int64_t base, int64_t j0, int n,
                                            const double (&o)[IPT]) {
    const int tid = (int)threadIdx.x;
    if constexpr (DOUT == kF32) {
        const __amdgpu_buffer_rsrc_t yr = buffer_rsrc((float*)Y + base + j0, (uint32_t)n * 4u);
#pragma unroll
        for (int t = 0; t < IPT; t++)
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, (float)o[t]), yr,
                                                  (uint32_t)((tid + t * kSplitThreads) * 4), 0, 2 /* nt */);
    } else {
#pragma unroll
        for (int t = 0; t < IPT; t++)
            if (tid + t * kSplitThreads < n) stx<DOUT>(Y, base + j0 + tid + t * kSplitThreads, o[t], dty);
    }
}

// (m, s) of chunk c of a row, the whole block participating: m is the chunk's
// max, s = sum exp(v - m), and v receives exp(v - m) per element, kept for the
// output.  Lanes past the chunk's end hold -inf, which never wins the max and
// whose exp is +0 whatever m is (-inf - m is -inf), so every lane runs the
// same straight-line code.  Lane indices are 32-bit (a chunk holds at most
// IPT * 256 elements).  f32 input: the max is taken on the floats themselves,
// the same comparisons on the same (exactly converted) values, so the same
// max; the f32 -inf start stands for the -DBL_MAX start (neither -inf nor NaN
// ever beats either).
template <int DIN, int IPT>
__device__ __forceinline__ void sm_chunk_partial(double (&v)[IPT], const void* __restrict__ X, int dtx, int64_t base,
                                                 int64_t L, int64_t chunk, int c, double* lds, double& mx, double& sum) {
    const int64_t j0 = c * chunk, j1 = j0 + chunk < L ? j0 + chunk : L;
    const int n = j1 > j0 ? (int)(j1 - j0) : 0;
    const int tid = (int)threadIdx.x;
    if constexpr (DIN == kF32) {
        const __amdgpu_buffer_rsrc_t xr = buffer_rsrc((const float*)X + base + j0, (uint32_t)n * 4u);
        float f[IPT];
#pragma unroll
        for (int t = 0; t < IPT; t++) {
            const float x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                          xr, (uint32_t)((tid + t * kSplitThreads) * 4), 0, 0));
            f[t] = tid + t * kSplitThreads < n ? x : -__builtin_inff();
        }
        float mf = -__builtin_inff();
#pragma unroll
        for (int t = 0; t < IPT; t++) mf = f[t] > mf ? f[t] : mf;
        mx = block_reduce<true, kSplitWaves>(mf == -__builtin_inff() ? -DBL_MAX : (double)mf, lds);
        sum = 0.0;
#pragma unroll
        for (int t = 0; t < IPT; t++) {
            v[t] = sm_exp((double)f[t] - mx);
            sum += v[t];
        }
    } else {
        load_chunk<DIN, IPT>(v, X, dtx, base, j0, j1);
        mx = -DBL_MAX;
#pragma unroll
        for (int t = 0; t < IPT; t++) {
            v[t] = tid + t * kSplitThreads < n ? v[t] : -__builtin_inf();
            mx = v[t] > mx ? v[t] : mx;
        }
        mx = block_reduce<true, kSplitWaves>(mx, lds);
        sum = 0.0;
#pragma unroll
        for (int t = 0; t < IPT; t++) {
            v[t] = sm_exp(v[t] - mx);
            sum += v[t];
        }
    }
    sum = block_reduce<false, kSplitWaves>(sum, lds);
}

template <int DIN, int IPT>
__global__ __launch_bounds__(kSplitThreads) void k_sm_part(const void* __restrict__ X, int dtx, int64_t L, int G,
                                                           double* __restrict__ part) {
    __shared__ double lds[kSplitWaves];
    const int64_t row = blockIdx.y, rows = gridDim.y, chunk = (L + G - 1) / G;
    const int64_t base = row * L;
    double mx = -DBL_MAX, sum = 0.0;
    if constexpr (IPT > 0) {
        double v[IPT];
        sm_chunk_partial<DIN, IPT>(v, X, dtx, base, L, chunk, (int)blockIdx.x, lds, mx, sum);
    } else {
        const int64_t j0 = blockIdx.x * chunk, j1 = j0 + chunk < L ? j0 + chunk : L;
        for (int64_t j = j0 + threadIdx.x; j < j1; j += kSplitThreads) {
            const double v = ldx<DIN>(X, base + j, dtx);
            mx = v > mx ? v : mx;
        }
        mx = block_reduce<true, kSplitWaves>(mx, lds);
        for (int64_t j = j0 + threadIdx.x; j < j1; j += kSplitThreads) sum += sm_exp(ldx<DIN>(X, base + j, dtx) - mx);
        sum = block_reduce<false, kSplitWaves>(sum, lds);
    }
    if (threadIdx.x == 0) {
        part[row * G + blockIdx.x] = mx;
        part[rows * G + row * G + blockIdx.x] = sum;
    }
}

// Split rows: pass 2.  Output exp(v - M) / S computed per chunk b as
// exp(v - m_b) * (exp(m_b - M) / S): a tolerance-class operator (~2e-7
// relative to the reference's double result), with one division per thread
// instead of an fp64 divide per element.
template <int DIN, int DOUT, int IPT>
__global__ __launch_bounds__(kSplitThreads) void k_sm_out(const void* __restrict__ X, int dtx, void* __restrict__ Y,
                                                          int dty, int64_t L, int G, const double* __restrict__ part) {
    const int64_t row = blockIdx.y, rows = gridDim.y, chunk = (L + G - 1) / G;
    const int64_t j0 = blockIdx.x * chunk, j1 = j0 + chunk < L ? j0 + chunk : L;
    const int64_t base = row * L;
    const double* pm = part + row * G;
    const double* ps = part + rows * G + row * G;
    // X first (independent of the partials), so its latency overlaps the fold
    double v[IPT > 0 ? IPT : 1];
    if constexpr (IPT > 0) load_chunk<DIN, IPT>(v, X, dtx, base, j0, j1);
    // Lane g folds partial g (G <= 64); every wave of every block of the row
    // runs the same butterfly on the same values, so all agree on M and S.
    const int lane = threadIdx.x & 63;
    const double m_l = lane < G ? pm[lane] : -DBL_MAX;
    const double M = wave_max(m_l);
    const double S = wave_sum(lane < G ? ps[lane] * sm_exp(m_l - M) : 0.0);
    // exp(v - M) / S as exp(v - m_b) * (exp(m_b - M) / S), m_b this chunk's
    // max: the one-launch kernel keeps exp(v - m_b) from its partial pass and
    // applies the same per-chunk factor, so the two forms return the same bits
    const double mb = pm[blockIdx.x];
    const double scale = sm_exp(mb - M) / S;
    if constexpr (IPT > 0) {
#pragma unroll
        for (int t = 0; t < IPT; t++) v[t] = sm_exp(v[t] - mb) * scale;
        store_chunk<DOUT, IPT>(Y, dty, base, j0, j1 > j0 ? (int)(j1 - j0) : 0, v);
    } else {
        for (int64_t j = j0 + threadIdx.x; j < j1; j += kSplitThreads)
            stx<DOUT>(Y, base + j, sm_exp(ldx<DIN>(X, base + j, dtx) - mb) * scale, dty);
    }
}

// Split rows in one launch (IPT > 0): block b of a row computes its chunk's
// partial (m_b, s_b) exactly as k_sm_part does, publishes it, waits for the
// row's other G - 1 partials, folds them exactly as k_sm_out does and writes
// its chunk from registers: X is read once and there is no second launch.
// Publication: four 64-bit words per block, (tag, high / low half of m_b),
// (tag, high / low half of s_b), written and polled with
// relaxed device-scope atomics (single-copy atomic words, coherent across the
// XCDs' L2s).  The tag is unique to the call, so a word is current exactly
// when it carries the call's tag: no fence, no zeroing, no reset of the
// workspace (stale words from earlier calls carry other tags).
// The wait is bounded (`spin` polls): if a partial has not appeared by then
// (the row's blocks are not all resident, e.g. other work fills the GPU), the
// whole block recomputes that chunk's partial from X with the same thread
// mapping and reduction order, which gives the same bits, so every block ends
// with the same (M, S) either way and every wave exits.
template <int DIN, int DOUT, int IPT>
__global__ __launch_bounds__(kSplitThreads) void k_sm_one(const void* __restrict__ X, int dtx, void* __restrict__ Y,
                                                          int dty, int64_t L, int G,
                                                          unsigned long long* __restrict__ slots, uint32_t tag,
                                                          int spin) {
    __shared__ double lds[kSplitWaves];
    __shared__ double fm[64], fs[64];          // partials recomputed by this block
    __shared__ unsigned long long s_missing;
    __shared__ double sM, sS;
    const int64_t row = blockIdx.y, chunk = (L + G - 1) / G;
    const int64_t base = row * L;
    const int64_t j0 = blockIdx.x * chunk, j1 = j0 + chunk < L ? j0 + chunk : L;
    double v[IPT];
    double mx, sum;
    sm_chunk_partial<DIN, IPT>(v, X, dtx, base, L, chunk, (int)blockIdx.x, lds, mx, sum);
    unsigned long long* rs = slots + (size_t)row * G * 4;
    if (threadIdx.x == 0) {
        const unsigned long long mb = __builtin_bit_cast(unsigned long long, mx);
        const unsigned long long sb = __builtin_bit_cast(unsigned long long, sum);
        xchg_pub(rs + blockIdx.x * 4 + 0, tag, (uint32_t)(mb >> 32));
        xchg_pub(rs + blockIdx.x * 4 + 1, tag, (uint32_t)mb);
        xchg_pub(rs + blockIdx.x * 4 + 2, tag, (uint32_t)(sb >> 32));
        xchg_pub(rs + blockIdx.x * 4 + 3, tag, (uint32_t)sb);
    }
    // Wave 0, lane g: wait for partial g (its own block's included).
    const int lane = threadIdx.x & 63;
    // lane g's partial: the published words, or the recomputed pair; lanes
    // past G hold the fold's neutral values
    const auto m_of = [&](uint32_t hi, uint32_t lo, const double* f, int l, bool h) {
        return l >= G ? -DBL_MAX : h ? __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo) : f[l];
    };
    const auto s_of = [&](uint32_t hi, uint32_t lo, const double* f, int l, bool h) {
        return l >= G ? 0.0 : h ? __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo) : f[l];
    };
    // the fold of k_sm_out, by wave 0 (all 64 lanes)
    const auto fold = [&](double m_l, double s_l) {
        const double M = wave_max(m_l);
        const double S = wave_sum(lane < G ? s_l * sm_exp(m_l - M) : 0.0);
        if (lane == 0) { sM = M; sS = S; }
    };
    uint32_t w0 = 0, w1 = 0, w2 = 0, w3 = 0;
    bool have = false;
    if (threadIdx.x < 64) {
        if (lane < G) {
            if (lane == (int)blockIdx.x) {
                const unsigned long long mb = __builtin_bit_cast(unsigned long long, mx);
                const unsigned long long sb = __builtin_bit_cast(unsigned long long, sum);
                w0 = (uint32_t)(mb >> 32);
                w1 = (uint32_t)mb;
                w2 = (uint32_t)(sb >> 32);
                w3 = (uint32_t)sb;
                have = true;
            }
            for (int it = 0; !have && it < spin; it++) {
                // four independent loads per poll (one round trip, not four in a row)
                const bool h0 = xchg_get(rs + lane * 4 + 0, tag, w0), h1 = xchg_get(rs + lane * 4 + 1, tag, w1);
                const bool h2 = xchg_get(rs + lane * 4 + 2, tag, w2), h3 = xchg_get(rs + lane * 4 + 3, tag, w3);
                have = h0 & h1 & h2 & h3;
                if (!have) __builtin_amdgcn_s_sleep(1);
            }
        } else {
            have = true;
        }
        const unsigned long long miss = __ballot(!have);
        // all partials here (the usual case): fold them now, so the block
        // needs a single barrier before the output
        if (miss == 0) fold(m_of(w0, w1, fm, lane, true), s_of(w2, w3, fs, lane, true));
        if (lane == 0) s_missing = miss;
    }
    __syncthreads();
    if (s_missing) {     // uniform over the block
        // Partials that did not arrive in time: recompute them here (uniform loop).
        for (unsigned long long miss = s_missing; miss; miss &= miss - 1) {
            const int c = __builtin_ctzll(miss);
            double w[IPT], m_c, s_c;
            sm_chunk_partial<DIN, IPT>(w, X, dtx, base, L, chunk, c, lds, m_c, s_c);
            if (threadIdx.x == 0) { fm[c] = m_c; fs[c] = s_c; }
        }
        __syncthreads();
        if (threadIdx.x < 64) fold(m_of(w0, w1, fm, lane, have), s_of(w2, w3, fs, lane, have));
        __syncthreads();
    }
    // v holds exp(v - m_b) from the partial pass (k_sm_out's per-chunk form)
    const double scale = sm_exp(mx - sM) / sS;
#pragma unroll
    for (int t = 0; t < IPT; t++) v[t] *= scale;
    store_chunk<DOUT, IPT>(Y, dty, base, j0, j1 > j0 ? (int)(j1 - j0) : 0, v);
}

// Workspace of split-row calls captured into a graph: the (m_b, s_b) partials
// of k_sm_part / k_sm_out, in a file-scope device array (each GPU holds its own
// copy until the process ends), since a captured call's workspace must outlive
// the call.  Host code uses only the address resolved at initialisation
// (g_sm_capture_ws); replays of captured split-row calls that overlap on one
// GPU share it and race.  Nothing in it needs to start at zero: k_sm_part
// writes every partial that k_sm_out reads.
constexpr int kSmCaptureParts = 2 * 1024;                  // (m, s) pairs of up to 1024 row chunks
static __device__ __align__(256) double sm_capture_ws[kSmCaptureParts];
double* g_sm_capture_ws = nullptr;

// Returns false when the workspace cannot be had (error set).
template <int DIN, int DOUT, int IPT>
bool launch_split_ipt(const void* x, int dtx, void* y, int dty, int64_t L, int G, dim3 g, hipStream_t s) {
    const bool captured = stream_capturing(s);
    if (IPT > 0 && !captured) {
        uint32_t tag = 0;
        unsigned long long* slots =
            (unsigned long long*)xchg_alloc(sizeof(unsigned long long) * 4 * (size_t)g.y * (size_t)G, &tag);
        if (!slots) return false;
        if constexpr (IPT > 0)
            hipLaunchKernelGGL((k_sm_one<DIN, DOUT, IPT>), g, dim3(kSplitThreads), 0, s, x, dtx, y, dty, L, G, slots,
                               tag, exchange_spin());
        xchg_free(slots);   // stream-ordered reuse: later work on this stream runs after the kernel
        return true;
    }
    const size_t nparts = 2 * (size_t)g.y * (size_t)G;
    double* part;
    if (captured) {
        if (nparts > (size_t)kSmCaptureParts) { set_error("softmax: %zu partials exceed the capture workspace", nparts); return false; }
        if (!(part = g_sm_capture_ws)) { set_error("softmax: capture workspace unavailable"); return false; }
    } else if (!(part = (double*)pool_alloc(sizeof(double) * nparts))) {
        return false;
    }
    hipLaunchKernelGGL((k_sm_part<DIN, IPT>), g, dim3(kSplitThreads), 0, s, x, dtx, L, G, part);
    hipLaunchKernelGGL((k_sm_out<DIN, DOUT, IPT>), g, dim3(kSplitThreads), 0, s, x, dtx, y, dty, L, G, part);
    if (!captured) pool_free(part);
    return true;
}

template <int DIN, int DOUT>
bool launch_split(const void* x, int dtx, void* y, int dty, int64_t L, int G, dim3 g, hipStream_t s) {
    const int64_t ipt = ((L + G - 1) / G + kSplitThreads - 1) / kSplitThreads;
    if (ipt <= 4) return launch_split_ipt<DIN, DOUT, 4>(x, dtx, y, dty, L, G, g, s);
    if (ipt <= 8) return launch_split_ipt<DIN, DOUT, 8>(x, dtx, y, dty, L, G, g, s);
    if (ipt <= 16) return launch_split_ipt<DIN, DOUT, 16>(x, dtx, y, dty, L, G, g, s);
    return launch_split_ipt<DIN, DOUT, 0>(x, dtx, y, dty, L, G, g, s);
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
    for (int64_t j = 0; j < L; j++) sum += sm_exp(ld_d_rt(dtx, X, base + j * inner) - mx);
    for (int64_t j = 0; j < L; j++) {
        const int64_t i = base + j * inner;
        st_d_rt(dty, Y, i, sm_exp(ld_d_rt(dtx, X, i) - mx) / sum);
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

constexpr int kPoolRows = 4;   // output rows per 256-thread block (one per wave)

// Any window: wave per output row, lane per output column.
template <int DIN, int DOUT>
__global__ __launch_bounds__(256) void k_maxpool_rows(const void* __restrict__ X, int dtx, void* __restrict__ Y,
                                                      int dty, PoolGeom g, int64_t planes) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int oh = blockIdx.x * kPoolRows + wave;
    if (oh >= g.OH) return;
    for (int64_t plane = blockIdx.y; plane < planes; plane += gridDim.y) {
        const int64_t xb = plane * (int64_t)g.H * g.W;
        const int64_t yb = (plane * g.OH + oh) * (int64_t)g.OW;
        for (int ow = lane; ow < g.OW; ow += 64) {
            double best = -__builtin_inf();
            for (int kh = 0; kh < g.KH; kh++) {
                const int ih = oh * g.sh + kh * g.dh - g.pt;
                if (ih < 0 || ih >= g.H) continue;
                const int64_t rb = xb + (int64_t)ih * g.W;
                for (int kw = 0; kw < g.KW; kw++) {
                    const int iw = ow * g.sw + kw * g.dw - g.pl;
                    if (iw < 0 || iw >= g.W) continue;
                    const double v = ldx<DIN>(X, rb + iw, dtx);
                    if (v > best) best = v;
                }
            }
            stx<DOUT>(Y, yb + ow, best, dty);
        }
    }
}

// f32, 3x3 window, stride 2, top/left pad 1, W == 2 * OW, OW <= 64: lane l
// loads columns (2l, 2l+1) of each input row with one 8-byte load and takes
// column 2l-1 from lane l-1 (lane 0: the left padding, skipped).
__global__ __launch_bounds__(256) void k_maxpool_3s2(const float* __restrict__ X, float* __restrict__ Y, PoolGeom g,
                                                     int64_t planes) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int oh = blockIdx.x * kPoolRows + wave;
    if (oh >= g.OH) return;
    const bool live = lane < g.OW;
    for (int64_t plane = blockIdx.y; plane < planes; plane += gridDim.y) {
        const float* xp = X + plane * (int64_t)g.H * g.W;
        float best = -__builtin_inff();
#pragma unroll
        for (int kh = 0; kh < 3; kh++) {
            const int ih = 2 * oh - 1 + kh;                     // uniform across the wave
            if (ih < 0 || ih >= g.H) continue;
            float2 v = make_float2(-__builtin_inff(), -__builtin_inff());
            if (live) v = *reinterpret_cast<const float2*>(xp + (int64_t)ih * g.W + 2 * lane);
            const float left = lane_prev(v.y);
            if (lane > 0 && left > best) best = left;           // kw = 0: column 2l - 1
            if (v.x > best) best = v.x;                          // kw = 1: column 2l
            if (v.y > best) best = v.y;                          // kw = 2: column 2l + 1
        }
        if (live) Y[(plane * g.OH + oh) * (int64_t)g.OW + lane] = best;
    }
}

constexpr int kPoolStrip = 8;           // output rows per wave of the strip kernel
constexpr int kPoolStripWaves = 8;      // waves per plane: OH <= 64

// f32, 3x3 window, stride 2, top/left pad 1, W == 2 * OW, OW <= 64, OH <= 64:
// one block per plane, wave w takes a strip of output rows.  Output row oh reads
// input rows 2oh-1, 2oh, 2oh+1; consecutive output rows share one, so every
// input row of the strip is loaded once, as one 8-byte load per lane (columns
// 2l, 2l+1; column 2l-1 comes from lane l-1).  FQ: each output value is also
// written fake-quantized (fq_apply) to Yq.
template <bool FQ>
__global__ __launch_bounds__(64 * kPoolStripWaves) void k_maxpool_3s2_strip(const float* __restrict__ X, float* __restrict__ Y,
                                                           PoolGeom g, int rows_per_wave, float* __restrict__ Yq,
                                                           FakeQuant fq) {
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int64_t plane = blockIdx.x;
    const uint32_t pin = (uint32_t)g.H * g.W, pout = (uint32_t)g.OH * g.OW;
    // the plane's input and output through buffer resources: a row's offset is
    // a scalar (soffset), each lane's column a fixed voffset, and the loads of
    // lanes past the row (lane >= OW) stay inside the plane or read zero
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X + plane * pin, pin * 4u);
    float* yp = Y + plane * (int64_t)pout;
    // (a wave without output rows still takes part in the block's barrier)
    const int oh0 = wave * rows_per_wave, oh1 = min(g.OH, oh0 + rows_per_wave);
    const float ninf = -__builtin_inff();
    const uint32_t lo = (uint32_t)lane * 8u;
    // Input row ih as (column 2l, column 2l+1) per lane; a row outside the
    // plane (the top padding row) is -inf, which never wins a strict >.  Each
    // input row is read once: streaming (nontemporal) loads.
    auto ldrow = [&](int ih) {
        float2 v = make_float2(ninf, ninf);
        if ((unsigned)ih < (unsigned)g.H) {     // uniform
            const uint64_t w = __builtin_bit_cast(
                uint64_t, __builtin_amdgcn_raw_buffer_load_b64(xr, lo, (uint32_t)ih * (uint32_t)g.W * 4u, 2 /* nt */));
            v = make_float2(__builtin_bit_cast(float, (uint32_t)w), __builtin_bit_cast(float, (uint32_t)(w >> 32)));
        }
        return v;
    };
    // Taps of one input row in the reference's kw order: 2l-1 (lane l-1's
    // second column; lane 0 gets -inf, the left padding), 2l, 2l+1.
    auto row_max = [&](float best, float2 v) {
        const float left = __builtin_bit_cast(
            float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, ninf), __builtin_bit_cast(int, v.y), 0x138 /* wave_shr:1 */,
                                               0xF, 0xF, false));
        best = left > best ? left : best;
        best = v.x > best ? v.x : best;
        best = v.y > best ? v.y : best;
        return best;
    };
    FQParm fqp;
    if constexpr (FQ) fqp = fq_parm(fq);
    // The whole strip (2 * rows + 1 input rows) is loaded up front: a wave
    // waits for memory once instead of once per output row.  Its last input
    // row is the next wave's first: that wave publishes it through LDS, so
    // every input row leaves HBM once (23.7 -> 23.1 us at config 4; the
    // plane's last wave loads its last row itself).
    __shared__ float2 edge[kPoolStripWaves][64];
    float2 rows[2 * kPoolStrip + 1];
    const int nrows = 2 * (oh1 - oh0) + 1;
    const bool own_last = oh1 == g.OH;
#pragma unroll
    for (int j = 0; j < 2 * kPoolStrip + 1; j++)
        rows[j] = (j < nrows - 1 || (j == nrows - 1 && own_last)) ? ldrow(2 * oh0 - 1 + j) : make_float2(ninf, ninf);
    if (wave > 0) edge[wave - 1][lane] = rows[0];
    __syncthreads();
    if (!own_last) {
#pragma unroll
        for (int j = 0; j < 2 * kPoolStrip + 1; j++)
            if (j == nrows - 1) rows[j] = edge[wave][lane];
    }
    const bool live = lane < g.OW;
#pragma unroll
    for (int o = 0; o < kPoolStrip; o++) {
        const int oh = oh0 + o;
        if (oh >= oh1) break;
        // rows 2oh-1, 2oh, 2oh+1; those past the plane's last row are -inf
        const float best = row_max(row_max(row_max(ninf, rows[2 * o]), rows[2 * o + 1]), rows[2 * o + 2]);
        if (live) {
            if constexpr (FQ) {
                yp[(int64_t)oh * g.OW + lane] = best;
                Yq[plane * (int64_t)pout + (int64_t)oh * g.OW + lane] = fq_apply(best, fqp);
            } else {
                // nontemporal: the output is not read back here (24.2 -> 23.7 us)
                __builtin_nontemporal_store(best, &yp[(int64_t)oh * g.OW + lane]);
            }
        }
    }
}

// ------------------------------------------------------------ GlobalAveragePool ---
// tensor_ops.c:2844-2868: each of the N*C planes summed in double in index
// order, then divided by H*W.  A block takes 64 consecutive planes (thread t
// owns plane p0 + t, so the sum keeps the reference's order and is bit-exact);
// the planes, contiguous in memory, are staged through LDS 64 elements per
// plane at a time (one pass for planes up to 8x8) with loads that are
// coalesced across the wave.
constexpr int kGapPlanes = 64, kGapChunk = 64;

template <int DIN, int DOUT>
__global__ __launch_bounds__(kGapPlanes) void k_gap(const void* __restrict__ X, int dtx, void* __restrict__ Y, int dty,
                                                    int64_t planes, int hw) {
    __shared__ double tile[kGapPlanes][kGapChunk + 1];
    const int t = threadIdx.x;
    const int64_t p0 = (int64_t)blockIdx.x * kGapPlanes;
    const int64_t np = planes - p0 < kGapPlanes ? planes - p0 : kGapPlanes;
    double sum = 0.0;
    for (int c0 = 0; c0 < hw; c0 += kGapChunk) {
        const int cn = hw - c0 < kGapChunk ? hw - c0 : kGapChunk;
#pragma unroll
        for (int i = 0; i < kGapChunk; i++) {
            const int e = t + i * kGapPlanes;               // element e of the 256 x 16 tile
            const int p = e / kGapChunk, k = e % kGapChunk;
            if (p < np && k < cn) tile[p][k] = ldx<DIN>(X, (p0 + p) * hw + c0 + k, dtx);
        }
        __syncthreads();
        for (int k = 0; k < cn; k++) sum += tile[t][k];
        __syncthreads();
    }
    if (t < np) stx<DOUT>(Y, p0 + t, sum / hw, dty);
}

// f32 planes of at most 128 values: a block's 64 planes are one contiguous
// region, copied into LDS by its four waves, then lane l of the first wave sums
// plane l from LDS in index order (the same exact sequential sum).  A full
// block of a 16-byte aligned X (ALIGNED; its region starts 256 hw b bytes past
// X and holds 64 hw values, a multiple of 4, so every 16-byte piece is wholly
// inside or wholly past it) copies it with buffer loads that write LDS
// directly, 64 lanes x 16 bytes per load, no register round trip
// ([64,512,7,7]: 3.83 -> 3.45 us); otherwise coalesced 4-byte loads (up to 16
// per thread in flight, so a region of up to 64 x 64 values arrives in one
// round trip) and LDS stores.
constexpr int kGapSmallHW = 128, kGapSmallThreads = 256;

template <int DOUT, bool ALIGNED>
__global__ __launch_bounds__(kGapSmallThreads) void k_gap_small_f32(const float* __restrict__ X, void* __restrict__ Y,
                                                                    int dty, int64_t planes, int hw) {
    __shared__ __attribute__((aligned(16))) float tile[64 * kGapSmallHW];
    const int t = threadIdx.x;
    const int64_t p0 = (int64_t)blockIdx.x * 64;
    const int np = planes - p0 < 64 ? (int)(planes - p0) : 64;
    const int cnt = np * hw;
    // buffer loads: reads past the region return 0 without touching memory
    const __amdgpu_buffer_rsrc_t r = buffer_rsrc(X + p0 * hw, (uint32_t)cnt * 4u);
    if (ALIGNED && np == 64) {       // uniform over the block
        const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
        const uint32_t lane = (uint32_t)t & 63u;
        for (int c = wave; c < (cnt + 255) / 256; c += kGapSmallThreads / 64)    // chunk c: values 256 c ..
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(tile + 256 * c), 16,
                                                     (uint32_t)(256 * c * 4) + lane * 16u, 0, 0, 0);
        __builtin_amdgcn_s_waitcnt(0x3f70);    // vmcnt(0): this wave's chunks are in LDS
    } else {
        for (int base = 0; base < cnt; base += kGapSmallThreads * 16) {
            float v[16];
#pragma unroll
            for (int j = 0; j < 16; j++)
                v[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                     r, (uint32_t)(base + t + kGapSmallThreads * j) * 4u, 0, 0));
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int i = base + t + kGapSmallThreads * j;
                if (i < cnt) tile[i] = v[j];
            }
        }
    }
    __syncthreads();
    if (t < np) {
        const float* tp = tile + t * hw;
        double sum = 0.0;
        int k = 0;
        for (; k + 4 <= hw; k += 4) {
            const float a = tp[k], b = tp[k + 1], c = tp[k + 2], d = tp[k + 3];
            sum += (double)a;
            sum += (double)b;
            sum += (double)c;
            sum += (double)d;
        }
        for (; k < hw; k++) sum += (double)tp[k];
        stx<DOUT>(Y, p0 + t, sum / hw, dty);
    }
}

// Gemm -> Softmax (last axis) with the Gemm's k split: one block per row adds
// the row's slice sums and the bias as k_splitk_reduce does (double sum in
// slice order, alpha * acc + beta * c, rounded to f32), writes the logits, and
// takes the row's softmax as k_softmax_row<1> does (max from -DBL_MAX with a
// strict >, sm_exp, the block sums, one reciprocal): both outputs equal the
// two launches they replace bit for bit.  cmode: 0 no bias, 1 one value, 2 per
// column, 3 per row.  N <= kRowThreads.
__global__ __launch_bounds__(kRowThreads) void k_splitk_softmax(const float* __restrict__ part, int nsplit, int M,
                                                                int N, double alpha, double beta,
                                                                const float* __restrict__ c, int cmode,
                                                                float* __restrict__ Y, float* __restrict__ P) {
    __shared__ double lds[kWaves];
    const int m = blockIdx.x, j = threadIdx.x;
    const int64_t mn = (int64_t)M * N, i = (int64_t)m * N + j;
    double v = -DBL_MAX;
    if (j < N) {
        double acc = 0.0;
        for (int sp = 0; sp < nsplit; sp++) acc += (double)part[(int64_t)sp * mn + i];
        double r = alpha * acc;
        if (cmode) r += beta * (double)c[cmode == 1 ? 0 : (cmode == 2 ? j : m)];
        const float y = (float)r;
        Y[i] = y;
        v = (double)y;
    }
    double mx = -DBL_MAX;
    mx = v > mx ? v : mx;
    mx = block_reduce<true, kWaves>(mx, lds);
    const double e = j < N ? sm_exp(v - mx) : 0.0;
    const double sum = block_reduce<false, kWaves>(e, lds);
    const double rs = 1.0 / sum;
    if (j < N) P[i] = (float)(e * rs);
}

}  // namespace

bool launch_splitk_softmax(const float* part, int nsplit, int M, int N, double alpha, double beta, const float* c,
                           int cmode, float* Y, float* P, hipStream_t s) {
    if (N < 1 || N > kRowThreads || M < 1 || cmode < 0 || cmode > 3) return false;
    hipLaunchKernelGGL(k_splitk_softmax, dim3((unsigned)M), dim3(kRowThreads), 0, s, part, nsplit, M, N, alpha, beta, c,
                       cmode, Y, P);
    return true;
}

// Resolves sm_capture_ws on the library's device (current during initialisation).
void init_reduce_workspace() {
    void* p = nullptr;
    if (check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(sm_capture_ws)), "hipGetSymbolAddress(sm_capture_ws)"))
        g_sm_capture_ws = (double*)p;
}
}  // namespace tohip

using namespace tohip;

extern "C" {

void global_average_pool_forward(const Tensor* input, Tensor* output) {
    const char* name = "global_average_pool_forward";
    if (!tensor_sane(input, name) || !tensor_sane(output, name)) return;
    if (input->ndim != 4) { set_error("%s: input must be 4-D (the reference leaves the output untouched)", name); return; }
    const int64_t planes = (int64_t)input->shape[0] * input->shape[1];
    const int hw = input->shape[2] * input->shape[3];
    if (output->size < (size_t)planes) { set_error("%s: output holds %zu of %lld values", name, output->size, (long long)planes); return; }
    if (!ensure_device()) return;
    Staging st;
    const void* x = st.in(input);
    void* y = st.out(output, (size_t)planes * dt_bytes((int)output->dtype));
    if (!x || !y) { st.finish(); return; }
    if (planes > 0) {
        const dim3 g((unsigned)((planes + kGapPlanes - 1) / kGapPlanes)), b(kGapPlanes);
        const int dtx = (int)input->dtype, dty = (int)output->dtype;
        hipStream_t s = stream();
        const dim3 gs((unsigned)((planes + 63) / 64)), bs(kGapSmallThreads);
        const bool al16 = ((uintptr_t)x & 15) == 0;
        if (dtx == kF32 && hw <= kGapSmallHW && dty == kF32 && al16)
            hipLaunchKernelGGL((k_gap_small_f32<kF32, true>), gs, bs, 0, s, (const float*)x, y, dty, planes, hw);
        else if (dtx == kF32 && hw <= kGapSmallHW && dty == kF32)
            hipLaunchKernelGGL((k_gap_small_f32<kF32, false>), gs, bs, 0, s, (const float*)x, y, dty, planes, hw);
        else if (dtx == kF32 && hw <= kGapSmallHW)
            hipLaunchKernelGGL((k_gap_small_f32<-1, false>), gs, bs, 0, s, (const float*)x, y, dty, planes, hw);
        else if (dtx == kF32 && dty == kF32)
            hipLaunchKernelGGL((k_gap<kF32, kF32>), g, b, 0, s, x, dtx, y, dty, planes, hw);
        else
            hipLaunchKernelGGL((k_gap<-1, -1>), g, b, 0, s, x, dtx, y, dty, planes, hw);
        if (!check_launch(name)) { st.finish(); return; }
    }
    st.finish();
}



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
        // Split rows over G blocks when there are too few rows to fill the chip:
        // about two blocks per CU ([64, 32000]: G = 8 took 8.3 us, G = 16 9.0 us,
        // G = 4 8.6 us, before nontemporal stores).
        int G = 1;
        if (inner == 1 && outer < num_cus() / 2 && outer <= 65535) {
            G = (int)((2 * num_cus() + outer - 1) / outer);
            const int64_t gmax = (L + 1023) / 1024;            // at least ~1K elements per block
            if (G > gmax) G = (int)gmax;
            if (G > 64) G = 64;
        }
        // (a captured call keeps its partials in the fixed capture workspace)
        if (G > 1 && 2 * outer * G > kSmCaptureParts && stream_capturing(s)) G = 1;
        if (inner == 1 && G > 1) {
            const dim3 g((unsigned)G, (unsigned)outer);
            bool ok;
            if (dtx == kF32 && dty == kF32) ok = launch_split<kF32, kF32>(x, dtx, y, dty, L, G, g, s);
            else if (dtx == kF32) ok = launch_split<kF32, -1>(x, dtx, y, dty, L, G, g, s);
            else ok = launch_split<-1, -1>(x, dtx, y, dty, L, G, g, s);
            if (!ok || !check_launch(name)) { st.finish(); return; }
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

}  // extern "C"

namespace {
// max_pool_forward; with fq_kind 1 / 2 (uint8 / int8 codes, parameters fq_t =
// {q scale, q zero point, d scale, d zero point} of one element each) the strip
// kernel also writes Yq = fake quantization of Y.  Returns whether it did.
bool maxpool_entry(const char* name, const Tensor* X, Tensor* Y, PoolParams* p, Tensor* Yq = nullptr, int fq_kind = 0,
                   const Tensor* const* fq_t = nullptr) {
    if (!tensor_sane(X, name) || !tensor_sane(Y, name)) return false;
    if (!p || !p->pads || !p->strides || !p->dilations || !p->kernel_shape) { set_error("%s: NULL params", name); return false; }
    if (X->ndim != 4 || Y->ndim != 4) { set_error("%s: X and Y must be 4-D (NCHW)", name); return false; }
    PoolGeom g;
    g.N = X->shape[0]; g.C = X->shape[1]; g.H = X->shape[2]; g.W = X->shape[3];
    g.OH = Y->shape[2]; g.OW = Y->shape[3];
    g.KH = p->kernel_shape[0]; g.KW = p->kernel_shape[1];
    g.pt = p->pads[0]; g.pl = p->pads[1]; g.sh = p->strides[0]; g.sw = p->strides[1];
    g.dh = p->dilations[0]; g.dw = p->dilations[1];
    if (Y->shape[0] != g.N || Y->shape[1] != g.C) { set_error("%s: Y batch/channels differ from X", name); return false; }
    if (!ensure_device()) return false;
    const int64_t planes = (int64_t)g.N * g.C;
    const int64_t total = planes * g.OH * g.OW;
    Staging st;
    const void* x = st.in(X);
    void* y = st.out(Y, (size_t)total * dt_bytes((int)Y->dtype));
    if (!x || !y) { st.finish(); return false; }
    hipStream_t s = stream();
    bool fq_done = false;
    if (total > 0) {
        const dim3 grid((unsigned)((g.OH + kPoolRows - 1) / kPoolRows), (unsigned)(planes < 65535 ? planes : 65535));
        const dim3 blk(256);
        const int dtx = (int)X->dtype, dty = (int)Y->dtype;
        const bool f32 = dtx == kF32 && dty == kF32;
        const bool res3s2 = f32 && g.KH == 3 && g.KW == 3 && g.sh == 2 && g.sw == 2 && g.dh == 1 && g.dw == 1 &&
                            g.pt == 1 && g.pl == 1 && g.W == 2 * g.OW && g.OW <= 64 && 2 * g.OH <= g.H + 2 &&
                            ((uintptr_t)x & 7) == 0;
        const int strip = (g.OH + kPoolStripWaves - 1) / kPoolStripWaves;
        const FakeQuant none{nullptr, nullptr, nullptr, nullptr, 0};
        if (res3s2 && planes <= 0x7FFFFFFF && strip <= kPoolStrip && fq_kind) {
            const void* fqd[4];
            for (int k = 0; k < 4; k++) fqd[k] = st.in(fq_t[k]);
            void* yq = st.out(Yq, (size_t)total * 4);
            if (!fqd[0] || !fqd[1] || !fqd[2] || !fqd[3] || !yq) { st.finish(); return false; }
            const FakeQuant fq{(const float*)fqd[0], fqd[1], (const float*)fqd[2], fqd[3], fq_kind};
            hipLaunchKernelGGL(k_maxpool_3s2_strip<true>, dim3((unsigned)planes), dim3(64 * kPoolStripWaves), 0, s,
                               (const float*)x, (float*)y, g, strip, (float*)yq, fq);
            fq_done = true;
        } else if (res3s2 && planes <= 0x7FFFFFFF && strip <= kPoolStrip)
            hipLaunchKernelGGL(k_maxpool_3s2_strip<false>, dim3((unsigned)planes), dim3(64 * kPoolStripWaves), 0, s,
                               (const float*)x, (float*)y, g, strip, nullptr, none);
        else if (res3s2)
            hipLaunchKernelGGL(k_maxpool_3s2, grid, blk, 0, s, (const float*)x, (float*)y, g, planes);
        else if (f32)
            hipLaunchKernelGGL((k_maxpool_rows<kF32, kF32>), grid, blk, 0, s, x, dtx, y, dty, g, planes);
        else
            hipLaunchKernelGGL((k_maxpool_rows<-1, -1>), grid, blk, 0, s, x, dtx, y, dty, g, planes);
        if (!check_launch(name)) { st.finish(); return false; }
    }
    st.finish();
    return fq_done;
}
}  // namespace

extern "C" {
void max_pool_forward(const Tensor* X, Tensor* Y, PoolParams* p) { maxpool_entry("max_pool_forward", X, Y, p); }

// MaxPool with a second, fake-quantized output; see tensor_ops.h.  The strip
// kernel writes both for the 3x3 / stride-2 case with uint8 / int8 codes and
// one-element f32 scales and zero points of the code dtype; otherwise
// max_pool_forward then quantize_dequantize_linear_forward(Y -> Yq).
void max_pool_qdq_forward(const Tensor* X, Tensor* Y, PoolParams* p, const Tensor* QScale, const Tensor* QZeroPoint,
                          const Tensor* DScale, const Tensor* DZeroPoint, int code_dtype, Tensor* Yq) {
    const char* name = "max_pool_qdq_forward";
    if (!tensor_sane(QScale, name) || !tensor_sane(QZeroPoint, name) || !tensor_sane(DScale, name) ||
        !tensor_sane(DZeroPoint, name) || !tensor_sane(Y, name) || !tensor_sane(Yq, name))
        return;
    if (Yq->size != Y->size) { set_error("%s: Yq must have Y's size", name); return; }
    const int kind = code_dtype == kU8 ? 1 : (code_dtype == kI8 ? 2 : 0);
    const bool fq_ok = kind && Y->dtype == kF32 && Yq->dtype == kF32 && QScale->dtype == kF32 &&
                       DScale->dtype == kF32 && QScale->size == 1 && DScale->size == 1 && QZeroPoint->size == 1 &&
                       DZeroPoint->size == 1 && (int)QZeroPoint->dtype == code_dtype &&
                       (int)DZeroPoint->dtype == code_dtype;
    const Tensor* fq_t[4] = {QScale, QZeroPoint, DScale, DZeroPoint};
    tensor_ops_hip_clear_error();
    const bool done = maxpool_entry(name, X, Y, p, Yq, fq_ok ? kind : 0, fq_t);
    if (!done && !tensor_ops_hip_last_error()[0])
        quantize_dequantize_linear_forward(Y, QScale, QZeroPoint, DScale, DZeroPoint, Yq, code_dtype);
}

}  // extern "C"
