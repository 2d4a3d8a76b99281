/*
 * tensor_ops_oracle.c — CPU restatement of the reference tensor_ops hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the GPU library is
 * compared against: only tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline leg may load it.  The product library (libtensor_ops_hip.so) never
 * links, calls or falls back to it.
 *
 * It exports the same C symbols as the reference library (create_tensor,
 * add_forward, ...) so a test can drive both through one ctypes binding.  Each
 * function cites the reference lines (tensor_ops/tensor_ops.c) whose behaviour
 * it restates.  The code is written from the observed semantics; where the
 * steps of an encoder must match, they produce the same bits by a formulation
 * of our own (checked by exhaustive sweeps against the compiled reference).
 *
 * Pinning (see tests/test_oracle.py):
 *   codecs       exhaustive 2^32 / 2^16 / 2^8 sweeps vs oracle/_ref and golden digests
 *   elementwise  golden vectors from oracle/_ref + closed forms (IEEE fp32 ops)
 *   cos          golden vectors from oracle/_ref (bit-exact LUT replica)
 *   Q/DQ         golden vectors + numpy float64 restatement + Appendix KATs
 *   conv/pool/gemm/softmax  golden vectors + numpy float64 brute force
 *   exp (softmax) uses the host libm exp, as the reference does: parity of exp
 *                 itself is unpinned (tolerance only).
 */
#include "../include/tensor_ops.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef union { float f; uint32_t u; } f32bits;

static inline uint32_t fbits(float f) { f32bits b; b.f = f; return b.u; }
static inline float bitsf(uint32_t u) { f32bits b; b.u = u; return b.f; }

/* ---------------- element sizes (tensor_ops.c:34-55, 383-423) ---------------- */
static size_t elem_bytes(int dt) {
    switch (dt) {
    case DTYPE_FLOAT16: case DTYPE_BFLOAT16: case DTYPE_INT16: return 2;
    case DTYPE_FLOAT32: case DTYPE_INT32: return 4;
    case DTYPE_FLOAT64: case DTYPE_INT64: return 8;
    case DTYPE_FLOAT8_E4M3: case DTYPE_FLOAT8_E5M2:
    case DTYPE_INT4: case DTYPE_INT8: case DTYPE_UINT8: return 1;
    default: return 4;
    }
}

static int is_int_dtype(int dt) {          /* tensor_ops.c:591 */
    return dt == DTYPE_INT4 || dt == DTYPE_INT8 || dt == DTYPE_UINT8 ||
           dt == DTYPE_INT16 || dt == DTYPE_INT32 || dt == DTYPE_INT64;
}

/* ---------------- integer clamps (tensor_ops.c:64-96) ---------------- */
static inline int64_t clamp_i64(int64_t v, int64_t lo, int64_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

/* x86-64 cvttsd2si semantics of (int64_t)d: values outside [-2^63, 2^63) and
 * NaN give INT64_MIN ("integer indefinite").  The reference relies on this
 * implicitly at tensor_ops.c:520-546 and 580-585. */
static inline int64_t trunc_i64_x86(double d) {
    if (d >= -9223372036854775808.0 && d < 9223372036854775808.0) return (int64_t)d;
    return INT64_MIN;
}

/* ---------------- f16 (tensor_ops.c:104-184) ---------------- */
/* Round-to-nearest-even f32 -> f16.  Quirks kept from the reference:
 * |x| < 2^-24 becomes a signed zero (a true RNE gives the smallest subnormal
 * for |x| in (2^-25, 2^-24)); any NaN becomes sign|0x7FFF. */
static uint16_t enc_f16(float f) {
    uint32_t u = fbits(f);
    uint16_t s = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return s | 0x7FFF;
    if (a == 0x7F800000u) return s | 0x7C00;
    uint32_t bexp = a >> 23;
    if (bexp == 0) return s;                        /* f32 zero / subnormal */
    int e = (int)bexp - 127;
    if (e <= -25) return s;
    uint32_t sig = (a & 0x7FFFFFu) | 0x800000u;    /* 24-bit significand */
    int drop = (e >= -14) ? 13 : (-1 - e);         /* 13..23 bits dropped */
    uint32_t q = sig >> drop;
    uint32_t rem = sig & ((1u << drop) - 1u);
    uint32_t half = 1u << (drop - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    uint32_t code;
    if (e >= -14) code = ((uint32_t)(e + 15) << 10) + (q - 0x400u);  /* carry ripples into exp */
    else code = q;                                  /* subnormal; 0x400 = min normal */
    if (code >= 0x7C00u) return s | 0x7C00;
    return (uint16_t)(s | code);
}

static float dec_f16(uint16_t h) {
    uint32_t s = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 31) return bitsf(s | 0x7F800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return bitsf(s);
        float v = (float)m * 0x1p-24f;              /* exact */
        return s ? -v : v;
    }
    return bitsf(s | ((e + 112u) << 23) | (m << 13));
}

/* ---------------- bf16 (tensor_ops.c:192-228) ---------------- */
static uint16_t enc_bf16(float f) {
    uint32_t u = fbits(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t r = u + 0x7FFFu + ((u >> 16) & 1u);  /* RNE on the low 16 bits */
    return (uint16_t)(r >> 16);
}

static float dec_bf16(uint16_t h) { return bitsf((uint32_t)h << 16); }

/* ---------------- fp8 e4m3 (tensor_ops.c:236-287) ---------------- */
/* RNE; magnitudes below 2^-6 flush to signed zero (no subnormal codes are
 * produced); overflow and inf saturate to 0x7E (448); NaN -> 0x7F | sign. */
static uint8_t enc_e4m3(float f) {
    uint32_t u = fbits(f);
    uint8_t s = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return s | 0x7F;
    uint32_t bexp = a >> 23;
    if (bexp == 0) return s;
    int e = (int)bexp - 127;
    if (e < -6) return s;
    if (e > 8) return s | 0x7E;
    uint32_t sig = (a & 0x7FFFFFu) | 0x800000u;
    uint32_t q = sig >> 20, rem = sig & 0xFFFFFu;
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) q++;
    uint32_t code = ((uint32_t)(e + 7) << 3) + (q - 8u);
    if (code > 0x7Eu) code = 0x7E;
    return (uint8_t)(s | code);
}

static float dec_e4m3(uint8_t c) {
    uint32_t s = ((uint32_t)c & 0x80u) << 24;
    uint32_t e = (c >> 3) & 0xFu, m = c & 7u;
    if (e == 15 && m == 7) return bitsf(s | 0x7FC00000u);
    float v = (e == 0) ? (float)m * 0x1p-9f : bitsf(((e + 120u) << 23) | (m << 20));
    return s ? -v : v;
}

/* ---------------- fp8 e5m2 (tensor_ops.c:295-347) ---------------- */
/* RNE; magnitudes below 2^-14 flush to signed zero; no saturation: results
 * that round to >= 2^16 and inf give 0x7C | sign; NaN -> 0x7D | sign. */
static uint8_t enc_e5m2(float f) {
    uint32_t u = fbits(f);
    uint8_t s = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return s | 0x7D;
    if (a == 0x7F800000u) return s | 0x7C;
    uint32_t bexp = a >> 23;
    if (bexp == 0) return s;
    int e = (int)bexp - 127;
    if (e < -14) return s;
    if (e > 15) return s | 0x7C;
    uint32_t sig = (a & 0x7FFFFFu) | 0x800000u;
    uint32_t q = sig >> 21, rem = sig & 0x1FFFFFu;
    if (rem > 0x100000u || (rem == 0x100000u && (q & 1u))) q++;
    uint32_t code = ((uint32_t)(e + 15) << 2) + (q - 4u);
    if (code > 0x7Cu) code = 0x7C;
    return (uint8_t)(s | code);
}

static float dec_e5m2(uint8_t c) {
    uint32_t s = ((uint32_t)c & 0x80u) << 24;
    uint32_t e = (c >> 2) & 0x1Fu, m = c & 3u;
    if (e == 31) return bitsf(s | 0x7F800000u | (m << 21) | (m ? 0x400000u : 0u));
    float v = (e == 0) ? (float)m * 0x1p-16f : bitsf(((e + 112u) << 23) | (m << 21));
    return s ? -v : v;
}

/* ---------------- typed element access (tensor_ops.c:488-588) ---------------- */
static inline int64_t read_int4(const void* p, size_t i) {
    int8_t v = ((const int8_t*)p)[i];
    return (v & 0x08) ? (int64_t)(int8_t)(v | 0xF0) : (int64_t)(v & 0x0F);
}

/* tensor_ops.c:488-514 */
static double read_f64(const Tensor* t, size_t i) {
    const void* p = t->data;
    switch ((int)t->dtype) {
    case DTYPE_FLOAT8_E4M3: return (double)dec_e4m3(((const uint8_t*)p)[i]);
    case DTYPE_FLOAT8_E5M2: return (double)dec_e5m2(((const uint8_t*)p)[i]);
    case DTYPE_FLOAT16: return (double)dec_f16(((const uint16_t*)p)[i]);
    case DTYPE_BFLOAT16: return (double)dec_bf16(((const uint16_t*)p)[i]);
    case DTYPE_FLOAT32: return (double)((const float*)p)[i];
    case DTYPE_FLOAT64: return ((const double*)p)[i];
    case DTYPE_INT4: return (double)read_int4(p, i);
    case DTYPE_INT8: return (double)((const int8_t*)p)[i];
    case DTYPE_UINT8: return (double)((const uint8_t*)p)[i];
    case DTYPE_INT16: return (double)((const int16_t*)p)[i];
    case DTYPE_INT32: return (double)((const int32_t*)p)[i];
    case DTYPE_INT64: return (double)((const int64_t*)p)[i];
    default: return 0.0;
    }
}

/* tensor_ops.c:520-546 — narrow floats go through rintf, f64 through rint. */
static int64_t read_i64(const Tensor* t, size_t i) {
    const void* p = t->data;
    switch ((int)t->dtype) {
    case DTYPE_FLOAT32: return trunc_i64_x86((double)rintf(((const float*)p)[i]));
    case DTYPE_FLOAT16: return trunc_i64_x86((double)rintf(dec_f16(((const uint16_t*)p)[i])));
    case DTYPE_BFLOAT16: return trunc_i64_x86((double)rintf(dec_bf16(((const uint16_t*)p)[i])));
    case DTYPE_FLOAT8_E4M3: return trunc_i64_x86((double)rintf(dec_e4m3(((const uint8_t*)p)[i])));
    case DTYPE_FLOAT8_E5M2: return trunc_i64_x86((double)rintf(dec_e5m2(((const uint8_t*)p)[i])));
    case DTYPE_FLOAT64: return trunc_i64_x86(rint(((const double*)p)[i]));
    case DTYPE_INT4: return read_int4(p, i);
    case DTYPE_INT8: return ((const int8_t*)p)[i];
    case DTYPE_UINT8: return ((const uint8_t*)p)[i];
    case DTYPE_INT16: return ((const int16_t*)p)[i];
    case DTYPE_INT32: return ((const int32_t*)p)[i];
    case DTYPE_INT64: return ((const int64_t*)p)[i];
    default: return 0;
    }
}

static void store_int(void* p, int dt, size_t i, int64_t v) {
    switch (dt) {
    case DTYPE_INT4: ((int8_t*)p)[i] = (int8_t)clamp_i64(v, -8, 7); break;
    case DTYPE_INT8: ((int8_t*)p)[i] = (int8_t)clamp_i64(v, -128, 127); break;
    case DTYPE_UINT8: ((uint8_t*)p)[i] = (uint8_t)clamp_i64(v, 0, 255); break;
    case DTYPE_INT16: ((int16_t*)p)[i] = (int16_t)clamp_i64(v, -32768, 32767); break;
    case DTYPE_INT32: ((int32_t*)p)[i] = (int32_t)clamp_i64(v, INT32_MIN, INT32_MAX); break;
    case DTYPE_INT64: ((int64_t*)p)[i] = v; break;
    default: break;
    }
}

/* tensor_ops.c:552-569 */
static void write_from_i64(Tensor* t, size_t i, int64_t v) {
    void* p = t->data;
    switch ((int)t->dtype) {
    case DTYPE_FLOAT8_E4M3: ((uint8_t*)p)[i] = enc_e4m3((float)v); break;
    case DTYPE_FLOAT8_E5M2: ((uint8_t*)p)[i] = enc_e5m2((float)v); break;
    case DTYPE_FLOAT16: ((uint16_t*)p)[i] = enc_f16((float)v); break;
    case DTYPE_BFLOAT16: ((uint16_t*)p)[i] = enc_bf16((float)v); break;
    case DTYPE_FLOAT32: ((float*)p)[i] = (float)v; break;
    case DTYPE_FLOAT64: ((double*)p)[i] = (double)v; break;
    default: store_int(p, (int)t->dtype, i, v); break;
    }
}

/* tensor_ops.c:571-588 — sub-f32 floats are written double -> float -> code. */
static void write_from_f64(Tensor* t, size_t i, double v) {
    void* p = t->data;
    switch ((int)t->dtype) {
    case DTYPE_FLOAT8_E4M3: ((uint8_t*)p)[i] = enc_e4m3((float)v); break;
    case DTYPE_FLOAT8_E5M2: ((uint8_t*)p)[i] = enc_e5m2((float)v); break;
    case DTYPE_FLOAT16: ((uint16_t*)p)[i] = enc_f16((float)v); break;
    case DTYPE_BFLOAT16: ((uint16_t*)p)[i] = enc_bf16((float)v); break;
    case DTYPE_FLOAT32: ((float*)p)[i] = (float)v; break;
    case DTYPE_FLOAT64: ((double*)p)[i] = v; break;
    default: store_int(p, (int)t->dtype, i, trunc_i64_x86(rint(v))); break;
    }
}

/* ---------------- lifecycle (tensor_ops.c:357-450) ---------------- */
Tensor* create_tensor(int* shape, int ndim, DataType dtype) {
    Tensor* t = (Tensor*)malloc(sizeof(Tensor));
    if (!t) return NULL;
    t->ndim = ndim;
    t->dtype = dtype;
    t->shape = (int*)malloc((size_t)(ndim > 0 ? ndim : 1) * sizeof(int));
    if (!t->shape) { free(t); return NULL; }
    size_t n = 1;
    for (int d = 0; d < ndim; d++) { t->shape[d] = shape[d]; n *= (size_t)shape[d]; }
    t->size = n;
    t->data = calloc(n ? n : 1, elem_bytes((int)dtype));
    if (!t->data) { free(t->shape); free(t); return NULL; }
    return t;
}

void free_tensor(Tensor* t) {
    if (!t) return;
    free(t->data);
    free(t->shape);
    free(t);
}

/* ---------------- Relu / Abs (tensor_ops.c:708-757) ---------------- */
static int unary_ok(const Tensor* in, const Tensor* out) {
    return in && out && in->data && out->data && in->size == out->size;
}

void relu_forward(const Tensor* in, Tensor* out) {
    if (!unary_ok(in, out)) return;
    int int_in = is_int_dtype((int)in->dtype);
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < in->size; i++) {
        if (int_in) {
            int64_t v = read_i64(in, i);
            write_from_i64(out, i, v > 0 ? v : 0);
        } else {
            double v = read_f64(in, i);
            write_from_f64(out, i, v > 0 ? v : 0.0);   /* NaN and -0 give +0 */
        }
    }
}

void abs_forward(const Tensor* in, Tensor* out) {
    if (!unary_ok(in, out)) return;
    int int_in = is_int_dtype((int)in->dtype);
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < in->size; i++) {
        if (int_in) {
            int64_t v = read_i64(in, i);
            write_from_i64(out, i, v == INT64_MIN ? INT64_MAX : (v < 0 ? -v : v));
        } else {
            write_from_f64(out, i, fabs(read_f64(in, i)));
        }
    }
}

/* ---------------- Cos (tensor_ops.c:763-854) ---------------- */
/* The reference evaluates cos by linear interpolation in a 4097-entry table
 * over [0, 2pi].  Entries come from truncated Taylor series (cos below pi/4,
 * sin(pi/2 - x) above) after folding into [0, pi/2].  The constants below are
 * the coefficients 1/2!, 1/4!, ... written as in the reference so the table
 * is bit-identical; this file is compiled with -ffp-contract=off. */
#define ORC_LUT_N 4096
static double orc_lut[ORC_LUT_N + 1];
static int orc_lut_ready = 0;
static pthread_mutex_t orc_lut_mu = PTHREAD_MUTEX_INITIALIZER;
static const double ORC_PI = 3.141592653589793238462643383279502884197;

void init_cos_lut(void) {
    pthread_mutex_lock(&orc_lut_mu);
    if (!orc_lut_ready) {
        const double two_pi = 2.0 * ORC_PI, half_pi = ORC_PI / 2.0;
        for (int i = 0; i <= ORC_LUT_N; i++) {
            double x = (double)i * two_pi / ORC_LUT_N;
            double sgn = 1.0;
            if (x > ORC_PI) x = two_pi - x;
            if (x > half_pi) { x = ORC_PI - x; sgn = -1.0; }
            double x2 = x * x, r;
            if (x < 0.785398163397448) {
                r = 1.0 + x2 * (-0.5 + x2 * (0.04166666666666666 +
                    x2 * (-0.001388888888888889 + x2 * 0.000024801587301587302)));
            } else {
                double t = half_pi - x, t2 = t * t;
                r = t * (1.0 + t2 * (-0.16666666666666666 + t2 * (0.008333333333333333 +
                    t2 * (-0.0001984126984126984 + t2 * 0.0000027557319223985893))));
            }
            orc_lut[i] = sgn * r;
        }
        __sync_synchronize();
        orc_lut_ready = 1;
    }
    pthread_mutex_unlock(&orc_lut_mu);
}

/* tensor_ops.c:815-833.  NaN / inf inputs: the reference indexes the table
 * with (int)NaN (out of bounds); here they return NaN. */
static double lut_cos(double x) {
    const double two_pi = 2.0 * ORC_PI;
    double r = fmod(fabs(x), two_pi);
    if (!(r == r)) return r;
    double pos = r * ORC_LUT_N / two_pi;
    int k = (int)pos;
    double w = pos - k;
    if (k >= ORC_LUT_N) { k = ORC_LUT_N - 1; w = 0.0; }
    return orc_lut[k] * (1.0 - w) + orc_lut[k + 1] * w;
}

void cos_forward(const Tensor* in, Tensor* out) {
    if (!unary_ok(in, out)) return;
    if (!orc_lut_ready) init_cos_lut();
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < in->size; i++) write_from_f64(out, i, lut_cos(read_f64(in, i)));
}

/* ---------------- Add / Sub / Mul / Div (tensor_ops.c:610-684, 864-997) ---------------- */
enum { OP_ADD, OP_SUB, OP_MUL, OP_DIV };

static inline int64_t int_op(int op, int64_t a, int64_t b) {
    uint64_t ua = (uint64_t)a, ub = (uint64_t)b;      /* wrap like the x86 build */
    switch (op) {
    case OP_ADD: return (int64_t)(ua + ub);
    case OP_SUB: return (int64_t)(ua - ub);
    case OP_MUL: return (int64_t)(ua * ub);
    default:
        if (b == 0) return a >= 0 ? INT64_MAX : INT64_MIN;
        if (a == INT64_MIN && b == -1) return INT64_MIN;  /* reference traps (idiv) here */
        return a / b;
    }
}

static inline double flt_op(int op, double a, double b) {
    switch (op) {
    case OP_ADD: return a + b;
    case OP_SUB: return a - b;
    case OP_MUL: return a * b;
    default: return a / b;
    }
}

static void binary(int op, const Tensor* A, const Tensor* B, Tensor* O) {
    if (!A || !B || !O || !A->data || !B->data || !O->data) return;
    if (A->size != B->size || A->size != O->size) return;
    size_t n = O->size;
    if (is_int_dtype((int)O->dtype)) {
        #pragma omp parallel for schedule(static)
        for (size_t i = 0; i < n; i++)
            store_int(O->data, (int)O->dtype, i, int_op(op, read_i64(A, i), read_i64(B, i)));
    } else {
        #pragma omp parallel for schedule(static)
        for (size_t i = 0; i < n; i++)
            write_from_f64(O, i, flt_op(op, read_f64(A, i), read_f64(B, i)));
    }
}

void add_forward(const Tensor* A, const Tensor* B, Tensor* O) { binary(OP_ADD, A, B, O); }
void sub_forward(const Tensor* A, const Tensor* B, Tensor* O) { binary(OP_SUB, A, B, O); }
void mul_forward(const Tensor* A, const Tensor* B, Tensor* O) { binary(OP_MUL, A, B, O); }
void div_forward(const Tensor* A, const Tensor* B, Tensor* O) { binary(OP_DIV, A, B, O); }

/* ---------------- QuantizeLinear / DequantizeLinear (tensor_ops.c:999-1034) ---------------- */
/* Operands are indexed flat over Y->size (the reference's Python caller
 * broadcasts Scale / ZeroPoint to full size first). */
void quantize_linear_forward(const Tensor* X, const Tensor* S, const Tensor* Z, Tensor* Y) {
    if (!X || !S || !Z || !Y) return;
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < Y->size; i++) {
        double x = read_f64(X, i), s = read_f64(S, i), z = read_f64(Z, i);
        write_from_f64(Y, i, s != 0.0 ? rint(x / s) + z : z);
    }
}

void dequantize_linear_forward(const Tensor* X, const Tensor* S, const Tensor* Z, Tensor* Y) {
    if (!X || !S || !Z || !Y) return;
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < Y->size; i++) {
        double x = read_f64(X, i), s = read_f64(S, i), z = read_f64(Z, i);
        write_from_f64(Y, i, (x - z) * s);
    }
}

/* ---------------- Conv2d (tensor_ops.c:687-700, 1036-1114) ---------------- */
/* Direct NCHW convolution; the double sum runs over (ic, kh, kw) in that
 * order, padded taps contribute 0.0 * w, and the bias is added last. */
void conv2d_forward(const Tensor* X, const Tensor* W, const Tensor* B, Tensor* Y, ConvParams* p) {
    const int N = X->shape[0], C = X->shape[1], H = X->shape[2], Wd = X->shape[3];
    const int M = W->shape[0], KH = W->shape[2], KW = W->shape[3];
    const int OH = Y->shape[2], OW = Y->shape[3];
    const int pt = p->pads[0], pl = p->pads[1], sh = p->strides[0], sw = p->strides[1];
    const int dh = p->dilations[0], dw = p->dilations[1], g = p->group;
    const int cg = C / g, mg = M / g;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; n++) {
        for (int m = 0; m < M; m++) {
            const int grp = m / mg;
            const double bias = (B && B->data) ? read_f64(B, (size_t)m) : 0.0;
            for (int oh = 0; oh < OH; oh++) {
                for (int ow = 0; ow < OW; ow++) {
                    double acc = 0.0;
                    for (int c = 0; c < cg; c++) {
                        const int ic = grp * cg + c;
                        for (int kh = 0; kh < KH; kh++) {
                            const int ih = oh * sh + kh * dh - pt;
                            for (int kw = 0; kw < KW; kw++) {
                                const int iw = ow * sw + kw * dw - pl;
                                double xv = 0.0;
                                if (ih >= 0 && ih < H && iw >= 0 && iw < Wd)
                                    xv = read_f64(X, (((size_t)n * C + ic) * H + ih) * Wd + iw);
                                double wv = read_f64(W, (((size_t)m * cg + c) * KH + kh) * KW + kw);
                                acc += xv * wv;
                            }
                        }
                    }
                    write_from_f64(Y, (((size_t)n * M + m) * OH + oh) * OW + ow, acc + bias);
                }
            }
        }
    }
}

/* ---------------- MaxPool (tensor_ops.c:1116-1165) ---------------- */
/* Starts from -inf, visits in-bounds taps only and keeps the first strict
 * maximum, so NaN is never selected and an all-padding window gives -inf. */
void max_pool_forward(const Tensor* X, Tensor* Y, PoolParams* p) {
    const int N = X->shape[0], C = X->shape[1], H = X->shape[2], Wd = X->shape[3];
    const int OH = Y->shape[2], OW = Y->shape[3];
    const int KH = p->kernel_shape[0], KW = p->kernel_shape[1];
    const int pt = p->pads[0], pl = p->pads[1], sh = p->strides[0], sw = p->strides[1];
    const int dh = p->dilations[0], dw = p->dilations[1];
    #pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; n++) {
        for (int c = 0; c < C; c++) {
            const size_t plane = ((size_t)n * C + c) * H * Wd;
            for (int oh = 0; oh < OH; oh++) {
                for (int ow = 0; ow < OW; ow++) {
                    double best = -INFINITY;
                    for (int kh = 0; kh < KH; kh++) {
                        const int ih = oh * sh + kh * dh - pt;
                        if (ih < 0 || ih >= H) continue;
                        for (int kw = 0; kw < KW; kw++) {
                            const int iw = ow * sw + kw * dw - pl;
                            if (iw < 0 || iw >= Wd) continue;
                            double v = read_f64(X, plane + (size_t)ih * Wd + iw);
                            if (v > best) best = v;
                        }
                    }
                    write_from_f64(Y, (((size_t)n * C + c) * OH + oh) * OW + ow, best);
                }
            }
        }
    }
}

/* ---------------- Gemm (tensor_ops.c:1167-1228) ---------------- */
/* Bias C: one element broadcasts everywhere; 1-D matches N (columns) first,
 * then M (rows); >= 2-D uses its last two dims with size-1 broadcast. */
static double gemm_bias(const Tensor* C, int m, int n, int M, int N) {
    if (C->size == 1) return read_f64(C, 0);
    if (C->ndim == 1) {
        if (C->shape[0] == N) return read_f64(C, (size_t)n);
        if (C->shape[0] == M) return read_f64(C, (size_t)m);
        return 0.0;
    }
    if (C->ndim >= 2) {
        const int H = C->shape[C->ndim - 2], Wc = C->shape[C->ndim - 1];
        const int r = (H == 1) ? 0 : m, q = (Wc == 1) ? 0 : n;
        if (r < H && q < Wc) return read_f64(C, (size_t)r * Wc + q);
    }
    return 0.0;
}

void gemm_forward(const Tensor* A, const Tensor* B, const Tensor* C, Tensor* Y,
                  float alpha, float beta, int transA, int transB) {
    const int M = transA ? A->shape[1] : A->shape[0];
    const int K = transA ? A->shape[0] : A->shape[1];
    const int N = transB ? B->shape[0] : B->shape[1];
    const size_t lda = (size_t)A->shape[1], ldb = (size_t)B->shape[1];
    const int has_c = C && C->data;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) {
            double acc = 0.0;
            for (int k = 0; k < K; k++) {
                size_t ia = transA ? (size_t)k * lda + m : (size_t)m * lda + k;
                size_t ib = transB ? (size_t)n * ldb + k : (size_t)k * ldb + n;
                acc += read_f64(A, ia) * read_f64(B, ib);
            }
            double r = (double)alpha * acc;
            if (has_c) r += (double)beta * gemm_bias(C, m, n, M, N);
            write_from_f64(Y, (size_t)m * N + n, r);
        }
    }
}

/* ---------------- Softmax (tensor_ops.c:1231-1270) ---------------- */
void softmax_forward(const Tensor* in, Tensor* out, int axis) {
    if (axis < 0) axis += in->ndim;
    const int L = in->shape[axis];
    int outer = 1, inner = 1;
    for (int d = 0; d < axis; d++) outer *= in->shape[d];
    for (int d = axis + 1; d < in->ndim; d++) inner *= in->shape[d];
    #pragma omp parallel for collapse(2) schedule(static)
    for (int o = 0; o < outer; o++) {
        for (int r = 0; r < inner; r++) {
            const size_t base = (size_t)o * L * inner + r;
            double mx = -DBL_MAX;
            for (int j = 0; j < L; j++) {
                double v = read_f64(in, base + (size_t)j * inner);
                if (v > mx) mx = v;
            }
            double sum = 0.0;
            for (int j = 0; j < L; j++) sum += exp(read_f64(in, base + (size_t)j * inner) - mx);
            for (int j = 0; j < L; j++) {
                size_t i = base + (size_t)j * inner;
                write_from_f64(out, i, exp(read_f64(in, i) - mx) / sum);
            }
        }
    }
}

/* ---------------- Flatten / Reshape (tensor_ops.c:1289-1299) ---------------- */
/* A byte copy of input->size elements of the input's width; sizes must match. */
void flatten_forward(const Tensor* in, Tensor* out) {
    if (!in || !out || in->size != out->size) return;
    memcpy(out->data, in->data, in->size * elem_bytes(in->dtype));
}
void reshape_forward(const Tensor* in, Tensor* out) { flatten_forward(in, out); }

/* ---------------- GlobalAveragePool (tensor_ops.c:2844-2868) ---------------- */
/* 4-D input only (anything else leaves the output untouched); each of the
 * N*C planes is summed in double in index order, then divided by H*W. */
void global_average_pool_forward(const Tensor* in, Tensor* out) {
    if (!in || !out || in->ndim != 4) return;
    const int planes = in->shape[0] * in->shape[1];
    const int hw = in->shape[2] * in->shape[3];
    #pragma omp parallel for schedule(static)
    for (int n = 0; n < planes; n++) {
        double sum = 0.0;
        for (int i = 0; i < hw; i++) sum += read_f64(in, (size_t)n * hw + i);
        write_from_f64(out, (size_t)n, sum / hw);
    }
}

/* ---------------- DynamicQuantizeLinear (tensor_ops.c:3760-3809) ---------------- */
/* min / max over x (NaN never compares), widened to include 0; scale =
 * (max - min) / 255 in double (1 when 0); zero point = round(-min / scale)
 * (half away from zero) clamped to [0, 255]; y = clamp(rint(x / scale) + zp,
 * 0, 255) with the double scale, written through the output encoder. */
void dynamic_quantize_linear_forward(const Tensor* x, Tensor* y, Tensor* y_scale, Tensor* y_zp) {
    if (!x || !y || !y_scale || !y_zp) return;
    double lo = DBL_MAX, hi = -DBL_MAX;
    for (size_t i = 0; i < x->size; i++) {
        const double v = read_f64(x, i);
        if (v < lo) lo = v;
        if (v > hi) hi = v;
    }
    lo = fmin(lo, 0.0);
    hi = fmax(hi, 0.0);
    double scale = (hi - lo) / 255.0;
    if (scale == 0.0) scale = 1.0;
    double zpd = round(0.0 - lo / scale);
    if (zpd < 0.0) zpd = 0.0;
    if (zpd > 255.0) zpd = 255.0;
    const uint8_t zp = (uint8_t)zpd;
    write_from_f64(y_scale, 0, scale);
    if (y_zp->dtype == DTYPE_UINT8) ((uint8_t*)y_zp->data)[0] = zp;
    else write_from_f64(y_zp, 0, (double)zp);
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < x->size; i++) {
        double q = rint(read_f64(x, i) / scale) + (double)zp;
        if (q < 0.0) q = 0.0;
        if (q > 255.0) q = 255.0;
        write_from_f64(y, i, q);
    }
}

/* ---------------- codec probes for exhaustive sweeps (oracle-only symbols) ---------------- */
void oracle_encode_f32(const float* x, void* out, size_t n, int dtype) {
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) {
        switch (dtype) {
        case DTYPE_FLOAT16: ((uint16_t*)out)[i] = enc_f16(x[i]); break;
        case DTYPE_BFLOAT16: ((uint16_t*)out)[i] = enc_bf16(x[i]); break;
        case DTYPE_FLOAT8_E4M3: ((uint8_t*)out)[i] = enc_e4m3(x[i]); break;
        case DTYPE_FLOAT8_E5M2: ((uint8_t*)out)[i] = enc_e5m2(x[i]); break;
        default: break;
        }
    }
}

/* Position-weighted checksum of a code stream: sum over i of (code_i + 1) * (base + i + 1)
 * modulo 2^64, with code_i read as an unsigned integer of elem bytes. */
uint64_t oracle_checksum(const void* codes, size_t n, int elem, uint64_t base) {
    uint64_t acc = 0;
    #pragma omp parallel for reduction(+:acc) schedule(static)
    for (size_t i = 0; i < n; i++) {
        uint64_t c = 0;
        if (elem == 1) c = ((const uint8_t*)codes)[i];
        else if (elem == 2) c = ((const uint16_t*)codes)[i];
        else if (elem == 4) c = ((const uint32_t*)codes)[i];
        else c = ((const uint64_t*)codes)[i];
        acc += (c + 1u) * (base + (uint64_t)i + 1u);
    }
    return acc;
}
