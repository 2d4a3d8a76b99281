/*
 * tensor_ops.h — C ABI of libtensor_ops_hip.so (MI355X / gfx950).
 *
 * The first block restates the reference operator library's interface for the
 * 13 hot-path operators, with identical type layouts (LP64) and identical
 * symbol names and signatures, so a caller that binds the reference library
 * through ctypes binds this one unchanged.  Every declaration cites the
 * reference declaration it replaces (paths relative to the reference tree).
 *
 * The second block lists additive extensions: new symbols only, the structs
 * are unchanged.  They add device-resident tensors (data pointer in HBM),
 * explicit streams, error reporting and per-axis quantization.
 *
 * Semantics common to all operators (tensor_ops/tensor_ops.c:488-588):
 *   every input element is decoded to double, the operator computes in double
 *   (or in a narrower type only where that is provably bit-identical), and the
 *   result is written through the output dtype's encoder.  Outputs are
 *   pre-created by the caller with their final shape and dtype.
 *
 * Residency: a Tensor made by create_tensor() holds host memory (pinned when a
 * GPU is present); operators on such tensors are synchronous and stage the
 * data through device memory.  A Tensor made by create_tensor_device() or
 * tensor_wrap_device() holds device memory; operators whose operands are all
 * device-resident are enqueued on the library stream and return immediately.
 *
 * Graph capture: operators on device tensors may be captured into a HIP graph
 * on the library stream.  Captured calls allocate nothing (no split-k slices;
 * Softmax over few long rows and DynamicQuantizeLinear keep their partials in
 * fixed per-GPU device arrays, so replays of such graphs that overlap on one
 * GPU race).  Anything that would allocate or synchronise under capture (host
 * tensors, create_tensor_device*, tensor_to_host / tensor_from_host, internal
 * temporaries of the fallback paths) is refused with an error instead.
 */
#ifndef TENSOR_OPS_HIP_H
#define TENSOR_OPS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types; values match tensor_ops/tensor_ops.h:10-23 and the Python
 * DTYPE_MAP of nn/__init__.py:20-34 (int4 is stored one value per byte). */
typedef enum {
    DTYPE_FLOAT8_E4M3 = 0,
    DTYPE_FLOAT8_E5M2 = 1,
    DTYPE_FLOAT16 = 2,
    DTYPE_BFLOAT16 = 3,
    DTYPE_FLOAT32 = 4,
    DTYPE_FLOAT64 = 5,
    DTYPE_INT4 = 6,
    DTYPE_INT8 = 7,
    DTYPE_UINT8 = 8,
    DTYPE_INT16 = 9,
    DTYPE_INT32 = 10,
    DTYPE_INT64 = 11
} DataType;

/* tensor_ops/tensor_ops.h:28-34 — sizeof 40: data@0 shape@8 ndim@16 size@24 dtype@32. */
typedef struct {
    void* data;
    int* shape;
    int ndim;
    size_t size;
    DataType dtype;
} Tensor;

/* tensor_ops/tensor_ops.h:39-44 — pads are [top, left, bottom, right]. */
typedef struct {
    int* pads;
    int* strides;
    int* dilations;
    int group;
} ConvParams;

/* tensor_ops/tensor_ops.h:49-54 */
typedef struct {
    int* pads;
    int* strides;
    int* dilations;
    int* kernel_shape;
} PoolParams;

/* ---------------------------------------------------------------------------
 * Reference ABI (hot path)
 * ------------------------------------------------------------------------- */

/* tensor_ops/tensor_ops.h:70 (tensor_ops.c:357-433): zero-filled host tensor,
 * NULL on allocation failure. */
Tensor* create_tensor(int* shape, int ndim, DataType dtype);
/* tensor_ops/tensor_ops.h:77 (tensor_ops.c:440-450): frees any tensor this
 * library made (host or device); NULL is ignored. */
void free_tensor(Tensor* tensor);
/* tensor_ops/tensor_ops.h:85 (tensor_ops.c:708-728) */
void relu_forward(const Tensor* input, Tensor* output);
/* tensor_ops/tensor_ops.h:91 (tensor_ops.c:763-807): builds the 4097-entry
 * cosine table once (thread-safe) and uploads it to the device. */
void init_cos_lut(void);
/* tensor_ops/tensor_ops.h:99 (tensor_ops.c:815-854) */
void cos_forward(const Tensor* input, Tensor* output);
/* tensor_ops/tensor_ops.h:107 (tensor_ops.c:736-757) */
void abs_forward(const Tensor* input, Tensor* output);
/* tensor_ops/tensor_ops.h:116,125,134,143 (tensor_ops.c:864-997).
 * Equal sizes: flat elementwise, as the reference.  Sizes that differ but
 * broadcast (numpy rules) to O's shape: broadcast in-kernel (the reference
 * returns without writing there; its Python caller broadcasts first). */
void add_forward(const Tensor* A, const Tensor* B, Tensor* O);
void sub_forward(const Tensor* A, const Tensor* B, Tensor* O);
void mul_forward(const Tensor* A, const Tensor* B, Tensor* O);
void div_forward(const Tensor* A, const Tensor* B, Tensor* O);
/* tensor_ops/tensor_ops.h:149 (tensor_ops.c:999-1016):
 * y = s != 0 ? rint(x / s) + zp : zp in double, then the output encoder.
 * Scale / ZeroPoint may be full-size (reference) or broadcastable to Y. */
void quantize_linear_forward(const Tensor* X, const Tensor* Scale, const Tensor* ZeroPoint, Tensor* Y);
/* tensor_ops/tensor_ops.h:155 (tensor_ops.c:1018-1034): y = (x - zp) * s in double. */
void dequantize_linear_forward(const Tensor* X, const Tensor* Scale, const Tensor* ZeroPoint, Tensor* Y);
/* tensor_ops/tensor_ops.h:161 (tensor_ops.c:1036-1114): NCHW, W [M, C/group, KH, KW],
 * B nullable [M]; output size is taken from Y's shape. */
void conv2d_forward(const Tensor* X, const Tensor* W, const Tensor* B, Tensor* Y, ConvParams* params);
/* tensor_ops/tensor_ops.h:166 (tensor_ops.c:1116-1165) */
void max_pool_forward(const Tensor* X, Tensor* Y, PoolParams* params);
/* tensor_ops/tensor_ops.h:173-174 (tensor_ops.c:1167-1228): Y = alpha * A' B' + beta * C. */
void gemm_forward(const Tensor* A, const Tensor* B, const Tensor* C, Tensor* Y,
                  float alpha, float beta, int transA, int transB);
/* tensor_ops/tensor_ops.h:179 (tensor_ops.c:1231-1270); negative axis counts from the end. */
void softmax_forward(const Tensor* input, Tensor* output, int axis);

/* ---------------------------------------------------------------------------
 * Reference ABI (operators next to the hot path: the ops a ResNet-style graph
 * needs between the conv blocks and the classifier, and dynamic quantization)
 * ------------------------------------------------------------------------- */

/* tensor_ops/tensor_ops.h:210 (tensor_ops.c:1289-1294): copies input->size
 * elements of the input's width when the sizes match, else does nothing. */
void flatten_forward(const Tensor* input, Tensor* output);
/* tensor_ops/tensor_ops.h:216 (tensor_ops.c:1297-1299): same as flatten_forward. */
void reshape_forward(const Tensor* input, Tensor* output);
/* tensor_ops/tensor_ops.h:466 (tensor_ops.c:2844-2868): 4-D input only; each
 * plane summed in double in index order, divided by H * W. */
void global_average_pool_forward(const Tensor* input, Tensor* output);
/* tensor_ops/tensor_ops.h:547 (tensor_ops.c:3760-3809): uint8 quantization
 * with scale / zero point from the tensor's min and max (widened to 0). */
void dynamic_quantize_linear_forward(const Tensor* x, Tensor* y, Tensor* y_scale, Tensor* y_zp);

/* ---------------------------------------------------------------------------
 * Extensions (no counterpart in the reference)
 * ------------------------------------------------------------------------- */

/* Zero-filled tensor in device memory (HBM).  NULL on failure, and while the library
 * stream is being captured into a graph (create device tensors before the capture). */
Tensor* create_tensor_device(int* shape, int ndim, DataType dtype);
/* Device tensor with undefined contents, for an operator output that the next
 * call writes in full (saves the fill of create_tensor_device).  NULL on failure and
 * under capture, as create_tensor_device. */
Tensor* create_tensor_device_empty(int* shape, int ndim, DataType dtype);
/* Tensor header over caller-owned device memory; free_tensor frees only the header. */
Tensor* tensor_wrap_device(void* device_ptr, int* shape, int ndim, DataType dtype);
/* 1 if t's data lives in device memory, else 0. */
int tensor_is_device(const Tensor* t);
/* Copy between a tensor (host or device) and plain host memory of t->size elements.
 * Both synchronise the library stream.  Return 0 on success, -1 on error. */
int tensor_to_host(const Tensor* t, void* host_dst);
int tensor_from_host(Tensor* t, const void* host_src);
/* Wait for all work enqueued by this library.  0 on success. */
int tensor_ops_hip_sync(void);
/* Use a caller-provided hipStream_t (NULL restores the library's own stream). */
void tensor_ops_hip_set_stream(void* stream);
/* Stream for the calling thread's subsequent calls only, overriding the one above (NULL
 * clears the override).  Nothing is drained: the caller orders work across its streams.
 * Library workspace buffers are reused only on the stream they were released on, and
 * those cached under the stream a thread leaves go to other streams only once the work
 * enqueued on it before the switch has completed (an event recorded at the switch); a
 * tensor used on several streams must be freed once the caller has ordered them. */
void tensor_ops_hip_set_thread_stream(void* stream);
void* tensor_ops_hip_get_stream(void);
/* Number of usable GPUs (0 on a machine without one). */
int tensor_ops_hip_device_count(void);
/* Last error of the calling thread ("" if none); cleared by tensor_ops_hip_clear_error. */
const char* tensor_ops_hip_last_error(void);
void tensor_ops_hip_clear_error(void);
/* Library version string. */
const char* tensor_ops_hip_version(void);
/* Gemm/Conv precision mode of the calling thread: 0 = MFMA fp32/fp16 accumulate
 * (default, tolerance class); 1 = exact replica of the reference (double accumulate,
 * sequential k, bit-identical).  Each thread starts from TENSOR_OPS_HIP_EXACT
 * (unset: 0); setting it affects only calls made by the same thread. */
void tensor_ops_hip_set_exact(int exact);
int tensor_ops_hip_get_exact(void);
/* Softmax over few long rows and f32 -> uint8 DynamicQuantizeLinear run one launch in
 * which blocks exchange partial results (a row's (max, sum) pairs; every block's
 * (min, max)) and wait for each other's with a bounded poll; a block whose wait runs out
 * recomputes the missing partials from X (same bits).  Sets that bound for both (polls
 * of ~64 cycles; 0 makes every block recompute, < 0 restores the default) and returns
 * the previous value.  For tests of the recompute path; process-wide. */
int tensor_ops_hip_set_softmax_spin(int polls);
/* Those exchanges tag their words with the low 32 bits of a per-process call count
 * (the high bits are an epoch: buffers are zero-filled again when it changes).  Moves
 * the count forward to at least `count` (never back, so tags stay unique within an
 * epoch) and returns the count now in effect; 0 only reads it.  For tests of the tag
 * wrap-around. */
unsigned long long tensor_ops_hip_advance_exchange_count(unsigned long long count);
/* Fills every device buffer that the library hands out with undefined contents
 * (create_tensor_device_empty, the staging copy of a host output) with `byte` (e.g.
 * 0xFF: NaN in every float format) before the operator writes it, so a test sees any
 * element an operator failed to write; < 0 turns it off (the default).  Returns the
 * previous setting.  Process-wide; for tests. */
int tensor_ops_hip_set_poison(int byte);
/* Fused elementwise chain: one pass over X that applies the steps in order to the
 * running value v; binary steps take operands[operand] broadcast to X's shape and
 * compute v op b (b op v when reversed).  Every step rounds to float32 as the
 * standalone operator (add_forward, ..., cos_forward) writes its output, so Y equals
 * the op-by-op chain bit for bit.  float32 only; at most 3 operands and 16 steps.
 * Replaces a sequence of the reference's unary / binary calls on one tensor
 * (tensor_ops/tensor_ops.h:85-143). */
enum {
    TENSOR_OPS_CHAIN_ADD = 0, TENSOR_OPS_CHAIN_SUB = 1, TENSOR_OPS_CHAIN_MUL = 2, TENSOR_OPS_CHAIN_DIV = 3,
    TENSOR_OPS_CHAIN_RELU = 4, TENSOR_OPS_CHAIN_ABS = 5, TENSOR_OPS_CHAIN_COS = 6
};
typedef struct {
    int op;         /* TENSOR_OPS_CHAIN_* */
    int operand;    /* index into operands (binary steps) */
    int reversed;   /* binary steps: 1 computes operand op v */
} TensorOpsChainStep;
void elementwise_chain_forward(const Tensor* X, const Tensor* const* operands, int noperands,
                               const TensorOpsChainStep* steps, int nsteps, Tensor* Y);
/* Per-axis quantize / dequantize with 1-D Scale / ZeroPoint of length X->shape[axis]. */
void quantize_linear_axis_forward(const Tensor* X, const Tensor* Scale, const Tensor* ZeroPoint,
                                  Tensor* Y, int axis);
void dequantize_linear_axis_forward(const Tensor* X, const Tensor* Scale, const Tensor* ZeroPoint,
                                    Tensor* Y, int axis);
/* Fake quantization: Y = DequantizeLinear(QuantizeLinear(X, QScale, QZeroPoint), DScale,
 * DZeroPoint), the quantize_linear_forward -> dequantize_linear_forward pair
 * (tensor_ops/tensor_ops.h:149, 155) with the codes of dtype code_dtype kept in registers
 * (never written), for the QuantizeLinear -> DequantizeLinear pairs of QDQ graphs whose codes
 * feed nothing else.  Y (float32, X's shape) equals the pair bit for bit.  The one-pass
 * kernel takes f32 X, one-element f32 scales and one-element zero points of code_dtype
 * (uint8 / int8 / e4m3 / e5m2); other operands run the pair through a temporary. */
void quantize_dequantize_linear_forward(const Tensor* X, const Tensor* QScale, const Tensor* QZeroPoint,
                                        const Tensor* DScale, const Tensor* DZeroPoint, Tensor* Y,
                                        int code_dtype);
/* Weight-only-quantized Gemm: Y = alpha * A' * DQ(Bq)' + beta * C with DQ(Bq) =
 * dequantize_linear_axis_forward(Bq, Scale, ZeroPoint, ., axis), in one pass that reads
 * Bq as int8 / uint8 codes (the f32 weight is never written).  Same arguments and output
 * as dequantize_linear_axis_forward followed by gemm_forward (tensor_ops/tensor_ops.h:155,
 * 173-174), and the same bits.  ZeroPoint may be NULL (zero). */
void dequantize_gemm_forward(const Tensor* A, const Tensor* Bq, const Tensor* Scale, const Tensor* ZeroPoint,
                             int axis, const Tensor* C, Tensor* Y, float alpha, float beta, int transA,
                             int transB);
/* Gemm followed by Softmax over the last axis: Y = gemm_forward(A, B, C, alpha, beta, transA,
 * transB) and P = softmax_forward(Y, axis = last) (tensor_ops/tensor_ops.h:173-174, 179), bit
 * for bit.  With f32 device Y and P and a Gemm that runs as a k-split product, the split
 * reduction also takes the softmax (one launch fewer); otherwise the two calls run. */
void gemm_softmax_forward(const Tensor* A, const Tensor* B, const Tensor* C, Tensor* Y, Tensor* P, float alpha,
                          float beta, int transA, int transB);
/* Convolution with the residual block's epilogue: Y = [Skip +] [Relu](Conv(X, W, B)), the
 * conv2d_forward -> relu_forward -> add_forward(., Skip) sequence (tensor_ops/tensor_ops.h:161,
 * 85, 116) in one pass over Y.  Each step rounds to the output dtype as the standalone
 * operator does, so Y equals the sequence bit for bit.  relu != 0 applies Relu; Skip may be
 * NULL (no Add) and broadcasts to Y as add_forward's B does. */
void conv2d_fused_forward(const Tensor* X, const Tensor* W, const Tensor* B, const Tensor* Skip, int relu,
                          Tensor* Y, ConvParams* params);
/* MaxPool with a second output: Y = max_pool_forward(X) and Yq = DequantizeLinear(
 * QuantizeLinear(Y, QScale, QZeroPoint), DScale, DZeroPoint), the max_pool_forward ->
 * quantize_linear_forward -> dequantize_linear_forward sequence (tensor_ops/tensor_ops.h:166,
 * 149, 155) with Y read once; Yq has the bits of quantize_dequantize_linear_forward(Y).  The
 * one-pass kernel covers f32 3x3 / stride-2 pooling (top / left pad 1) with uint8 / int8 codes
 * and one-element f32 scales and zero points of the code dtype; other arguments run the
 * sequence. */
void max_pool_qdq_forward(const Tensor* X, Tensor* Y, PoolParams* params, const Tensor* QScale,
                          const Tensor* QZeroPoint, const Tensor* DScale, const Tensor* DZeroPoint,
                          int code_dtype, Tensor* Yq);
/* Convolution with the residual block's epilogue and the next block's activation fake
 * quantization: Y = DequantizeLinear(QuantizeLinear(conv2d_fused_forward's Y, QScale,
 * QZeroPoint), DScale, DZeroPoint), the conv2d_fused_forward -> quantize_linear_forward ->
 * dequantize_linear_forward sequence (tensor_ops/tensor_ops.h:161, 85, 116, 149, 155) in one
 * pass over Y (the pre-quantization activation is never written), with the same bits as
 * conv2d_fused_forward followed by quantize_dequantize_linear_forward.  code_dtype names the
 * intermediate codes' dtype as there; the one-pass epilogue covers uint8 / int8 codes with
 * one-element f32 scales and zero points of the code dtype, other arguments run the
 * sequence. */
void conv2d_fused_qdq_forward(const Tensor* X, const Tensor* W, const Tensor* B, const Tensor* Skip, int relu,
                              const Tensor* QScale, const Tensor* QZeroPoint, const Tensor* DScale,
                              const Tensor* DZeroPoint, int code_dtype, Tensor* Y, ConvParams* params);
/* The QDQ convolution: Y = [Skip +] [Relu](Conv(DequantizeLinear(Xq, XScale, XZero), W, B)), the
 * dequantize_linear_forward -> conv2d_fused_forward sequence (tensor_ops/tensor_ops.h:155, 161)
 * in one pass that reads the uint8 / int8 activation codes directly; the same bits as the
 * sequence.  XScale / XZero hold one element (per-tensor); XZero may be NULL (zero). */
void dequantize_conv2d_fused_forward(const Tensor* Xq, const Tensor* XScale, const Tensor* XZero,
                                     const Tensor* W, const Tensor* B, const Tensor* Skip, int relu,
                                     Tensor* Y, ConvParams* params);
/* DynamicQuantizeLinear that allocates nothing.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments and the same bits as
 * dynamic_quantize_linear_forward; every tensor must be device-resident (an error
 * otherwise: host tensors would need staging buffers).  Its min / max partials live in a
 * fixed 32,784-byte device array per GPU (at most 2048 partials, whatever the input size),
 * held until the process ends and shared by every call on that GPU (and by captured calls
 * of dynamic_quantize_linear_forward): calls that overlap on one GPU race. */
void dynamic_quantize_linear_forward_noalloc(const Tensor* x, Tensor* y, Tensor* y_scale, Tensor* y_zp);

/* ---------------------------------------------------------------------------
 * QDQ convolution blocks on int8 MFMA.  They replace, for a QDQ residual block,
 * the sequence quantize_linear_forward -> dequantize_linear_forward (activation,
 * tensor_ops/tensor_ops.h:149, 155) -> dequantize_linear_axis_forward (int8
 * weights, per output channel, zero point 0) -> conv2d_forward (:161) ->
 * relu_forward (:85) -> add_forward (:116) with the skip or a 1x1 projection
 * conv2d_forward of the same activation, and the next block's
 * quantize_linear_forward.  The convolution sums sum_k w (x - zx) exactly in
 * int32 and scales it once (sx * sw[m], in double, rounded to float32): the
 * tolerance class of the MFMA convolution, not the reference's bits, and no
 * exact mode (qconv_block_forward fails while tensor_ops_hip_set_exact(1) is in
 * effect).  Activations between blocks are channels-last int8 [N, H, W, C]
 * holding code - 128 for uint8 codes (the code for int8): an internal layout
 * that only these calls read.  Device tensors only; C a multiple of 32.
 * ------------------------------------------------------------------------- */
/* Y (int8 [N, H, W, C]) = QuantizeLinear(X, Scale, ZeroPoint) in that layout; X float32
 * [N, C, H, W], Scale one float32, ZeroPoint one element of code_dtype (uint8 / int8)
 * or NULL (0).  The codes are quantize_linear_forward's, bit for bit. */
void quantize_linear_nhwc_forward(const Tensor* X, const Tensor* Scale, const Tensor* ZeroPoint,
                                  int code_dtype, Tensor* Y);
/* Y = max_pool_forward(X, params) (tensor_ops/tensor_ops.h:166) and Yc (int8 [N, OH, OW, C]
 * in the layout above) = quantize_linear_nhwc_forward(Y, Scale, ZeroPoint, code_dtype), bit
 * for bit, in one pass that reads X once (f32, 3x3 window, stride 2, top / left padding 1,
 * W == 2 * OW <= 128, C a multiple of 16; other pools run as those two calls). */
void max_pool_quantize_nhwc_forward(const Tensor* X, Tensor* Y, PoolParams* params, const Tensor* Scale,
                                    const Tensor* ZeroPoint, int code_dtype, Tensor* Yc);
/* Weight codes int8 [M, C, KH, KW] -> Wk int8 [M, KH, KW, C] and WSum int32 [M, KH, KW],
 * the sum of each tap's C codes (the zero-point correction). */
void qconv_pack_weights(const Tensor* Wq, Tensor* Wk, Tensor* WSum);
typedef struct {
    const Tensor* x_scale;   /* one float32: DequantizeLinear scale of the input codes */
    const Tensor* x_zero;    /* one element of x_codes' dtype, or NULL (0) */
    int x_codes;             /* DataType of the input codes: DTYPE_UINT8 or DTYPE_INT8 */
    const Tensor* w;         /* int8 [M, KH, KW, C] (qconv_pack_weights), zero points 0 */
    const Tensor* w_sum;     /* int32 [M, KH, KW] (qconv_pack_weights) */
    const Tensor* w_scale;   /* float32 [M]: per-output-channel weight scale */
    const Tensor* bias;      /* float32 [M] or NULL */
    int relu;                /* 1: Relu after the bias */
    const Tensor* p;         /* 1x1 projection (pads 0, the conv's strides) added after the
                                Relu: int8 [M, 1, 1, C], or NULL */
    const Tensor* p_sum;     /* int32 [M, 1, 1] */
    const Tensor* p_scale;   /* float32 [M] */
    const Tensor* skip;      /* float32 [N, M, OH, OW] added after the Relu, or NULL */
    const Tensor* q_scale;   /* one float32: quantize the output for the next block
                                (Y int8 [N, OH, OW, M] in the layout above), or NULL:
                                Y float32 [N, M, OH, OW] */
    const Tensor* q_zero;    /* one element of y_codes' dtype, or NULL (0) */
    int y_codes;             /* DataType of the output codes: DTYPE_UINT8 or DTYPE_INT8 */
} QConvBlock;
/* Y = [Q](Relu?(Conv(DQ(X), DQ(w)) + bias) [+ Conv1x1(DQ(X), DQ(p))] [+ skip]); params as
 * conv2d_forward's (group 1; the output size follows from the pads, strides and
 * dilations).  M a multiple of 64. */
void qconv_block_forward(const Tensor* X, const QConvBlock* block, Tensor* Y, ConvParams* params);

#ifdef __cplusplus
}
#endif

#endif /* TENSOR_OPS_HIP_H */
