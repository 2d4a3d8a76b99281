// runtime.h — host runtime of libtensor_ops_hip.so: device/stream state,
// memory registry and caching pools, error reporting, and the staging helper
// that lets one operator entry point serve host tensors (reference
// semantics: synchronous, host-addressable data) and device tensors
// (asynchronous, HBM-resident) alike.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <vector>

#include "../../include/tensor_ops.h"
#include "common.h"

namespace tohip {

// ---- errors ---------------------------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
bool check_hip(hipError_t e, const char* what);   // false (and error set) on failure

// ---- device / stream --------------------------------------------------------
bool ensure_device();            // lazily initialises; false + error when no GPU
hipStream_t stream();            // current library stream
int device_count();
bool exact_mode();
const double* device_cos_lut();  // 4097 doubles in device memory (after init_cos_lut)
int num_cus();
int device_id();                 // the device the library stream belongs to (after ensure_device)

// ---- one-launch exchanges ----------------------------------------------------
// Kernels whose blocks exchange partial results through device memory in one
// launch (softmax over few long rows, DynamicQuantizeLinear) tag each published
// word with a number unique to the call, wait for the other blocks' words with a
// bounded poll and recompute what did not arrive.  The words live in buffers
// that hold nothing but exchange words: created zero-filled (0 is never a tag)
// and zero-filled again before their first use after the 32-bit tag counter
// wraps, so a word carries a call's tag only if that call wrote it.  A call
// captured into a graph would replay with its capture-time tag, so captured
// calls take the multi-launch forms (xchg_alloc refuses under capture).
// xchg_alloc: a buffer of at least `bytes` for one call on the library stream,
// and that call's tag in *tag; nullptr with the error set on failure.
void* xchg_alloc(size_t bytes, uint32_t* tag);
void xchg_free(void* p);         // back to the current stream's exchange list
int exchange_spin();             // the poll bound (tensor_ops_hip_set_softmax_spin)
bool stream_capturing(hipStream_t s);

// ---- fixed workspaces ----------------------------------------------------------
// Some paths keep their workspace in a file-scope __device__ array (each GPU
// holds its own copy until the process ends): the no-allocation entry point and
// calls captured into a graph, whose workspace must outlive the call.  In host
// code such an array's name is a host-side stand-in, so each owning file
// resolves the device address once, with hipGetSymbolAddress, in these hooks,
// which the device initialisation calls with the library's device current (no
// call under capture resolves one).  They record an error and leave the address
// null on failure; the paths that need it then report that error.
void init_qdq_workspace();
void init_reduce_workspace();

// Gemm -> Softmax over the last axis after a k-split Gemm (reduce.hip): adds the
// nsplit slices of M x N partial sums at part with the bias (cmode 0 none, 1
// one value, 2 per column, 3 per row of f32 c) into Y (f32 logits) and writes
// their row softmax to P (f32), bit for bit as the split reduction followed by
// softmax_forward.  false (nothing launched) unless 1 <= N <= 1024.
bool launch_splitk_softmax(const float* part, int nsplit, int M, int N, double alpha, double beta, const float* c,
                           int cmode, float* Y, float* P, hipStream_t s);

// ---- memory -----------------------------------------------------------------
enum class Mem { kHostPinned, kHostMalloc, kDevOwned, kDevBorrowed, kHostForeign, kDevForeign };
Mem classify(const void* p);     // registry first, then hipPointerGetAttributes
inline bool is_dev(Mem m) { return m == Mem::kDevOwned || m == Mem::kDevBorrowed || m == Mem::kDevForeign; }

// Device memory from the caching pool, reused in the order of the stream it was
// released on.  Refused (nullptr, error set) while the library stream is being
// captured into a graph: a buffer taken inside a capture goes back to the pool
// when the call returns while the graph goes on using it, and a fresh one would
// need hipMalloc inside the capture.
void* pool_alloc(size_t bytes);
void pool_free(void* p);

size_t tensor_bytes(const Tensor* t);
bool tensor_sane(const Tensor* t, const char* what);   // non-null, valid dtype, data present

// ---- launch shape -------------------------------------------------------------
inline unsigned grid_for(size_t work_items, unsigned block, unsigned max_blocks = 1u << 20) {
    size_t g = (work_items + block - 1) / block;
    if (g < 1) g = 1;
    if (g > max_blocks) g = max_blocks;
    return (unsigned)g;
}
bool check_launch(const char* kernel);   // reports hipGetLastError after a launch

// ---- broadcast descriptor -------------------------------------------------------
// Build a collapsed descriptor for `nop` operands against output shape `oshape`.
// Operand k is broadcast numpy-style (right-aligned; size-1 dims repeat).
// Returns false if a shape does not broadcast to oshape.
bool make_bdesc(BDesc& d, const int* oshape, int ond, const Tensor* const* ops, int nop);
// Flat descriptor (every operand indexed 0..n-1, or stride 0 for size-1 operands).
void make_flat_bdesc(BDesc& d, size_t n, const Tensor* const* ops, int nop);
// Descriptor against output Y: operands with Y->size elements index flat (as
// the reference does, whatever their shape), size-1 operands broadcast, and
// any other operand broadcasts numpy-style by its own shape.
bool make_bdesc_for(BDesc& d, const Tensor* Y, const Tensor* const* ops, int nop);

// ---- staging ----------------------------------------------------------------------
// Resolves each operand to a device pointer.  Host inputs are copied to pool
// buffers (H2D on the library stream); a host output gets a pool buffer that
// finish() copies back.  finish() synchronises only if staging happened, so
// calls on device-resident tensors stay asynchronous.  Under graph capture a
// host operand is an error (staging needs pool buffers and a synchronisation).
class Staging {
  public:
    Staging() = default;
    ~Staging();
    const void* in(const Tensor* t);               // nullptr on error (error set)
    void* out(Tensor* t, size_t bytes_written);    // bytes_written: prefix copied back
    bool finish();                                 // D2H + sync when needed
    bool staged() const { return staged_; }

  private:
    struct Buf { void* dev; void* host; size_t bytes; bool writeback; };
    std::vector<Buf> bufs_;
    bool staged_ = false;
    bool failed_ = false;
};

}  // namespace tohip
