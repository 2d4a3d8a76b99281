// runtime.hip — device state, memory registry, caching pools, staging and the
// tensor lifecycle entry points of libtensor_ops_hip.so.
#include "runtime.h"

#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>

namespace tohip {

// ---- errors -------------------------------------------------------------------
static thread_local std::string t_err;

void set_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_err = buf;
}

bool check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    set_error("%s: %s", what, hipGetErrorString(e));
    return false;
}

bool check_launch(const char* kernel) { return check_hip(hipGetLastError(), kernel); }

// ---- process-wide state (intentionally never destroyed: avoids teardown order
// problems with the HIP runtime at exit) ------------------------------------------
struct State {
    std::once_flag once;
    bool ok = false;
    std::string init_err;
    int ndev = 0, dev = 0, cus = 0;
    hipStream_t own = nullptr;
    std::atomic<hipStream_t> user{nullptr};

    std::mutex mu;                                        // registries + pools
    // Residency of data pointers (for classify): kind and the number of live
    // headers over the pointer, so two headers over one buffer (a wrapper over
    // a library tensor's data, or two wrappers) keep it classified until the
    // last one is freed.
    struct Res { Mem m; int refs; };
    std::unordered_map<const void*, Res> reg;
    // Ownership per header: how free_tensor releases the data of each header
    // this library returned (kDevBorrowed: the caller owns the data).
    std::unordered_map<const Tensor*, Mem> owners;
    // Cached HBM buffers per stream: a buffer freed while stream S was current
    // is handed out again only to work on S, so reuse follows S's order.
    std::map<hipStream_t, std::multimap<size_t, void*>> dev_free;
    std::unordered_map<void*, size_t> dev_size;
    size_t dev_cached = 0;
    std::multimap<size_t, void*> pin_free;
    std::unordered_map<void*, size_t> pin_size;
    size_t pin_cached = 0;
    // Exchange-word buffers (xchg_alloc), kept apart from the pool above so
    // they never hold anything but exchange words: per-stream free lists, and
    // per buffer its size and the tag epoch it was last zero-filled in.
    struct XBuf { size_t bytes; uint32_t epoch; };
    std::map<hipStream_t, std::multimap<size_t, void*>> xchg_free;
    std::unordered_map<void*, XBuf> xchg_info;
    // Cached buffers of a stream that a thread left (tensor_ops_hip_set_thread_stream):
    // free for any stream once `ev`, recorded on the old stream at the switch, completes.
    struct Parked { hipEvent_t ev; std::multimap<size_t, void*> dev, xchg; };
    std::vector<Parked> parked;

    std::mutex lut_mu;
    std::atomic<int> lut_host_ready{0};
    std::atomic<int> lut_dev_ready{0};
    double lut[4097];
    double* d_lut = nullptr;
};

static State& S() {
    static State* s = new State;
    return *s;
}

static void reclaim_parked(State& s, hipStream_t st);

static constexpr size_t kDevCacheLimit = size_t(32) << 30;   // 32 GiB of cached HBM buffers
static constexpr size_t kPinCacheLimit = size_t(4) << 30;

static void do_init() {
    State& s = S();
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        s.init_err = "no HIP device available (libtensor_ops_hip needs an MI355X / gfx950 GPU)";
        return;
    }
    s.ndev = n;
    if (hipGetDevice(&s.dev) != hipSuccess) s.dev = 0;
    if (hipSetDevice(s.dev) != hipSuccess ||
        hipStreamCreateWithFlags(&s.own, hipStreamDefault) != hipSuccess) {
        (void)hipGetLastError();
        s.init_err = "failed to set up the HIP device / stream";
        return;
    }
    if (hipDeviceGetAttribute(&s.cus, hipDeviceAttributeMultiprocessorCount, s.dev) != hipSuccess)
        s.cus = 256;
    s.ok = true;
    init_qdq_workspace();
    init_reduce_workspace();
}

bool ensure_device() {
    State& s = S();
    std::call_once(s.once, do_init);
    if (!s.ok) set_error("%s", s.init_err.c_str());
    return s.ok;
}

int device_count() {
    State& s = S();
    std::call_once(s.once, do_init);
    return s.ok ? s.ndev : 0;
}

// Stream of the calling thread (tensor_ops_hip_set_thread_stream), if set.
static thread_local hipStream_t t_stream = nullptr;

hipStream_t stream() {
    if (t_stream) return t_stream;
    State& s = S();
    hipStream_t u = s.user.load();
    return u ? u : s.own;
}

// Precision mode per calling thread (-1: not set yet, take the process default).
static thread_local int t_exact = -1;

static int default_exact() {
    const char* ex = getenv("TENSOR_OPS_HIP_EXACT");
    return (ex && *ex == '1') ? 1 : 0;
}

bool exact_mode() {
    if (t_exact < 0) t_exact = default_exact();
    return t_exact != 0;
}
int num_cus() { return S().cus > 0 ? S().cus : 256; }
int device_id() { return S().dev; }

// ---- one-launch exchanges ---------------------------------------------------------
// One 64-bit count per call: its low 32 bits are the call's tag (0 skipped, so
// zero-filled words never match), its high bits the epoch.  Tags are unique
// within an epoch; a buffer handed out in an epoch other than the one it was
// last zero-filled in is zero-filled first (on the stream, before the kernel),
// so a word carrying a call's tag was written by that call.
std::atomic<uint64_t> g_xchg_count{0};

void* xchg_alloc(size_t bytes, uint32_t* tag) {
    State& s = S();
    const hipStream_t st = stream();
    if (stream_capturing(st)) {
        set_error("exchange workspace requested while the library stream is being captured");
        return nullptr;
    }
    uint64_t c;
    do c = g_xchg_count.fetch_add(1, std::memory_order_relaxed) + 1; while ((uint32_t)c == 0);
    const uint32_t epoch = (uint32_t)(c >> 32);
    const size_t need = bytes < 256 ? 256 : (bytes + 255) / 256 * 256;
    void* p = nullptr;
    size_t have = 0;
    bool fill = true;
    {
        std::lock_guard<std::mutex> g(s.mu);
        if (!s.parked.empty()) reclaim_parked(s, st);
        auto fl = s.xchg_free.find(st);
        if (fl != s.xchg_free.end()) {
            auto it = fl->second.lower_bound(need);    // any larger one serves (they are a few KB)
            if (it != fl->second.end()) {
                p = it->second;
                fl->second.erase(it);
                State::XBuf& xb = s.xchg_info[p];
                have = xb.bytes;
                fill = xb.epoch != epoch;
                xb.epoch = epoch;
            }
        }
    }
    if (!p) {
        if (!check_hip(hipMalloc(&p, need), "exchange workspace")) return nullptr;
        have = need;
        std::lock_guard<std::mutex> g(s.mu);
        s.xchg_info[p] = State::XBuf{need, epoch};
    }
    if (fill && !check_hip(hipMemsetAsync(p, 0, have, st), "exchange workspace fill")) {
        std::lock_guard<std::mutex> g(s.mu);
        s.xchg_info[p].epoch = epoch + 1;             // not filled: fill before its next use
        s.xchg_free[st].emplace(have, p);
        return nullptr;
    }
    *tag = (uint32_t)c;
    return p;
}

void xchg_free(void* p) {
    if (!p) return;
    State& s = S();
    std::lock_guard<std::mutex> g(s.mu);
    auto it = s.xchg_info.find(p);
    if (it == s.xchg_info.end()) return;
    s.xchg_free[stream()].emplace(it->second.bytes, p);
}

// Polls of ~64 cycles each before a block recomputes what has not arrived (about
// 0.5 ms: far longer than any co-resident block takes to publish).
constexpr int kXchgSpinDefault = 1 << 14;
std::atomic<int> g_xchg_spin{kXchgSpinDefault};
int exchange_spin() { return g_xchg_spin.load(std::memory_order_relaxed); }

bool stream_capturing(hipStream_t s) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return cs != hipStreamCaptureStatusNone;
}

// Test hook: byte that fills every buffer handed out with undefined contents
// (create_tensor_device_empty, staged outputs), or -1 for none.
std::atomic<int> g_poison{-1};

// ---- memory -------------------------------------------------------------------------
// Records a new header t over data p.  An owning kind (library allocation)
// takes precedence over a borrowed one for the residency entry.
static void reg_put(const Tensor* t, const void* p, Mem m) {
    std::lock_guard<std::mutex> g(S().mu);
    S().owners[t] = m;
    auto it = S().reg.find(p);
    if (it == S().reg.end()) {
        S().reg.emplace(p, State::Res{m, 1});
    } else {
        it->second.refs++;
        if (m != Mem::kDevBorrowed) it->second.m = m;
    }
}

// Forgets header t; returns false for a header this library did not create.
// *m is how t's data must be released.
static bool reg_take(const Tensor* t, Mem* m) {
    std::lock_guard<std::mutex> g(S().mu);
    auto ot = S().owners.find(t);
    if (ot == S().owners.end()) return false;
    *m = ot->second;
    S().owners.erase(ot);
    auto it = S().reg.find(t->data);
    if (it != S().reg.end() && --it->second.refs <= 0) S().reg.erase(it);
    return true;
}

Mem classify(const void* p) {
    {
        std::lock_guard<std::mutex> g(S().mu);
        auto it = S().reg.find(p);
        if (it != S().reg.end()) return it->second.m;
    }
    if (!S().ok) return Mem::kHostForeign;
    hipPointerAttribute_t a;
    memset(&a, 0, sizeof a);
    if (hipPointerGetAttributes(&a, p) == hipSuccess &&
        (a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged))
        return Mem::kDevForeign;
    (void)hipGetLastError();
    return Mem::kHostForeign;
}

static size_t round_bytes(size_t b) {
    if (b <= 256) return 256;
    if (b < (size_t(1) << 20)) {
        size_t r = 512;
        while (r < b) r <<= 1;
        return r;
    }
    const size_t mb = size_t(1) << 20;
    return (b + mb - 1) / mb * mb;
}

// Parked buffers whose event has completed join stream st's lists (s.mu held).
static void reclaim_parked(State& s, hipStream_t st) {
    for (size_t i = 0; i < s.parked.size();) {
        State::Parked& pk = s.parked[i];
        if (hipEventQuery(pk.ev) != hipSuccess) { (void)hipGetLastError(); i++; continue; }
        (void)hipEventDestroy(pk.ev);
        if (!pk.dev.empty()) s.dev_free[st].insert(pk.dev.begin(), pk.dev.end());
        if (!pk.xchg.empty()) s.xchg_free[st].insert(pk.xchg.begin(), pk.xchg.end());
        s.parked.erase(s.parked.begin() + (std::ptrdiff_t)i);
    }
}

static void* take_cached(std::multimap<size_t, void*>& fl, size_t need, size_t& cached) {
    auto it = fl.lower_bound(need);
    if (it == fl.end() || it->first > need + need / 8) return nullptr;
    void* p = it->second;
    cached -= it->first;
    fl.erase(it);
    return p;
}

void* pool_alloc(size_t bytes) {
    State& s = S();
    if (stream_capturing(stream())) {
        set_error("device memory requested while the library stream is being captured into a graph "
                  "(allocate before the capture; captured calls must not allocate)");
        return nullptr;
    }
    const size_t need = round_bytes(bytes);
    {
        std::lock_guard<std::mutex> g(s.mu);
        if (!s.parked.empty()) reclaim_parked(s, stream());
        auto fl = s.dev_free.find(stream());
        if (fl != s.dev_free.end())
            if (void* p = take_cached(fl->second, need, s.dev_cached)) return p;
    }
    void* p = nullptr;
    if (hipMalloc(&p, need) != hipSuccess) {
        (void)hipGetLastError();
        // Release the cache and retry once (parked buffers after their event).
        std::lock_guard<std::mutex> g(s.mu);
        for (State::Parked& pk : s.parked) {
            (void)hipEventSynchronize(pk.ev);
            (void)hipEventDestroy(pk.ev);
            for (auto& kv : pk.dev) {
                (void)hipFree(kv.second);
                s.dev_size.erase(kv.second);
            }
            if (!pk.xchg.empty()) s.xchg_free[stream()].insert(pk.xchg.begin(), pk.xchg.end());
        }
        s.parked.clear();
        for (auto& per_stream : s.dev_free)
            for (auto& kv : per_stream.second) {
                (void)hipFree(kv.second);
                s.dev_size.erase(kv.second);
            }
        s.dev_free.clear();
        s.dev_cached = 0;
        if (hipMalloc(&p, need) != hipSuccess) {
            (void)hipGetLastError();
            set_error("hipMalloc(%zu) failed: out of device memory", need);
            return nullptr;
        }
    }
    std::lock_guard<std::mutex> g(s.mu);
    s.dev_size[p] = need;
    return p;
}

void pool_free(void* p) {
    if (!p) return;
    State& s = S();
    std::lock_guard<std::mutex> g(s.mu);
    auto it = s.dev_size.find(p);
    if (it == s.dev_size.end()) return;
    if (s.dev_cached + it->second > kDevCacheLimit) {
        (void)hipFree(p);
        s.dev_size.erase(it);
        return;
    }
    s.dev_cached += it->second;
    s.dev_free[stream()].emplace(it->second, p);
}

static void* pinned_alloc(size_t bytes) {
    State& s = S();
    const size_t need = round_bytes(bytes);
    {
        std::lock_guard<std::mutex> g(s.mu);
        if (void* p = take_cached(s.pin_free, need, s.pin_cached)) return p;
    }
    void* p = nullptr;
    if (hipHostMalloc(&p, need, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    std::lock_guard<std::mutex> g(s.mu);
    s.pin_size[p] = need;
    return p;
}

static void pinned_free(void* p) {
    State& s = S();
    std::lock_guard<std::mutex> g(s.mu);
    auto it = s.pin_size.find(p);
    if (it == s.pin_size.end()) return;
    if (s.pin_cached + it->second > kPinCacheLimit) {
        (void)hipHostFree(p);
        s.pin_size.erase(it);
        return;
    }
    s.pin_cached += it->second;
    s.pin_free.emplace(it->second, p);
}

size_t tensor_bytes(const Tensor* t) { return t->size * dt_bytes((int)t->dtype); }

bool tensor_sane(const Tensor* t, const char* what) {
    if (!t) { set_error("%s: NULL tensor", what); return false; }
    if (!dt_valid((int)t->dtype)) { set_error("%s: invalid dtype %d", what, (int)t->dtype); return false; }
    if (!t->data && t->size) { set_error("%s: tensor has no data", what); return false; }
    return true;
}

// ---- broadcast descriptors ------------------------------------------------------------
bool make_bdesc(BDesc& d, const int* oshape, int ond, const Tensor* const* ops, int nop) {
    if (ond < 0 || ond > 16) { set_error("rank %d not supported (max 16)", ond); return false; }
    int64_t dims[17];
    int64_t st[kMaxOperands][17];
    int nd = ond;
    for (int a = 0; a < nd; a++) dims[a] = oshape[a];
    for (int k = 0; k < nop; k++) {
        const Tensor* t = ops[k];
        if (t->ndim > ond) {
            // Leading size-1 dims beyond the output rank are allowed.
            for (int a = 0; a < t->ndim - ond; a++)
                if (t->shape[a] != 1) { set_error("operand %d rank %d exceeds output rank %d", k, t->ndim, ond); return false; }
        }
        int64_t stride = 1;
        for (int a = nd - 1; a >= 0; a--) {
            const int ta = t->ndim - (nd - a);
            const int64_t ext = ta >= 0 ? t->shape[ta] : 1;
            if (ext == dims[a]) st[k][a] = (ext == 1) ? 0 : stride;
            else if (ext == 1) st[k][a] = 0;
            else { set_error("operand %d shape does not broadcast to the output shape", k); return false; }
            stride *= ext;
        }
    }
    // Drop size-1 dims, then merge neighbours that are contiguous for every operand.
    int64_t cd[17], cs[kMaxOperands][17];
    int m = 0;
    for (int a = 0; a < nd; a++) {
        if (dims[a] == 1) continue;
        if (m > 0) {
            bool merge = true;
            for (int k = 0; k < nop; k++)
                if (cs[k][m - 1] != st[k][a] * dims[a]) { merge = false; break; }
            if (merge) {
                cd[m - 1] *= dims[a];
                for (int k = 0; k < nop; k++) cs[k][m - 1] = st[k][a];
                continue;
            }
        }
        cd[m] = dims[a];
        for (int k = 0; k < nop; k++) cs[k][m] = st[k][a];
        m++;
    }
    if (m == 0) {
        cd[0] = 1;
        for (int k = 0; k < nop; k++) cs[k][0] = 0;
        m = 1;
    }
    if (m > kMaxDims) { set_error("broadcast pattern needs %d dims (max %d)", m, kMaxDims); return false; }
    d.nd = m;
    for (int a = 0; a < m; a++) {
        d.dim64[a] = cd[a];
        d.dim[a] = (uint32_t)(cd[a] > 0xFFFFFFFFll ? 0xFFFFFFFFu : cd[a]);
        d.fd[a] = make_fastdiv(d.dim[a] ? d.dim[a] : 1);
        for (int k = 0; k < kMaxOperands; k++) d.st[k][a] = k < nop ? cs[k][a] : 0;
    }
    return true;
}

void make_flat_bdesc(BDesc& d, size_t n, const Tensor* const* ops, int nop) {
    d.nd = 1;
    d.dim64[0] = (int64_t)n;
    d.dim[0] = (uint32_t)(n > 0xFFFFFFFFull ? 0xFFFFFFFFu : n);
    d.fd[0] = make_fastdiv(d.dim[0] ? d.dim[0] : 1);
    for (int k = 0; k < kMaxOperands; k++) d.st[k][0] = (k < nop && ops[k]->size != 1) ? 1 : 0;
}

bool make_bdesc_for(BDesc& d, const Tensor* Y, const Tensor* const* ops, int nop) {
    bool all_flat = true;
    for (int k = 0; k < nop; k++)
        if (ops[k]->size != Y->size && ops[k]->size != 1) all_flat = false;
    if (all_flat) {
        make_flat_bdesc(d, Y->size, ops, nop);
        return true;
    }
    Tensor views[kMaxOperands];
    const Tensor* vp[kMaxOperands];
    for (int k = 0; k < nop; k++) {
        views[k] = *ops[k];
        if (ops[k]->size == Y->size) { views[k].shape = Y->shape; views[k].ndim = Y->ndim; }
        vp[k] = &views[k];
    }
    return make_bdesc(d, Y->shape, Y->ndim, vp, nop);
}

// ---- staging --------------------------------------------------------------------------
Staging::~Staging() {
    for (auto& b : bufs_) pool_free(b.dev);
}

// A host operand under graph capture: staging would allocate and synchronise.
static bool refuse_host_under_capture() {
    if (!stream_capturing(stream())) return false;
    set_error("host tensor used while the library stream is being captured into a graph "
              "(captured calls take device tensors only)");
    return true;
}

const void* Staging::in(const Tensor* t) {
    if (!t->size) return t->data;
    const Mem m = classify(t->data);
    if (is_dev(m)) return t->data;
    if (refuse_host_under_capture()) { failed_ = true; return nullptr; }
    const size_t b = tensor_bytes(t);
    void* d = pool_alloc(b);
    if (!d) { failed_ = true; return nullptr; }
    bufs_.push_back({d, nullptr, b, false});
    staged_ = true;
    if (!check_hip(hipMemcpyAsync(d, t->data, b, hipMemcpyHostToDevice, stream()), "H2D copy")) {
        failed_ = true;
        return nullptr;
    }
    return d;
}

void* Staging::out(Tensor* t, size_t bytes_written) {
    if (!t->size) return t->data;
    const Mem m = classify(t->data);
    if (is_dev(m)) return t->data;
    if (refuse_host_under_capture()) { failed_ = true; return nullptr; }
    void* d = pool_alloc(tensor_bytes(t));
    if (!d) { failed_ = true; return nullptr; }
    const int poison = g_poison.load(std::memory_order_relaxed);
    if (poison >= 0 && !check_hip(hipMemsetAsync(d, poison, tensor_bytes(t), stream()), "poison fill")) {
        pool_free(d);
        failed_ = true;
        return nullptr;
    }
    bufs_.push_back({d, t->data, bytes_written, true});
    staged_ = true;
    return d;
}

bool Staging::finish() {
    if (!staged_) return !failed_;
    bool ok = !failed_;
    if (ok) {
        for (auto& b : bufs_)
            if (b.writeback && b.bytes &&
                !check_hip(hipMemcpyAsync(b.host, b.dev, b.bytes, hipMemcpyDeviceToHost, stream()), "D2H copy"))
                ok = false;
    }
    if (!check_hip(hipStreamSynchronize(stream()), "stream synchronize")) ok = false;
    return ok;
}

// ---- cosine table ---------------------------------------------------------------------
// Replica of tensor_ops.c:763-807, evaluated on the host in double with
// contraction off (this file is compiled with -ffp-contract=off), which gives
// the reference's table bit for bit.  The literals are the reference's.
static void build_lut(double* T) {
    const double pi = 3.141592653589793238462643383279502884197;
    const double two_pi = 2.0 * pi, half_pi = pi / 2.0;
    for (int i = 0; i <= 4096; i++) {
        double x = (double)i * two_pi / 4096;
        double sg = 1.0;
        if (x > pi) x = two_pi - x;
        if (x > half_pi) { x = pi - x; sg = -1.0; }
        const double x2 = x * x;
        double r;
        if (x < 0.785398163397448) {
            r = 1.0 + x2 * (-0.5 + x2 * (0.04166666666666666 +
                x2 * (-0.001388888888888889 + x2 * 0.000024801587301587302)));
        } else {
            const double t = half_pi - x, t2 = t * t;
            r = t * (1.0 + t2 * (-0.16666666666666666 + t2 * (0.008333333333333333 +
                t2 * (-0.0001984126984126984 + t2 * 0.0000027557319223985893))));
        }
        T[i] = sg * r;
    }
}

static bool lut_ready_on_device() {
    State& s = S();
    if (s.lut_dev_ready.load(std::memory_order_acquire)) return true;
    std::lock_guard<std::mutex> g(s.lut_mu);
    if (!s.lut_host_ready.load()) {
        build_lut(s.lut);
        s.lut_host_ready.store(1, std::memory_order_release);
    }
    if (s.lut_dev_ready.load()) return true;
    if (!ensure_device()) return false;
    if (!check_hip(hipMalloc(&s.d_lut, sizeof s.lut), "cos table alloc")) return false;
    if (!check_hip(hipMemcpy(s.d_lut, s.lut, sizeof s.lut, hipMemcpyHostToDevice), "cos table upload"))
        return false;
    s.lut_dev_ready.store(1, std::memory_order_release);
    return true;
}

const double* device_cos_lut() { return lut_ready_on_device() ? S().d_lut : nullptr; }

}  // namespace tohip

using namespace tohip;

// ======================= C ABI: lifecycle and extensions ==============================
extern "C" {

static Tensor* new_header(const int* shape, int ndim, DataType dtype) {
    if (ndim < 0 || (ndim > 0 && !shape)) { set_error("create_tensor: bad shape"); return nullptr; }
    Tensor* t = (Tensor*)malloc(sizeof(Tensor));
    if (!t) return nullptr;
    t->ndim = ndim;
    t->dtype = dtype;
    t->shape = (int*)malloc((size_t)(ndim > 0 ? ndim : 1) * sizeof(int));
    if (!t->shape) { free(t); return nullptr; }
    size_t n = 1;
    for (int d = 0; d < ndim; d++) {
        t->shape[d] = shape[d];
        n *= (size_t)(shape[d] > 0 ? shape[d] : 0);
    }
    t->size = n;
    t->data = nullptr;
    return t;
}

// tensor_ops.c:357-433 — zeroed host data.  With a GPU present the data is
// pinned (DMA-capable) host memory; otherwise calloc, as the reference.
Tensor* create_tensor(int* shape, int ndim, DataType dtype) {
    Tensor* t = new_header(shape, ndim, dtype);
    if (!t) return nullptr;
    const size_t bytes = t->size * dt_bytes((int)dtype);
    void* p = nullptr;
    Mem kind = Mem::kHostMalloc;
    if (device_count() > 0 && bytes >= 4096 && (p = pinned_alloc(bytes)) != nullptr) {
        memset(p, 0, bytes);
        kind = Mem::kHostPinned;
    } else {
        p = calloc(t->size ? t->size : 1, dt_bytes((int)dtype));
    }
    if (!p) { free(t->shape); free(t); return nullptr; }
    t->data = p;
    reg_put(t, p, kind);
    return t;
}

// Refused while the library stream is being captured into a graph: the pool
// buffer would go back to the pool at free_tensor while the graph still holds
// it, and the fill would record a memset node.
static Tensor* device_tensor(int* shape, int ndim, DataType dtype, bool zero) {
    if (!ensure_device()) return nullptr;
    if (stream_capturing(stream())) {
        set_error("%s: device tensors cannot be created while the library stream is being captured into a graph "
                  "(create them before the capture)", zero ? "create_tensor_device" : "create_tensor_device_empty");
        return nullptr;
    }
    Tensor* t = new_header(shape, ndim, dtype);
    if (!t) return nullptr;
    const size_t bytes = t->size * dt_bytes((int)dtype);
    void* p = pool_alloc(bytes ? bytes : 1);
    if (!p) { free(t->shape); free(t); return nullptr; }
    const int fill = zero ? 0 : g_poison.load(std::memory_order_relaxed);
    if (fill >= 0 && !check_hip(hipMemsetAsync(p, fill, bytes ? bytes : 1, stream()), "fill")) {
        pool_free(p);
        free(t->shape);
        free(t);
        return nullptr;
    }
    t->data = p;
    reg_put(t, p, Mem::kDevOwned);
    return t;
}

Tensor* create_tensor_device(int* shape, int ndim, DataType dtype) { return device_tensor(shape, ndim, dtype, true); }
Tensor* create_tensor_device_empty(int* shape, int ndim, DataType dtype) {
    return device_tensor(shape, ndim, dtype, false);
}

Tensor* tensor_wrap_device(void* device_ptr, int* shape, int ndim, DataType dtype) {
    Tensor* t = new_header(shape, ndim, dtype);
    if (!t) return nullptr;
    t->data = device_ptr;
    reg_put(t, device_ptr, Mem::kDevBorrowed);
    return t;
}

// tensor_ops.c:440-450.  Data is released according to how this header was
// created (create_tensor: host memory; create_tensor_device*: HBM pool;
// tensor_wrap_device: left to the caller), whatever other headers share it.
// A header this library did not create is not touched (its memory cannot be
// attributed to an allocator) and an error is recorded.
void free_tensor(Tensor* t) {
    if (!t) return;
    Mem m;
    if (!reg_take(t, &m)) {
        set_error("free_tensor: tensor was not created by this library");
        return;
    }
    if (t->data) {
        if (m == Mem::kHostMalloc) free(t->data);
        else if (m == Mem::kHostPinned) pinned_free(t->data);
        else if (m == Mem::kDevOwned) pool_free(t->data);
        // kDevBorrowed: caller owns the memory.
    }
    free(t->shape);
    free(t);
}

int tensor_is_device(const Tensor* t) { return (t && t->data && is_dev(classify(t->data))) ? 1 : 0; }

// A copy that synchronises, refused under graph capture (a synchronisation
// there would invalidate the capture).
static bool sync_copy_under_capture(const char* name) {
    if (!stream_capturing(stream())) return false;
    set_error("%s: synchronous copy while the library stream is being captured into a graph", name);
    return true;
}

int tensor_to_host(const Tensor* t, void* host_dst) {
    if (!tensor_sane(t, "tensor_to_host") || !host_dst) return -1;
    const size_t b = tensor_bytes(t);
    if (!b) return 0;
    if (is_dev(classify(t->data))) {
        if (sync_copy_under_capture("tensor_to_host")) return -1;
        if (!check_hip(hipMemcpyAsync(host_dst, t->data, b, hipMemcpyDeviceToHost, stream()), "D2H copy") ||
            !check_hip(hipStreamSynchronize(stream()), "stream synchronize"))
            return -1;
    } else {
        memcpy(host_dst, t->data, b);
    }
    return 0;
}

int tensor_from_host(Tensor* t, const void* host_src) {
    if (!tensor_sane(t, "tensor_from_host") || !host_src) return -1;
    const size_t b = tensor_bytes(t);
    if (!b) return 0;
    if (is_dev(classify(t->data))) {
        if (sync_copy_under_capture("tensor_from_host")) return -1;
        if (!check_hip(hipMemcpyAsync(t->data, host_src, b, hipMemcpyHostToDevice, stream()), "H2D copy") ||
            !check_hip(hipStreamSynchronize(stream()), "stream synchronize"))
            return -1;
    } else {
        memcpy(t->data, host_src, b);
    }
    return 0;
}

// tensor_ops.c:1289-1299: a byte copy of input->size elements of the input's
// width, done only when the element counts match.  Device tensors copy on the
// library stream (asynchronous); a host operand makes the call synchronous.
// Where the reference would silently do nothing (count mismatch) or overrun a
// narrower output, an error is reported instead.
static void copy_tensor(const Tensor* in, Tensor* out, const char* name) {
    if (!tensor_sane(in, name) || !tensor_sane(out, name)) return;
    if (in->size != out->size) { set_error("%s: %zu elements into %zu", name, in->size, out->size); return; }
    const size_t b = in->size * dt_bytes((int)in->dtype);
    if (b > tensor_bytes(out)) { set_error("%s: output holds fewer bytes than the input", name); return; }
    if (!b || in->data == out->data) return;
    const bool di = is_dev(classify(in->data)), dout = is_dev(classify(out->data));
    if (!di && !dout) { memcpy(out->data, in->data, b); return; }
    if (!ensure_device()) return;
    if (!(di && dout) && sync_copy_under_capture(name)) return;
    if (!check_hip(hipMemcpyAsync(out->data, in->data, b, hipMemcpyDefault, stream()), name)) return;
    if (!(di && dout)) (void)check_hip(hipStreamSynchronize(stream()), "stream synchronize");
}

void flatten_forward(const Tensor* input, Tensor* output) { copy_tensor(input, output, "flatten_forward"); }
void reshape_forward(const Tensor* input, Tensor* output) { copy_tensor(input, output, "reshape_forward"); }

int tensor_ops_hip_sync(void) {
    if (!ensure_device()) return -1;
    return check_hip(hipStreamSynchronize(stream()), "stream synchronize") ? 0 : -1;
}

// Buffers cached under stream `from` (pool and exchange lists) now serve `to`.
// The caller has drained `from`, so no work of it still uses them.
static void move_cached(hipStream_t from, hipStream_t to) {
    if (from == to) return;
    State& st = S();
    std::lock_guard<std::mutex> g(st.mu);
    for (auto* lists : {&st.dev_free, &st.xchg_free}) {
        auto it = lists->find(from);
        if (it == lists->end()) continue;
        auto& dst = (*lists)[to];
        for (auto& kv : it->second) dst.emplace(kv.first, kv.second);
        lists->erase(it);
    }
}

// Buffers cached under stream `from`, which the calling thread leaves without
// draining it: they wait behind an event recorded on `from` now, and any
// stream may take them once that event has completed (reclaim_parked).
static void park_cached(hipStream_t from) {
    State& st = S();
    std::lock_guard<std::mutex> g(st.mu);
    auto d = st.dev_free.find(from);
    auto x = st.xchg_free.find(from);
    if (d == st.dev_free.end() && x == st.xchg_free.end()) return;
    State::Parked pk{nullptr, {}, {}};
    if (hipEventCreateWithFlags(&pk.ev, hipEventDisableTiming) != hipSuccess ||
        hipEventRecord(pk.ev, from) != hipSuccess) {
        (void)hipGetLastError();
        if (pk.ev) (void)hipEventDestroy(pk.ev);
        return;                       // left under `from` (used again if the thread comes back to it)
    }
    if (d != st.dev_free.end()) { pk.dev.swap(d->second); st.dev_free.erase(d); }
    if (x != st.xchg_free.end()) { pk.xchg.swap(x->second); st.xchg_free.erase(x); }
    st.parked.push_back(std::move(pk));
}

void tensor_ops_hip_set_stream(void* s) {
    if (!ensure_device()) return;
    State& st = S();
    // Drain the previous stream, then its cached buffers may serve the new one.
    const hipStream_t old_s = st.user.load() ? st.user.load() : st.own;
    (void)hipStreamSynchronize(old_s);
    st.user.store((hipStream_t)s);
    move_cached(old_s, s ? (hipStream_t)s : st.own);
}

// A thread leaving its own stream (cleared or replaced) parks the buffers
// cached under it behind an event on that stream, so nothing stays keyed by a
// handle that the caller may destroy (and the runtime may give to a new stream
// while the old one's work still uses them); nothing is drained.
void tensor_ops_hip_set_thread_stream(void* s) {
    if (!ensure_device()) return;
    const hipStream_t old_s = t_stream;
    if (old_s && old_s != (hipStream_t)s && !stream_capturing(old_s)) park_cached(old_s);
    t_stream = (hipStream_t)s;
}

void* tensor_ops_hip_get_stream(void) { return ensure_device() ? (void*)stream() : nullptr; }

int tensor_ops_hip_device_count(void) { return device_count(); }

const char* tensor_ops_hip_last_error(void) { return t_err.c_str(); }

void tensor_ops_hip_clear_error(void) { t_err.clear(); }

const char* tensor_ops_hip_version(void) { return "libtensor_ops_hip 0.1 (gfx950)"; }

void tensor_ops_hip_set_exact(int exact) { t_exact = exact ? 1 : 0; }

int tensor_ops_hip_set_softmax_spin(int polls) {
    return tohip::g_xchg_spin.exchange(polls < 0 ? tohip::kXchgSpinDefault : polls);
}

int tensor_ops_hip_get_exact(void) { return exact_mode() ? 1 : 0; }

int tensor_ops_hip_set_poison(int byte) {
    return tohip::g_poison.exchange(byte < 0 ? -1 : (byte & 0xFF));
}

unsigned long long tensor_ops_hip_advance_exchange_count(unsigned long long count) {
    uint64_t cur = tohip::g_xchg_count.load();
    while (cur < count && !tohip::g_xchg_count.compare_exchange_weak(cur, count)) {
    }
    return tohip::g_xchg_count.load();
}

// tensor_ops.c:763-807 — builds the table once and uploads it when a GPU is present.
void init_cos_lut(void) {
    State& s = S();
    {
        std::lock_guard<std::mutex> g(s.lut_mu);
        if (!s.lut_host_ready.load()) {
            build_lut(s.lut);
            s.lut_host_ready.store(1, std::memory_order_release);
        }
    }
    if (device_count() > 0) (void)lut_ready_on_device();
}

}  // extern "C"
