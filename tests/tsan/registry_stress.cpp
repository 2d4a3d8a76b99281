// Multi-threaded stress of libtensor_ops_hip's host runtime (tensor lifecycle,
// residency / ownership registry, thread-local errors and precision mode),
// built with ThreadSanitizer on a machine without a GPU (tests/test_tsan_runtime.py).
// Exits 0 when every check holds; TSan reports races on stderr.
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/tensor_ops.h"

// runtime.hip's device initialisation calls the workspace hooks of the kernel
// files, which this CPU-only build does not link; no device is initialised here.
namespace tohip {
void init_qdq_workspace() {}
void init_reduce_workspace() {}
}  // namespace tohip

static float shared_buf[64];

int main() {
    const int kThreads = 8, kIters = 400;
    std::vector<std::thread> ts;
    int failures[kThreads] = {};
    for (int t = 0; t < kThreads; t++) {
        ts.emplace_back([t, &failures]() {
            int shape[2] = {4, 16};
            for (int i = 0; i < kIters; i++) {
                Tensor* a = create_tensor(shape, 2, DTYPE_FLOAT32);
                if (!a || a->size != 64) { failures[t]++; continue; }
                for (int k = 0; k < 64; k++)
                    if (((float*)a->data)[k] != 0.0f) failures[t]++;
                // a wrapper over a library tensor's data, and several threads
                // wrapping one caller-owned buffer at once
                Tensor* w = tensor_wrap_device(a->data, shape, 2, DTYPE_FLOAT32);
                Tensor* s = tensor_wrap_device(shared_buf, shape, 2, DTYPE_FLOAT32);
                (void)tensor_is_device(w);
                (void)tensor_is_device(s);
                if ((i + t) & 1) { free_tensor(w); free_tensor(a); }
                else { free_tensor(a); free_tensor(w); }
                free_tensor(s);
                tensor_ops_hip_set_exact((i + t) & 1);
                if (tensor_ops_hip_get_exact() != ((i + t) & 1)) failures[t]++;
                tensor_ops_hip_clear_error();
                Tensor bogus;
                memset(&bogus, 0, sizeof bogus);
                free_tensor(&bogus);                      // not created by the library: refused
                if (!strstr(tensor_ops_hip_last_error(), "not created")) failures[t]++;
                tensor_ops_hip_clear_error();
            }
        });
    }
    for (auto& th : ts) th.join();
    int total = 0;
    for (int t = 0; t < kThreads; t++) total += failures[t];
    std::printf("registry_stress: %d threads x %d iterations, %d failed checks\n", kThreads, kIters, total);
    return total ? 1 : 0;
}
