// e8t_workspace.cpp -- scratch device memory owned by the library: the fp32 partial sums
// of the prefill GEMM's K split.  One buffer per (device, stream), so launches on
// different streams never share scratch and launches on one stream are ordered by it.  A
// buffer only grows (in 8-MiB steps); the old one is freed after its stream has drained.
// Nothing is allocated while the stream is capturing a graph: the caller then runs the
// unsplit kernel, so a captured launch never depends on memory this file may free later.

#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "e8t_internal.h"

namespace ojx {
namespace {

struct Workspace {
    int dev;
    hipStream_t stream;
    void* ptr;
    size_t bytes;
};

std::mutex g_mu;
// Never destroyed: freeing device memory from a static destructor can run after the HIP
// runtime has shut down.  The buffers live until the process ends.
std::vector<Workspace>* g_spaces = new std::vector<Workspace>();

constexpr size_t kStep = size_t(8) << 20;

}  // namespace

void* stream_workspace(hipStream_t stream, size_t bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    Workspace* w = nullptr;
    for (Workspace& e : *g_spaces)
        if (e.dev == dev && e.stream == stream) {
            w = &e;
            break;
        }
    if (w && w->bytes >= bytes) return w->ptr;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &st) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (st != hipStreamCaptureStatusNone) return nullptr;
    if (w && w->ptr) {
        if (hipStreamSynchronize(stream) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        (void)hipFree(w->ptr);
        w->ptr = nullptr;
        w->bytes = 0;
    }
    const size_t want = (bytes + kStep - 1) / kStep * kStep;
    void* p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (w) {
        w->ptr = p;
        w->bytes = want;
    } else {
        g_spaces->push_back(Workspace{dev, stream, p, want});
    }
    return p;
}

}  // namespace ojx
