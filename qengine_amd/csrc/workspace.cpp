// Library-owned workspaces of the prefill GEMMs (split-K partial sums, the W4A8 / W8A8 and fp16-accumulate
// pre-pass buffers) and of the one-pass decode's tail (counters and part sums), one buffer per (kind, device, stream).
//
// The reference keeps these buffers thread_local (src/kernels/gemm.cu:3258-3368), so two host threads never share
// one. Here the key is the stream a call is enqueued on: calls on one stream run in order, so they can share a
// buffer, while calls on two streams of one device (or two graphs replayed on two streams) get two buffers and cannot
// overwrite each other's data. A buffer grows on a call outside graph capture; the outgrown one is kept allocated
// (retired, never freed: a graph captured earlier may still read it). During capture a buffer that is too small is
// not grown: stream_ws returns nullptr and the caller either runs without it (the GEMM's split) or aborts with a
// message (the pre-passes), so callers size it first with an eager call or stream_ws_reserve on that stream.
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "qe_api.hpp"

namespace {
struct Ws {
    void* p = nullptr;
    size_t bytes = 0;
};
std::mutex g_mu;
std::map<std::tuple<int, int, hipStream_t>, Ws> g_ws;  // (kind, device, stream) -> buffer
std::vector<void*> g_retired;
}  // namespace

void* stream_ws(int kind, size_t bytes, hipStream_t st) {
    CHECK(kind >= 0 && kind < kNumWs, "workspace kind %d", kind);
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_mu);
    Ws& w = g_ws[std::make_tuple(kind, dev, st)];
    if (w.bytes >= bytes) return w.p;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIP_CHECK(hipStreamIsCapturing(st, &cs));
    if (cs != hipStreamCaptureStatusNone) return nullptr;
    void* np = nullptr;
    HIP_CHECK(hipMalloc(&np, bytes));
    if (kind == kWsDec) {  // counters start at zero (the kernel sets them back to zero at the end of every call)
        HIP_CHECK(hipMemsetAsync(np, 0, bytes, st));
        HIP_CHECK(hipStreamSynchronize(st));
    }
    if (w.p) g_retired.push_back(w.p);
    w.p = np;
    w.bytes = bytes;
    return np;
}

size_t dec_tail_ctr_bytes() { return ((size_t)qe_num_cus() * 4 + 255) / 256 * 256; }

char* dec_tail_ws(hipStream_t st) {
    return static_cast<char*>(stream_ws(kWsDec, dec_tail_ctr_bytes() + (size_t)qe_num_cus() * 2 * 32 * 64 * 4, st));
}

void stream_ws_reserve(int kind, size_t bytes, hipStream_t st) {
    if (bytes > 0) CHECK(stream_ws(kind, bytes, st) != nullptr, "workspace reserve: called during graph capture");
}

int stream_ws_count(int kind) {
    std::lock_guard<std::mutex> lk(g_mu);
    int c = 0;
    for (const auto& e : g_ws)
        if (std::get<0>(e.first) == kind && e.second.p) c++;
    return c;
}
