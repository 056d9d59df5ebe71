// runtime.hip -- error state, device memory, streams and events of the C ABI.
#include "hip_common.h"

#include <map>
#include <mutex>
#include <utility>
#include <vector>

namespace cactus_hip {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
    set_error(msg);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(CACTUS_HIP_ERUNTIME, std::string(what) + ": " + hipGetErrorString(e));
    return CACTUS_HIP_OK;
}

// Byte fill as a kernel (no hipMemsetAsync node, so it is safe to capture
// into a HIP graph and replay).
__global__ void fill_bytes_kernel(uint8_t* dst, uint32_t word, size_t bytes) {
    const size_t nw = bytes / 4;
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    if (((uintptr_t)dst & 3) == 0) {
        uint32_t* d = reinterpret_cast<uint32_t*>(dst);
        for (size_t i = tid; i < nw; i += stride) d[i] = word;
        for (size_t i = nw * 4 + tid; i < bytes; i += stride) dst[i] = (uint8_t)word;
    } else {
        for (size_t i = tid; i < bytes; i += stride) dst[i] = (uint8_t)word;
    }
}

// ------------------------------------------------ per-stream scratch
namespace {
struct ScratchBuf {
    void* ptr = nullptr;
    size_t bytes = 0;
    bool captured = false;   // handed out during a graph capture
};
struct Retired {
    void* ptr;
    hipEvent_t done;         // null: kept until the stream is destroyed
};
struct StreamScratch {
    ScratchBuf cur[SCR_KINDS];
    std::vector<Retired> retired;
};
std::mutex g_scr_mu;
std::map<std::pair<int, void*>, StreamScratch> g_scr;

// frees the retired buffers whose stream work has finished
void reap(StreamScratch& S) {
    size_t keep = 0;
    for (size_t i = 0; i < S.retired.size(); i++) {
        Retired& r = S.retired[i];
        if (r.done && hipEventQuery(r.done) == hipSuccess) {
            (void)hipFree(r.ptr);
            (void)hipEventDestroy(r.done);
        } else {
            S.retired[keep++] = r;
        }
    }
    S.retired.resize(keep);
}
}  // namespace

int stream_scratch(int kind, void* stream, size_t bytes, bool zero, void** out) {
    CH_REQUIRE(kind >= 0 && kind < SCR_KINDS && out, "scratch: bad request");
    int dev = 0;
    CH_HIP(hipGetDevice(&dev));
    const hipStream_t st = as_stream(stream);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (st) CH_HIP(hipStreamIsCapturing(st, &cs));
    const bool capturing = cs == hipStreamCaptureStatusActive;
    std::lock_guard<std::mutex> lk(g_scr_mu);
    StreamScratch& S = g_scr[std::make_pair(dev, stream)];
    reap(S);
    ScratchBuf& b = S.cur[kind];
    if (b.bytes < bytes || !b.ptr) {
        const size_t want = (bytes + bytes / 4 + 255) & ~(size_t)255;
        void* p = nullptr;
        CH_HIP(hipMalloc(&p, want ? want : 256));
        if (b.ptr) {
            Retired r{b.ptr, nullptr};
            if (!b.captured && !capturing) {
                // work queued before this point may still read the old buffer
                hipEvent_t e = nullptr;
                if (hipEventCreateWithFlags(&e, hipEventDisableTiming) == hipSuccess) {
                    if (hipEventRecord(e, st) == hipSuccess) r.done = e;
                    else (void)hipEventDestroy(e);
                }
            }
            S.retired.push_back(r);
        }
        b.ptr = p;
        b.bytes = want ? want : 256;
        b.captured = false;
        if (zero) {
            size_t blocks = (b.bytes / 4 + 255) / 256;
            if (blocks > 4096) blocks = 4096;
            hipLaunchKernelGGL(fill_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (uint8_t*)p, 0u,
                               b.bytes);
            int rc = check_launch("scratch zero fill");
            if (rc) return rc;
        }
    }
    if (capturing) b.captured = true;
    *out = b.ptr;
    return CACTUS_HIP_OK;
}

int stream_scratch_release(void* stream) {
    std::lock_guard<std::mutex> lk(g_scr_mu);
    bool synced = false;
    for (auto it = g_scr.begin(); it != g_scr.end();) {
        if (it->first.second != stream) {
            ++it;
            continue;
        }
        if (!synced) {
            CH_HIP(hipStreamSynchronize(as_stream(stream)));
            synced = true;
        }
        StreamScratch& S = it->second;
        for (ScratchBuf& b : S.cur)
            if (b.ptr) (void)hipFree(b.ptr);
        for (Retired& r : S.retired) {
            (void)hipFree(r.ptr);
            if (r.done) (void)hipEventDestroy(r.done);
        }
        it = g_scr.erase(it);
    }
    return CACTUS_HIP_OK;
}

}  // namespace cactus_hip

using namespace cactus_hip;

extern "C" {

const char* cactus_hip_last_error(void) { return g_last_error.c_str(); }

int cactus_hip_init(int device) {
    int n = 0;
    CH_HIP(hipGetDeviceCount(&n));
    CH_REQUIRE(device >= 0 && device < n, "cactus_hip_init: no such device");
    CH_HIP(hipSetDevice(device));
    return CACTUS_HIP_OK;
}

int cactus_hip_device_count(int* count) {
    CH_REQUIRE(count, "cactus_hip_device_count: null");
    hipError_t e = hipGetDeviceCount(count);
    if (e != hipSuccess) { *count = 0; }
    return CACTUS_HIP_OK;
}

int cactus_hip_device_memory(size_t* free_bytes, size_t* total_bytes) {
    CH_REQUIRE(free_bytes && total_bytes, "cactus_hip_device_memory: null");
    CH_HIP(hipMemGetInfo(free_bytes, total_bytes));
    return CACTUS_HIP_OK;
}

int cactus_hip_malloc(void** ptr, size_t bytes) {
    CH_REQUIRE(ptr, "cactus_hip_malloc: null out pointer");
    *ptr = nullptr;
    if (bytes == 0) return CACTUS_HIP_OK;
    hipError_t e = hipMalloc(ptr, bytes);
    if (e != hipSuccess) return fail(CACTUS_HIP_ENOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
    return CACTUS_HIP_OK;
}

int cactus_hip_free(void* ptr) {
    if (ptr) CH_HIP(hipFree(ptr));
    return CACTUS_HIP_OK;
}

int cactus_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(dst && src, "memcpy_h2d: null pointer");
    CH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
    CH_HIP(hipStreamSynchronize(as_stream(stream)));
    return CACTUS_HIP_OK;
}

int cactus_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(dst && src, "memcpy_d2h: null pointer");
    CH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
    CH_HIP(hipStreamSynchronize(as_stream(stream)));
    return CACTUS_HIP_OK;
}

int cactus_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(dst && src, "memcpy_d2d: null pointer");
    CH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
    return CACTUS_HIP_OK;
}

int cactus_hip_memset(void* dst, int byte_value, size_t bytes, void* stream) {
    if (bytes == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(dst, "memset: null pointer");
    const uint32_t b = (uint32_t)(byte_value & 0xFF);
    const uint32_t word = b | (b << 8) | (b << 16) | (b << 24);
    size_t blocks = (bytes / 4 + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fill_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                       (uint8_t*)dst, word, bytes);
    return check_launch("memset");
}

int cactus_hip_stream_create(void** stream) {
    CH_REQUIRE(stream, "stream_create: null");
    hipStream_t s;
    CH_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return CACTUS_HIP_OK;
}

int cactus_hip_stream_destroy(void* stream) {
    if (!stream) return CACTUS_HIP_OK;
    // the library's scratch buffers of the stream go with it
    int rc = stream_scratch_release(stream);
    if (rc) return rc;
    CH_HIP(hipStreamDestroy(as_stream(stream)));
    return CACTUS_HIP_OK;
}

int cactus_hip_stream_sync(void* stream) {
    CH_HIP(hipStreamSynchronize(as_stream(stream)));
    return CACTUS_HIP_OK;
}

int cactus_hip_event_create(void** event) {
    CH_REQUIRE(event, "event_create: null");
    hipEvent_t e;
    CH_HIP(hipEventCreate(&e));
    *event = e;
    return CACTUS_HIP_OK;
}

int cactus_hip_event_destroy(void* event) {
    if (event) CH_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
    return CACTUS_HIP_OK;
}

int cactus_hip_event_record(void* event, void* stream) {
    CH_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream)));
    return CACTUS_HIP_OK;
}

int cactus_hip_stream_wait_event(void* stream, void* event) {
    CH_REQUIRE(event, "stream_wait_event: null event");
    CH_HIP(hipStreamWaitEvent(as_stream(stream), reinterpret_cast<hipEvent_t>(event), 0));
    return CACTUS_HIP_OK;
}

int cactus_hip_event_elapsed_ms(void* start, void* end, float* ms) {
    CH_REQUIRE(ms, "event_elapsed_ms: null");
    CH_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(end)));
    CH_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                               reinterpret_cast<hipEvent_t>(end)));
    return CACTUS_HIP_OK;
}

int cactus_hip_graph_capture_begin(void* stream) {
    CH_REQUIRE(stream, "graph capture needs a non-default stream");
    CH_HIP(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal));
    return CACTUS_HIP_OK;
}

int cactus_hip_graph_capture_end(void* stream, void** graph_exec) {
    CH_REQUIRE(graph_exec, "graph_capture_end: null out pointer");
    hipGraph_t g = nullptr;
    CH_HIP(hipStreamEndCapture(as_stream(stream), &g));
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return fail(CACTUS_HIP_ERUNTIME, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    *graph_exec = ge;
    return CACTUS_HIP_OK;
}

int cactus_hip_graph_launch(void* graph_exec, void* stream) {
    CH_HIP(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph_exec), as_stream(stream)));
    return CACTUS_HIP_OK;
}

int cactus_hip_graph_destroy(void* graph_exec) {
    if (graph_exec) CH_HIP(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph_exec)));
    return CACTUS_HIP_OK;
}

}  // extern "C"
