// Memory, stream, event and hipGraph entry points of the device C ABI.

#include "common.hpp"
#include "mlvc_hip_device.h"

#include <cstring>

namespace mlvc_hip {
namespace {
thread_local std::string g_error;
}
void set_error(const std::string& message) { g_error = message; }
}  // namespace mlvc_hip

using namespace mlvc_hip;

extern "C" {

const char* mlvc_hip_last_error(void) { return g_error.c_str(); }

int mlvc_hip_device_count(int* count)
{
    return guard([&] { check(hipGetDeviceCount(count), "hipGetDeviceCount"); });
}

int mlvc_hip_set_device(int device)
{
    return guard([&] { check(hipSetDevice(device), "hipSetDevice"); });
}

int mlvc_hip_device_name(int device, char* buf, size_t len)
{
    return guard([&] {
        hipDeviceProp_t p;
        check(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties");
        std::snprintf(buf, len, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    });
}

int mlvc_hip_malloc(void** ptr, size_t bytes)
{
    return guard([&] { check(hipMalloc(ptr, bytes ? bytes : 1), "hipMalloc"); });
}

int mlvc_hip_free(void* ptr)
{
    return guard([&] { if (ptr) check(hipFree(ptr), "hipFree"); });
}

int mlvc_hip_host_alloc(void** ptr, size_t bytes)
{
    return guard([&] { check(hipHostMalloc(ptr, bytes ? bytes : 1, hipHostMallocDefault), "hipHostMalloc"); });
}

int mlvc_hip_host_free(void* ptr)
{
    return guard([&] { if (ptr) check(hipHostFree(ptr), "hipHostFree"); });
}

int mlvc_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, mlvc_hip_stream s)
{
    return guard([&] { check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, to_stream(s)), "hipMemcpyAsync H2D"); });
}

int mlvc_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, mlvc_hip_stream s)
{
    return guard([&] { check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, to_stream(s)), "hipMemcpyAsync D2H"); });
}

int mlvc_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, mlvc_hip_stream s)
{
    return guard([&] { check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, to_stream(s)), "hipMemcpyAsync D2D"); });
}

int mlvc_hip_stream_create(mlvc_hip_stream* s)
{
    return guard([&] {
        hipStream_t st;
        check(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hipStreamCreateWithFlags");
        *s = reinterpret_cast<mlvc_hip_stream>(st);
    });
}

int mlvc_hip_stream_destroy(mlvc_hip_stream s)
{
    return guard([&] { if (s) check(hipStreamDestroy(to_stream(s)), "hipStreamDestroy"); });
}

int mlvc_hip_stream_synchronize(mlvc_hip_stream s)
{
    return guard([&] { check(hipStreamSynchronize(to_stream(s)), "hipStreamSynchronize"); });
}

int mlvc_hip_event_create(mlvc_hip_event* e)
{
    return guard([&] {
        hipEvent_t ev;
        check(hipEventCreate(&ev), "hipEventCreate");
        *e = reinterpret_cast<mlvc_hip_event>(ev);
    });
}

int mlvc_hip_event_destroy(mlvc_hip_event e)
{
    return guard([&] { if (e) check(hipEventDestroy(reinterpret_cast<hipEvent_t>(e)), "hipEventDestroy"); });
}

int mlvc_hip_event_record(mlvc_hip_event e, mlvc_hip_stream s)
{
    return guard([&] { check(hipEventRecord(reinterpret_cast<hipEvent_t>(e), to_stream(s)), "hipEventRecord"); });
}

int mlvc_hip_event_synchronize(mlvc_hip_event e)
{
    return guard([&] { check(hipEventSynchronize(reinterpret_cast<hipEvent_t>(e)), "hipEventSynchronize"); });
}

int mlvc_hip_event_elapsed_ms(mlvc_hip_event start, mlvc_hip_event stop, float* ms)
{
    return guard([&] {
        check(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop)),
              "hipEventElapsedTime");
    });
}

int mlvc_hip_capture_begin(mlvc_hip_stream s)
{
    return guard([&] { check(hipStreamBeginCapture(to_stream(s), hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture"); });
}

int mlvc_hip_capture_end(mlvc_hip_stream s, mlvc_hip_graph* graph)
{
    return guard([&] {
        hipGraph_t g = nullptr;
        check(hipStreamEndCapture(to_stream(s), &g), "hipStreamEndCapture");
        hipGraphExec_t exec = nullptr;
        const hipError_t err = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        check(err, "hipGraphInstantiate");
        *graph = reinterpret_cast<mlvc_hip_graph>(exec);
    });
}

int mlvc_hip_graph_launch(mlvc_hip_graph graph, mlvc_hip_stream s)
{
    return guard([&] { check(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph), to_stream(s)), "hipGraphLaunch"); });
}

int mlvc_hip_graph_destroy(mlvc_hip_graph graph)
{
    return guard([&] { if (graph) check(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph)), "hipGraphExecDestroy"); });
}

}  // extern "C"
