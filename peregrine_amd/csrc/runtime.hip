// Runtime half of the C ABI: device, memory, streams, events, errors.
// Replaces the Objective-C Metal bridge (reference: src/runtime/bridge.m:1-389,
// declared in src/runtime/bridge.h:23-97). Metal's shared/private buffers map
// to pinned host / device allocations; a command buffer maps to work queued on
// a HIP stream; commit+wait maps to a stream synchronise.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "attention.hpp"
#include "common.hpp"

namespace prg {

static thread_local char g_last_error[512] = {0};

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace prg

using prg::set_error;

namespace {
// Plain streaming copy (16 B per thread per step): the calibration reference
// for HBM byte counters (FETCH_SIZE / WRITE_SIZE per dispatch).
__global__ void copy_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n16) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    dst[i] = src[i];
}
// Streaming read: a grid-stride loop of non-temporal 16-byte loads, one per
// thread per pass, folded into a value that is stored only if it hits an
// impossible pattern, so the loads stay live. One word of *sink is written at
// most. Of the configurations measured on MI355X (1024-4096 blocks of 256
// threads, 1-4 loads in flight per thread), 2048 blocks with one load in
// flight read 9.45 / 28.3 / 56.7 MB fastest (2.88 / 5.79 / 9.9 us per
// graph-replayed launch); the launcher uses that grid.
__global__ __launch_bounds__(256) void read_kernel(const prg::u32x4* __restrict__ src, size_t n16,
                                                   uint32_t* __restrict__ sink) {
  const size_t T = static_cast<size_t>(gridDim.x) * blockDim.x;
  uint32_t acc = 0;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += T) {
    const prg::u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v[0] ^ v[3];
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}
}  // namespace

extern "C" {

int prg_hip_read_kernel(const void* src, size_t bytes, uint32_t* sink, void* stream) {
  PRG_CHECK_ARG(src && sink, "prg_hip_read_kernel: null pointer");
  PRG_CHECK_ARG(bytes % 16 == 0, "prg_hip_read_kernel: bytes %zu not a multiple of 16", bytes);
  hipLaunchKernelGGL(read_kernel, dim3(2048), dim3(256), 0, prg::as_stream(stream),
                     static_cast<const prg::u32x4*>(src), bytes / 16, sink);
  PRG_CHECK_LAUNCH("prg_hip_read_kernel");
  return PRG_OK;
}

int prg_hip_copy_kernel(void* dst, const void* src, size_t bytes, void* stream) {
  PRG_CHECK_ARG(dst && src, "prg_hip_copy_kernel: null pointer");
  PRG_CHECK_ARG(bytes % 16 == 0, "prg_hip_copy_kernel: bytes %zu not a multiple of 16", bytes);
  const size_t n16 = bytes / 16;
  hipLaunchKernelGGL(copy_kernel, dim3(2048), dim3(256), 0, prg::as_stream(stream),
                     static_cast<const uint4*>(src), static_cast<uint4*>(dst), n16);
  PRG_CHECK_LAUNCH("prg_hip_copy_kernel");
  return PRG_OK;
}

const char* prg_last_error(void) { return prg::g_last_error; }

const char* prg_version(void) { return "peregrine_amd 0.1 gfx950"; }

int prg_hip_device_count(int* count) {
  PRG_CHECK_ARG(count != nullptr, "prg_hip_device_count: null count");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    *count = 0;
    return set_error(PRG_ERR_NO_DEVICE, "hipGetDeviceCount: %s", hipGetErrorString(e));
  }
  *count = n;
  return PRG_OK;
}

int prg_hip_device_init(int ordinal) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
    return set_error(PRG_ERR_NO_DEVICE, "no HIP device visible");
  PRG_CHECK_ARG(ordinal >= 0 && ordinal < n, "device ordinal %d out of range [0,%d)", ordinal, n);
  PRG_HIP(hipSetDevice(ordinal));
  return prg::attn_noalloc_setup();
}

int prg_hip_device_name(char* buf, size_t len) {
  PRG_CHECK_ARG(buf != nullptr && len > 0, "prg_hip_device_name: bad buffer");
  int dev = 0;
  PRG_HIP(hipGetDevice(&dev));
  hipDeviceProp_t p;
  PRG_HIP(hipGetDeviceProperties(&p, dev));
  snprintf(buf, len, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
  return PRG_OK;
}

int prg_hip_alloc_device(void** ptr, size_t bytes) {
  PRG_CHECK_ARG(ptr != nullptr, "prg_hip_alloc_device: null out pointer");
  *ptr = nullptr;
  if (bytes == 0) return PRG_OK;
  hipError_t e = hipMalloc(ptr, bytes);
  if (e != hipSuccess)
    return set_error(PRG_ERR_OOM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  return PRG_OK;
}

int prg_hip_free_device(void* ptr) {
  if (ptr == nullptr) return PRG_OK;
  PRG_HIP(hipFree(ptr));
  return PRG_OK;
}

int prg_hip_alloc_host(void** ptr, size_t bytes) {
  PRG_CHECK_ARG(ptr != nullptr, "prg_hip_alloc_host: null out pointer");
  *ptr = nullptr;
  if (bytes == 0) return PRG_OK;
  hipError_t e = hipHostMalloc(ptr, bytes, hipHostMallocDefault);
  if (e != hipSuccess)
    return set_error(PRG_ERR_OOM, "hipHostMalloc(%zu): %s", bytes, hipGetErrorString(e));
  return PRG_OK;
}

int prg_hip_free_host(void* ptr) {
  if (ptr == nullptr) return PRG_OK;
  PRG_HIP(hipHostFree(ptr));
  return PRG_OK;
}

int prg_hip_memcpy(void* dst, const void* src, size_t bytes, int kind, void* stream, int sync) {
  if (bytes == 0) return PRG_OK;
  PRG_CHECK_ARG(dst != nullptr && src != nullptr, "prg_hip_memcpy: null pointer");
  hipMemcpyKind k;
  switch (kind) {
    case 0: k = hipMemcpyHostToDevice; break;
    case 1: k = hipMemcpyDeviceToHost; break;
    case 2: k = hipMemcpyDeviceToDevice; break;
    default: return set_error(PRG_ERR_INVALID_ARG, "prg_hip_memcpy: bad kind %d", kind);
  }
  hipStream_t s = prg::as_stream(stream);
  PRG_HIP(hipMemcpyAsync(dst, src, bytes, k, s));
  if (sync) PRG_HIP(hipStreamSynchronize(s));
  return PRG_OK;
}

int prg_hip_memset_device(void* dst, int value, size_t bytes, void* stream) {
  if (bytes == 0) return PRG_OK;
  PRG_CHECK_ARG(dst != nullptr, "prg_hip_memset_device: null pointer");
  PRG_HIP(hipMemsetAsync(dst, value, bytes, prg::as_stream(stream)));
  return PRG_OK;
}

int prg_hip_stream_create(void** stream) {
  PRG_CHECK_ARG(stream != nullptr, "prg_hip_stream_create: null out pointer");
  hipStream_t s = nullptr;
  PRG_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return PRG_OK;
}

int prg_hip_stream_destroy(void* stream) {
  if (stream == nullptr) return PRG_OK;
  PRG_HIP(hipStreamDestroy(prg::as_stream(stream)));
  return PRG_OK;
}

int prg_hip_stream_synchronize(void* stream) {
  PRG_HIP(hipStreamSynchronize(prg::as_stream(stream)));
  return PRG_OK;
}

int prg_hip_device_synchronize(void) {
  PRG_HIP(hipDeviceSynchronize());
  return PRG_OK;
}

int prg_hip_event_create(void** event) {
  PRG_CHECK_ARG(event != nullptr, "prg_hip_event_create: null out pointer");
  hipEvent_t e = nullptr;
  PRG_HIP(hipEventCreate(&e));
  *event = e;
  return PRG_OK;
}

int prg_hip_event_destroy(void* event) {
  if (event == nullptr) return PRG_OK;
  PRG_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
  return PRG_OK;
}

int prg_hip_event_record(void* event, void* stream) {
  PRG_CHECK_ARG(event != nullptr, "prg_hip_event_record: null event");
  PRG_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(event), prg::as_stream(stream)));
  return PRG_OK;
}

int prg_hip_event_elapsed_ms(void* start, void* stop, float* ms) {
  PRG_CHECK_ARG(start && stop && ms, "prg_hip_event_elapsed_ms: null argument");
  PRG_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop)));
  PRG_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                              reinterpret_cast<hipEvent_t>(stop)));
  return PRG_OK;
}

// Command-sequence capture (bridge.h:60-97 command buffers -> HIP graphs).
int prg_hip_graph_begin(void* stream) {
  PRG_CHECK_ARG(stream, "prg_hip_graph_begin: capture needs a created stream, not the NULL stream");
  PRG_HIP(hipStreamBeginCapture(prg::as_stream(stream), hipStreamCaptureModeRelaxed));
  return PRG_OK;
}

int prg_hip_graph_end(void* stream, void** graph) {
  PRG_CHECK_ARG(stream && graph, "prg_hip_graph_end: null argument");
  hipGraph_t g = nullptr;
  PRG_HIP(hipStreamEndCapture(prg::as_stream(stream), &g));
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return prg::set_error(PRG_ERR_HIP, "prg_hip_graph_end: instantiate: %s", hipGetErrorString(e));
  *graph = exec;
  return PRG_OK;
}

int prg_hip_graph_launch(void* graph, void* stream) {
  PRG_CHECK_ARG(graph, "prg_hip_graph_launch: null graph");
  PRG_HIP(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph), prg::as_stream(stream)));
  return PRG_OK;
}

int prg_hip_graph_destroy(void* graph) {
  if (graph) PRG_HIP(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph)));
  return PRG_OK;
}

}  // extern "C"
