// Context, memory, timing and error reporting of the anvil_mi355x C ABI.
#include <cstdarg>
#include <cstdlib>
#include <cstring>

#include "common.h"

namespace anvil {

static thread_local std::string g_last_error;
__thread KernelTimer g_timer;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return set_error(ANVIL_E_RUNTIME, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

int check_ctx(anvil_ctx* ctx) {
  if (!ctx) return set_error(ANVIL_E_VALUE, "null context");
  ANVIL_HIP(hipSetDevice(ctx->device));
  return ANVIL_OK;
}

__global__ void zero_kernel(uint8_t* __restrict__ p, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  // 16-byte body on an aligned pointer, byte head/tail otherwise
  if (((uintptr_t)p & 15) == 0) {
    size_t n16 = n / 16;
    uint4 z = {0, 0, 0, 0};
    for (size_t j = i; j < n16; j += stride) reinterpret_cast<uint4*>(p)[j] = z;
    for (size_t j = n16 * 16 + i; j < n; j += stride) p[j] = 0;
  } else {
    for (size_t j = i; j < n; j += stride) p[j] = 0;
  }
}

int zero_fill(hipStream_t s, void* dst, size_t bytes) {
  size_t blocks = (bytes / 16 + 255) / 256;
  blocks = blocks < 1 ? 1 : (blocks > 4096 ? 4096 : blocks);
  ANVIL_LAUNCH(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, s, (uint8_t*)dst, bytes);
  ANVIL_LAUNCHED();
  return ANVIL_OK;
}

}  // namespace anvil

using namespace anvil;

extern "C" {

const char* anvil_last_error(void) { return g_last_error.c_str(); }

int anvil_version(void) { return 1; }

int anvil_init(int device, anvil_ctx** out) {
  if (!out) return set_error(ANVIL_E_VALUE, "anvil_init: null output pointer");
  *out = nullptr;
  int n = 0;
  ANVIL_HIP(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return set_error(ANVIL_E_VALUE, "anvil_init: device %d of %d", device, n);
  ANVIL_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  ANVIL_HIP(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return set_error(ANVIL_E_RUNTIME, "anvil_init: device %d is %s, this library is built for gfx950", device,
                     prop.gcnArchName);
  anvil_ctx* c = new anvil_ctx();
  c->device = device;
  c->num_cu = prop.multiProcessorCount;
  if (const char* cfg = std::getenv("ANVIL_GEMM_CFG")) c->gemm_cfg = std::atoi(cfg);
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipMalloc(&c->flags, 256);
  if (e == hipSuccess) e = hipMemset(c->flags, 0, 256);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    anvil_destroy(c);
    return hip_fail(e, "anvil_init");
  }
  if (int r = gemm_scratch_setup(device)) {
    anvil_destroy(c);
    return r;
  }
  *out = c;
  return ANVIL_OK;
}

int anvil_destroy(anvil_ctx* ctx) {
  if (!ctx) return ANVIL_OK;
  if (g_timer.stream == ctx->stream) g_timer = KernelTimer{};
  hipSetDevice(ctx->device);
  if (ctx->stream) hipStreamSynchronize(ctx->stream);
  gemm_scratch_release(ctx);
  for (auto& ev : ctx->events)
    if (ev) hipEventDestroy(ev);
  if (ctx->flags) hipFree(ctx->flags);
  if (ctx->ws) hipFree(ctx->ws);
  for (int* w : ctx->ws_retired) hipFree(w);
  if (ctx->stream) hipStreamDestroy(ctx->stream);
  delete ctx;
  return ANVIL_OK;
}

int anvil_sync(anvil_ctx* ctx) {
  if (int r = check_ctx(ctx)) return r;
  ANVIL_HIP(hipStreamSynchronize(ctx->stream));
  unsigned flags = 0;
  ANVIL_HIP(hipMemcpy(&flags, ctx->flags, sizeof flags, hipMemcpyDeviceToHost));
  if (!flags) return ANVIL_OK;
  ANVIL_HIP(hipMemset(ctx->flags, 0, sizeof(unsigned)));
  if (flags & FLAG_OVERFLOW) return set_error(ANVIL_E_OVERFLOW, "an int32 intermediate overflowed on the device");
  if (flags & FLAG_ZERODIV) return set_error(ANVIL_E_ZERODIV, "a softmax row summed to zero");
  if (flags & FLAG_SHIFT) return set_error(ANVIL_E_VALUE, "an rmsnorm shift s + k left [0, 31]");
  if (flags & FLAG_NONFINITE) return set_error(ANVIL_E_VALUE, "a float input holds NaN or infinite values");
  return set_error(ANVIL_E_VALUE, "an operand left its dtype range on the device (flags %u)", flags);
}

int anvil_alloc(anvil_ctx* ctx, size_t bytes, void** dptr) {
  if (int r = check_ctx(ctx)) return r;
  if (!dptr) return set_error(ANVIL_E_VALUE, "anvil_alloc: null output pointer");
  *dptr = nullptr;
  ANVIL_HIP(hipMalloc(dptr, bytes ? bytes : 1));
  return ANVIL_OK;
}

int anvil_free(anvil_ctx* ctx, void* dptr) {
  if (int r = check_ctx(ctx)) return r;
  if (!dptr) return ANVIL_OK;
  ANVIL_HIP(hipStreamSynchronize(ctx->stream));
  ANVIL_HIP(hipFree(dptr));
  return ANVIL_OK;
}

int anvil_host_alloc(anvil_ctx* ctx, size_t bytes, void** hptr) {
  if (int r = check_ctx(ctx)) return r;
  if (!hptr) return set_error(ANVIL_E_VALUE, "anvil_host_alloc: null output pointer");
  *hptr = nullptr;
  ANVIL_HIP(hipHostMalloc(hptr, bytes ? bytes : 1, hipHostMallocDefault));
  return ANVIL_OK;
}

int anvil_host_free(anvil_ctx* ctx, void* hptr) {
  if (int r = check_ctx(ctx)) return r;
  if (!hptr) return ANVIL_OK;
  ANVIL_HIP(hipStreamSynchronize(ctx->stream));
  ANVIL_HIP(hipHostFree(hptr));
  return ANVIL_OK;
}

int anvil_upload(anvil_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (int r = check_ctx(ctx)) return r;
  if (!bytes) return ANVIL_OK;
  if (!dst || !src) return set_error(ANVIL_E_VALUE, "anvil_upload: null pointer");
  ANVIL_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  ANVIL_HIP(hipStreamSynchronize(ctx->stream));
  return ANVIL_OK;
}

int anvil_download(anvil_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (int r = check_ctx(ctx)) return r;
  if (!bytes) return ANVIL_OK;
  if (!dst || !src) return set_error(ANVIL_E_VALUE, "anvil_download: null pointer");
  ANVIL_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  ANVIL_HIP(hipStreamSynchronize(ctx->stream));
  return ANVIL_OK;
}

int anvil_zero(anvil_ctx* ctx, void* dst, size_t bytes) {
  if (int r = check_ctx(ctx)) return r;
  if (!bytes) return ANVIL_OK;
  if (!dst) return set_error(ANVIL_E_VALUE, "anvil_zero: null pointer");
  return zero_fill(ctx->stream, dst, bytes);
}

int anvil_graph_begin(anvil_ctx* ctx) {
  if (int r = check_ctx(ctx)) return r;
  ANVIL_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed));
  return ANVIL_OK;
}

int anvil_graph_end(anvil_ctx* ctx, void** graph) {
  if (int r = check_ctx(ctx)) return r;
  if (!graph) return set_error(ANVIL_E_VALUE, "anvil_graph_end: null output pointer");
  *graph = nullptr;
  hipGraph_t g = nullptr;
  ANVIL_HIP(hipStreamEndCapture(ctx->stream, &g));       // ends the capture whatever happened inside it
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  if (e != hipSuccess) return ::anvil::hip_fail(e, "hipGraphInstantiate");
  *graph = exec;
  return ANVIL_OK;
}

int anvil_graph_launch(anvil_ctx* ctx, void* graph) {
  if (int r = check_ctx(ctx)) return r;
  if (!graph) return set_error(ANVIL_E_VALUE, "anvil_graph_launch: null graph");
  ANVIL_HIP(hipGraphLaunch((hipGraphExec_t)graph, ctx->stream));
  return ANVIL_OK;
}

int anvil_graph_destroy(anvil_ctx* ctx, void* graph) {
  if (int r = check_ctx(ctx)) return r;
  if (!graph) return ANVIL_OK;
  ANVIL_HIP(hipStreamSynchronize(ctx->stream));
  ANVIL_HIP(hipGraphExecDestroy((hipGraphExec_t)graph));
  return ANVIL_OK;
}

// The context's events only time work (anvil_event_elapsed, anvil_time_kernels); nothing reads device memory through
// them, so they are created without the system-scope release / acquire fence: recording one then costs no L2
// writeback and invalidation, which would also slow the next kernel.
static int ensure_event(anvil_ctx* ctx, int slot) {
  if (!ctx->events[slot]) ANVIL_HIP(hipEventCreateWithFlags(&ctx->events[slot], hipEventDisableSystemFence));
  return ANVIL_OK;
}

int anvil_event_record(anvil_ctx* ctx, int slot) {
  if (slot < 0 || slot >= EVENT_SLOTS)
    return set_error(ANVIL_E_VALUE, "event slot %d outside [0, %d)", slot, EVENT_SLOTS);
  if (int r = check_ctx(ctx)) return r;
  if (int r = ensure_event(ctx, slot)) return r;
  ANVIL_HIP(hipEventRecord(ctx->events[slot], ctx->stream));
  return ANVIL_OK;
}

int anvil_time_kernels(anvil_ctx* ctx, int slot0, int slot1) {
  if (int r = check_ctx(ctx)) return r;
  if (slot0 < 0 && slot1 < 0) {
    if (g_timer.stream == ctx->stream) g_timer = KernelTimer{};
    return ANVIL_OK;
  }
  if (slot0 < 0 || slot0 >= EVENT_SLOTS || slot1 < 0 || slot1 >= EVENT_SLOTS || slot0 == slot1)
    return set_error(ANVIL_E_VALUE, "anvil_time_kernels: slots %d, %d must be two distinct slots in [0, %d)", slot0,
                     slot1, EVENT_SLOTS);
  for (int s : {slot0, slot1})
    if (int r = ensure_event(ctx, s)) return r;
  g_timer = KernelTimer{ctx->stream, ctx->events[slot0], ctx->events[slot1]};
  return ANVIL_OK;
}

int anvil_event_elapsed(anvil_ctx* ctx, int slot0, int slot1, float* ms) {
  if (slot0 < 0 || slot0 >= EVENT_SLOTS || slot1 < 0 || slot1 >= EVENT_SLOTS || !ms)
    return set_error(ANVIL_E_VALUE, "anvil_event_elapsed: bad slot or null output");
  if (int r = check_ctx(ctx)) return r;
  if (!ctx->events[slot0] || !ctx->events[slot1])
    return set_error(ANVIL_E_VALUE, "anvil_event_elapsed: slot never recorded");
  ANVIL_HIP(hipEventSynchronize(ctx->events[slot1]));
  ANVIL_HIP(hipEventElapsedTime(ms, ctx->events[slot0], ctx->events[slot1]));
  return ANVIL_OK;
}

}  // extern "C"
