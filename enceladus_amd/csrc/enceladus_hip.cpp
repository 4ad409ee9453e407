// libenceladus_hip.so: the C-ABI runtime shim over HIP and hiprtc for gfx950.
// Declarations and the reference interfaces they replace: include/enceladus_hip.h.
#include "../../include/enceladus_hip.h"

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

// The HIP runtime's launch with dispatch-boundary events (declared in hip/hip_ext.h, whose
// kernel-launch templates need the HIP compiler; this file is host code built by g++).
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX,
                                               uint32_t globalWorkSizeY, uint32_t globalWorkSizeZ,
                                               uint32_t localWorkSizeX, uint32_t localWorkSizeY,
                                               uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                               hipStream_t hStream, void** kernelParams,
                                               void** extra, hipEvent_t startEvent,
                                               hipEvent_t stopEvent, uint32_t flags);

namespace {

int fail(char* err, size_t errlen, const std::string& msg) {
  if (err && errlen) {
    std::snprintf(err, errlen, "%s", msg.c_str());
  }
  return 1;
}

int check(hipError_t e, const char* what, char* err, size_t errlen) {
  if (e == hipSuccess) return 0;
  std::string msg = std::string(what) + ": " + hipGetErrorName(e) + " (" +
                    hipGetErrorString(e) + ")";
  return fail(err, errlen, msg);
}

#define EK_CHECK(call) \
  do { if (int _rc = check((call), #call, err, errlen)) return _rc; } while (0)

}  // namespace

extern "C" {

const char* ek_version(void) { return "enceladus_hip 0.1 (gfx950)"; }

int ek_runtime_version(int* version) {
  return hipRuntimeGetVersion(version) == hipSuccess ? 0 : 1;
}

int ek_device_count(int* count, char* err, size_t errlen) {
  EK_CHECK(hipGetDeviceCount(count));
  return 0;
}

int ek_set_device(int device, char* err, size_t errlen) {
  EK_CHECK(hipSetDevice(device));
  return 0;
}

int ek_device_get_info(int device, ek_device_info* out, char* err, size_t errlen) {
  hipDeviceProp_t p;
  EK_CHECK(hipGetDeviceProperties(&p, device));
  std::memset(out, 0, sizeof(*out));
  std::snprintf(out->name, sizeof(out->name), "%s", p.name);
  std::snprintf(out->arch, sizeof(out->arch), "%s", p.gcnArchName);
  out->compute_units = p.multiProcessorCount;
  out->warp_size = p.warpSize;
  out->max_threads_per_block = p.maxThreadsPerBlock;
  out->lds_per_block = (int64_t)p.sharedMemPerBlock;
  out->total_mem = (int64_t)p.totalGlobalMem;
  out->clock_khz = p.clockRate;
  out->mem_clock_khz = p.memoryClockRate;
  out->mem_bus_width = p.memoryBusWidth;
  out->l2_bytes = p.l2CacheSize;
  return 0;
}

int ek_compile(const char* source, const char* name, const char* const* options,
               int num_options, void** code, size_t* code_size, char* log, size_t loglen) {
  *code = nullptr;
  *code_size = 0;
  if (log && loglen) log[0] = 0;
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, source, name, 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS) {
    return fail(log, loglen, std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(r));
  }
  r = hiprtcCompileProgram(prog, num_options, const_cast<const char**>(options));
  size_t n = 0;
  hiprtcGetProgramLogSize(prog, &n);
  std::string text;
  if (n > 1) {
    text.resize(n);
    hiprtcGetProgramLog(prog, &text[0]);
  }
  if (r != HIPRTC_SUCCESS) {
    fail(log, loglen, std::string("hiprtcCompileProgram: ") + hiprtcGetErrorString(r) +
                          "\n" + text);
    hiprtcDestroyProgram(&prog);
    return 1;
  }
  if (log && loglen && !text.empty()) std::snprintf(log, loglen, "%s", text.c_str());
  size_t sz = 0;
  r = hiprtcGetCodeSize(prog, &sz);
  if (r != HIPRTC_SUCCESS || sz == 0) {
    hiprtcDestroyProgram(&prog);
    return fail(log, loglen, "hiprtcGetCodeSize failed");
  }
  void* buf = std::malloc(sz);
  r = hiprtcGetCode(prog, static_cast<char*>(buf));
  hiprtcDestroyProgram(&prog);
  if (r != HIPRTC_SUCCESS) {
    std::free(buf);
    return fail(log, loglen, "hiprtcGetCode failed");
  }
  *code = buf;
  *code_size = sz;
  return 0;
}

void ek_buffer_free(void* p) { std::free(p); }

int ek_module_load(const void* code, size_t code_size, void** module, char* err,
                   size_t errlen) {
  (void)code_size;
  hipModule_t m;
  EK_CHECK(hipModuleLoadData(&m, code));
  *module = m;
  return 0;
}

int ek_module_unload(void* module, char* err, size_t errlen) {
  EK_CHECK(hipModuleUnload(static_cast<hipModule_t>(module)));
  return 0;
}

int ek_module_function(void* module, const char* name, void** function, char* err,
                       size_t errlen) {
  hipFunction_t f;
  EK_CHECK(hipModuleGetFunction(&f, static_cast<hipModule_t>(module), name));
  *function = f;
  return 0;
}

int ek_function_get_attrs(void* function, ek_function_attrs* out, char* err,
                          size_t errlen) {
  hipFunction_t f = static_cast<hipFunction_t>(function);
  int v = 0;
  std::memset(out, 0, sizeof(*out));
  EK_CHECK(hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_NUM_REGS, f));
  out->num_regs = v;
  EK_CHECK(hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, f));
  out->shared_bytes = v;
  EK_CHECK(hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_LOCAL_SIZE_BYTES, f));
  out->local_bytes = v;
  EK_CHECK(hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, f));
  out->max_threads = v;
  return 0;
}

int ek_launch(void* stream, void* function, uint32_t gx, uint32_t gy, uint32_t gz,
              uint32_t bx, uint32_t by, uint32_t bz, uint32_t dyn_lds, void* kernarg,
              size_t kernarg_size, char* err, size_t errlen) {
  size_t size = kernarg_size;
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, kernarg, HIP_LAUNCH_PARAM_BUFFER_SIZE,
                    &size, HIP_LAUNCH_PARAM_END};
  EK_CHECK(hipModuleLaunchKernel(static_cast<hipFunction_t>(function), gx, gy, gz, bx, by,
                                 bz, dyn_lds, static_cast<hipStream_t>(stream), nullptr,
                                 config));
  return 0;
}

int ek_launch_timed_events(void* stream, void* function, uint32_t gx, uint32_t gy,
                           uint32_t gz, uint32_t bx, uint32_t by, uint32_t bz,
                           uint32_t dyn_lds, void* kernarg, size_t kernarg_size,
                           void* start_event, void* stop_event, char* err, size_t errlen) {
  const uint64_t tx = (uint64_t)gx * bx, ty = (uint64_t)gy * by, tz = (uint64_t)gz * bz;
  if (tx > 0xFFFFFFFFull || ty > 0xFFFFFFFFull || tz > 0xFFFFFFFFull) {
    return fail(err, errlen, "ek_launch_timed_events: more than 2^32 threads along one "
                             "dimension; time this launch with ek_event_record instead");
  }
  size_t size = kernarg_size;
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, kernarg, HIP_LAUNCH_PARAM_BUFFER_SIZE,
                    &size, HIP_LAUNCH_PARAM_END};
  EK_CHECK(hipExtModuleLaunchKernel(static_cast<hipFunction_t>(function), (uint32_t)tx,
                                    (uint32_t)ty, (uint32_t)tz, bx, by, bz, dyn_lds,
                                    static_cast<hipStream_t>(stream), nullptr, config,
                                    static_cast<hipEvent_t>(start_event),
                                    static_cast<hipEvent_t>(stop_event), 0));
  return 0;
}

int ek_stream_new(void** stream, char* err, size_t errlen) {
  hipStream_t s;
  EK_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return 0;
}

int ek_stream_free(void* stream, char* err, size_t errlen) {
  EK_CHECK(hipStreamDestroy(static_cast<hipStream_t>(stream)));
  return 0;
}

int ek_stream_sync(void* stream, char* err, size_t errlen) {
  EK_CHECK(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  EK_CHECK(hipGetLastError());
  return 0;
}

int ek_device_sync(char* err, size_t errlen) {
  EK_CHECK(hipDeviceSynchronize());
  return 0;
}

int ek_malloc(void** ptr, size_t bytes, char* err, size_t errlen) {
  EK_CHECK(hipMalloc(ptr, bytes ? bytes : 16));
  return 0;
}

int ek_free(void* ptr, char* err, size_t errlen) {
  EK_CHECK(hipFree(ptr));
  return 0;
}

int ek_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream, char* err,
                  size_t errlen) {
  EK_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice,
                          static_cast<hipStream_t>(stream)));
  EK_CHECK(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  return 0;
}

int ek_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream, char* err,
                  size_t errlen) {
  EK_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost,
                          static_cast<hipStream_t>(stream)));
  EK_CHECK(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  return 0;
}

int ek_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream, char* err,
                  size_t errlen) {
  EK_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice,
                          static_cast<hipStream_t>(stream)));
  return 0;
}

int ek_memset(void* dst, int value, size_t bytes, void* stream, char* err, size_t errlen) {
  EK_CHECK(hipMemsetAsync(dst, value, bytes, static_cast<hipStream_t>(stream)));
  return 0;
}

int ek_event_new(void** event, char* err, size_t errlen) {
  hipEvent_t e;
  EK_CHECK(hipEventCreate(&e));
  *event = e;
  return 0;
}

int ek_event_free(void* event, char* err, size_t errlen) {
  EK_CHECK(hipEventDestroy(static_cast<hipEvent_t>(event)));
  return 0;
}

int ek_event_record(void* event, void* stream, char* err, size_t errlen) {
  EK_CHECK(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)));
  return 0;
}

int ek_event_elapsed_ms(void* start, void* stop, float* ms, char* err, size_t errlen) {
  EK_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
  EK_CHECK(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                               static_cast<hipEvent_t>(stop)));
  return 0;
}

int ek_timed_launch(void* stream, void* function, uint32_t gx, uint32_t gy, uint32_t gz,
                    uint32_t bx, uint32_t by, uint32_t bz, uint32_t dyn_lds, void* kernarg,
                    size_t kernarg_size, int reps, float* ms_per_launch, char* err,
                    size_t errlen) {
  hipEvent_t a, b;
  EK_CHECK(hipEventCreate(&a));
  EK_CHECK(hipEventCreate(&b));
  hipStream_t s = static_cast<hipStream_t>(stream);
  EK_CHECK(hipEventRecord(a, s));
  for (int i = 0; i < reps; ++i) {
    if (int rc = ek_launch(stream, function, gx, gy, gz, bx, by, bz, dyn_lds, kernarg,
                           kernarg_size, err, errlen)) {
      (void)hipEventDestroy(a);
      (void)hipEventDestroy(b);
      return rc;
    }
  }
  EK_CHECK(hipEventRecord(b, s));
  EK_CHECK(hipEventSynchronize(b));
  float ms = 0;
  EK_CHECK(hipEventElapsedTime(&ms, a, b));
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  *ms_per_launch = reps > 0 ? ms / reps : 0.0f;
  return 0;
}

}  // extern "C"
