// The launch that allocates nothing: a privatised-bin kernel and its second flush level
// with their partial-result buffer in this library's static device array, for callers that
// cannot call hipMalloc (code under HIP graph capture, serving loops, harnesses that
// forbid allocation). Declaration and contract: include/enceladus_hip.h
// (ek_launch_flush_noalloc).
//
// Compiled by hipcc as HIP (the array lives in this file's device code object; there are
// no kernels here). The kernels themselves are the hiprtc-compiled ones the caller passes.
#include "../../include/enceladus_hip.h"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

// The scratch buffer: one copy per GPU, resident until the process ends. Host code never
// passes this name to a kernel (on the host it is only a stand-in for the symbol); it uses
// the per-device address from hipGetSymbolAddress below.
static __device__ __align__(256) unsigned char scratch[EK_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
constexpr size_t kMaxKernarg = 4096;

std::mutex g_mu;
void* g_scratch[kMaxDevices];  // device address of `scratch` on each device, once looked up

int fail(char* err, size_t errlen, const std::string& msg) {
  if (err && errlen) std::snprintf(err, errlen, "%s", msg.c_str());
  return 1;
}

int check(hipError_t e, const char* what, char* err, size_t errlen) {
  if (e == hipSuccess) return 0;
  return fail(err, errlen, std::string(what) + ": " + hipGetErrorName(e) + " (" +
                               hipGetErrorString(e) + ")");
}

#define EK_CHECK(call) \
  do { if (int _rc = check((call), #call, err, errlen)) return _rc; } while (0)

// The device address of `scratch` on the current device (looked up on the first call per
// device, with that device current).
int scratch_address(void** out, char* err, size_t errlen) {
  int dev = 0;
  EK_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) {
    return fail(err, errlen, "ek_launch_flush_noalloc: device index out of range");
  }
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    EK_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (p == nullptr) return fail(err, errlen, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return 0;
}

int launch(void* stream, void* function, uint32_t gx, uint32_t gy, uint32_t gz,
           uint32_t block, unsigned char* kernarg, size_t size, char* err, size_t errlen) {
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, kernarg, HIP_LAUNCH_PARAM_BUFFER_SIZE,
                    &size, HIP_LAUNCH_PARAM_END};
  EK_CHECK(hipModuleLaunchKernel(static_cast<hipFunction_t>(function), gx, gy, gz, block, 1,
                                 1, 0, static_cast<hipStream_t>(stream), nullptr, config));
  return 0;
}

}  // namespace

extern "C" int ek_launch_flush_noalloc(
    void* stream, void* function, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t block,
    const void* kernarg, size_t kernarg_size, size_t scratch_offset, void* flush_function,
    uint32_t fgx, uint32_t fgy, uint32_t fblock, const void* flush_kernarg,
    size_t flush_kernarg_size, size_t flush_scratch_offset, size_t scratch_bytes, char* err,
    size_t errlen) {
  if (scratch_bytes > EK_SCRATCH_BYTES) {
    return fail(err, errlen, "ek_launch_flush_noalloc: the launch needs " +
                                 std::to_string(scratch_bytes) + " bytes of scratch, above " +
                                 "the " + std::to_string((size_t)EK_SCRATCH_BYTES) +
                                 "-byte static buffer; use the allocating launch");
  }
  if (!function || !flush_function || !kernarg || !flush_kernarg) {
    return fail(err, errlen, "ek_launch_flush_noalloc: NULL function or kernarg");
  }
  if (kernarg_size > kMaxKernarg || flush_kernarg_size > kMaxKernarg ||
      scratch_offset % 8 || flush_scratch_offset % 8 ||
      scratch_offset + sizeof(void*) > kernarg_size ||
      flush_scratch_offset + sizeof(void*) > flush_kernarg_size) {
    return fail(err, errlen, "ek_launch_flush_noalloc: scratch pointer offset outside the "
                             "kernarg buffer (or a kernarg buffer above 4096 bytes)");
  }
  void* ptr = nullptr;
  if (int rc = scratch_address(&ptr, err, errlen)) return rc;
  unsigned char ka[kMaxKernarg], fa[kMaxKernarg];
  std::memcpy(ka, kernarg, kernarg_size);
  std::memcpy(ka + scratch_offset, &ptr, sizeof(ptr));
  std::memcpy(fa, flush_kernarg, flush_kernarg_size);
  std::memcpy(fa + flush_scratch_offset, &ptr, sizeof(ptr));
  if (int rc = launch(stream, function, gx, gy, gz, block, ka, kernarg_size, err, errlen)) {
    return rc;
  }
  return launch(stream, flush_function, fgx, fgy, 1, fblock, fa, flush_kernarg_size, err,
                errlen);
}
