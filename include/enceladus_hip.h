/*
 * enceladus_hip.h — the C ABI of the MI355X runtime shim (libenceladus_hip.so).
 *
 * It replaces the reference's Objective-C++ Metal runtime ABI (`fr_*`, reference
 * src/enceladus/_C/enceladus_rt.h:13-166). Conventions kept from it:
 *   - opaque handles, each with an explicit release;
 *   - 0 on success, non-zero on failure, with the error text written into a
 *     caller-provided buffer (`err`, `errlen`; the reference uses FR_ERR_LEN=65536);
 *   - plain pointers and sizes only, so any FFI (ctypes here) can bind it.
 * All functions are thread-safe: hiprtc programs are per call, and HIP streams are
 * internally synchronized.
 */
#ifndef ENCELADUS_HIP_H
#define ENCELADUS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EK_ERR_LEN 65536

/* Device query. Replaces fr_device_* (reference _C/enceladus_rt.mm:39-79). */
typedef struct ek_device_info {
  char name[256];
  char arch[64];            /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int32_t compute_units;
  int32_t warp_size;        /* 64 on CDNA */
  int32_t max_threads_per_block;
  int64_t lds_per_block;    /* bytes */
  int64_t total_mem;        /* bytes */
  int32_t clock_khz;
  int32_t mem_clock_khz;
  int32_t mem_bus_width;
  int32_t l2_bytes;
} ek_device_info;

int ek_device_count(int* count, char* err, size_t errlen);
int ek_device_get_info(int device, ek_device_info* out, char* err, size_t errlen);
int ek_set_device(int device, char* err, size_t errlen);

/* Runtime compile: HIP C++ source -> gfx950 code object via hiprtc.
 * Replaces fr_library_new (reference _C/enceladus_rt.mm:208-230).
 * On success *code is a malloc'd buffer of *code_size bytes (free with ek_buffer_free);
 * the hiprtc log (warnings or errors) is written into `log`. */
int ek_compile(const char* source, const char* name, const char* const* options,
               int num_options, void** code, size_t* code_size, char* log, size_t loglen);
void ek_buffer_free(void* p);

/* Module and kernel handles. Replaces fr_pipeline_new + reflection
 * (reference _C/enceladus_rt.mm:251-313). */
int ek_module_load(const void* code, size_t code_size, void** module, char* err, size_t errlen);
int ek_module_unload(void* module, char* err, size_t errlen);
int ek_module_function(void* module, const char* name, void** function, char* err,
                       size_t errlen);
typedef struct ek_function_attrs {
  int32_t num_regs;
  int32_t shared_bytes;      /* static LDS */
  int32_t local_bytes;       /* scratch (register spills) per thread */
  int32_t max_threads;
} ek_function_attrs;
int ek_function_get_attrs(void* function, ek_function_attrs* out, char* err, size_t errlen);

/* Launch with a packed kernarg buffer (natural alignment, as the AMDGPU ABI lays out
 * kernel parameters). Replaces fr_stream_dispatch/encode (reference
 * _C/enceladus_rt.mm:394-427). `stream` may be NULL for the null stream. */
int ek_launch(void* stream, void* function, uint32_t gx, uint32_t gy, uint32_t gz,
              uint32_t bx, uint32_t by, uint32_t bz, uint32_t dyn_lds, void* kernarg,
              size_t kernarg_size, char* err, size_t errlen);

/* Streams. Replaces fr_stream_new/fr_stream_sync (reference _C/enceladus_rt.mm:357-577). */
int ek_stream_new(void** stream, char* err, size_t errlen);
int ek_stream_free(void* stream, char* err, size_t errlen);
int ek_stream_sync(void* stream, char* err, size_t errlen);
int ek_device_sync(char* err, size_t errlen);

/* Device memory. Replaces shared MTLBuffers (reference _C/enceladus_rt.mm:317-352). */
int ek_malloc(void** ptr, size_t bytes, char* err, size_t errlen);
int ek_free(void* ptr, char* err, size_t errlen);
int ek_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream, char* err,
                  size_t errlen);
int ek_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream, char* err,
                  size_t errlen);
int ek_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream, char* err,
                  size_t errlen);
int ek_memset(void* dst, int value, size_t bytes, void* stream, char* err, size_t errlen);

/* GPU timing with events on `stream`. Replaces fr_stream_timed_run /
 * fr_stream_flush_timed (reference _C/enceladus_rt.mm:605, 626). */
int ek_event_new(void** event, char* err, size_t errlen);
int ek_event_free(void* event, char* err, size_t errlen);
int ek_event_record(void* event, void* stream, char* err, size_t errlen);
int ek_event_elapsed_ms(void* start, void* stop, float* ms, char* err, size_t errlen);

/* ek_launch that also records `start_event` (may be NULL) when the dispatch begins and
 * `stop_event` (may be NULL) when it ends, so the elapsed time between them is the GPU time
 * of the dispatches alone, without the host's launch latency. Replaces the GPU timestamps
 * of a flushed command buffer (fr_stream_flush_timed, reference _C/enceladus_rt.mm:626).
 * Grid x block must stay below 2^32 threads per dimension. */
int ek_launch_timed_events(void* stream, void* function, uint32_t gx, uint32_t gy,
                           uint32_t gz, uint32_t bx, uint32_t by, uint32_t bz,
                           uint32_t dyn_lds, void* kernarg, size_t kernarg_size,
                           void* start_event, void* stop_event, char* err, size_t errlen);

/* Launches `function` `reps` times back to back between two events and returns the
 * average milliseconds per launch. */
int ek_timed_launch(void* stream, void* function, uint32_t gx, uint32_t gy, uint32_t gz,
                    uint32_t bx, uint32_t by, uint32_t bz, uint32_t dyn_lds, void* kernarg,
                    size_t kernarg_size, int reps, float* ms_per_launch, char* err,
                    size_t errlen);

/* No counterpart in the reference. For callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): launches a
 * kernel that keeps per-workgroup partial results in a scratch buffer (a privatised-bin
 * kernel), then its second flush level, exactly as the allocating path does with two
 * ek_launch calls and a library-allocated partial buffer, but with the scratch in this
 * library's static device array of EK_SCRATCH_BYTES per GPU (held until the process ends).
 * `kernarg` / `flush_kernarg` are packed as for ek_launch; the scratch address is written
 * at byte offset `scratch_offset` / `flush_scratch_offset` (8-byte aligned) of copies of
 * them. Block sizes are 1-D. Fails, launching nothing, when `scratch_bytes` exceeds
 * EK_SCRATCH_BYTES. Calls no allocating routine. Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams, other threads) race; calls in one
 * stream's order do not. Nothing needs clearing between calls: the first kernel writes
 * every bin word of the partial rows before the flush kernel reads it. The flush's 16-byte
 * loads also read the padding words between bin groups (bin counts are rounded up to 4),
 * which no kernel writes; no atomic targets them, so their stale contents are discarded. */
#define EK_SCRATCH_BYTES (16u << 20)
int ek_launch_flush_noalloc(void* stream, void* function, uint32_t gx, uint32_t gy,
                            uint32_t gz, uint32_t block, const void* kernarg,
                            size_t kernarg_size, size_t scratch_offset, void* flush_function,
                            uint32_t fgx, uint32_t fgy, uint32_t fblock,
                            const void* flush_kernarg, size_t flush_kernarg_size,
                            size_t flush_scratch_offset, size_t scratch_bytes, char* err,
                            size_t errlen);

/* Version string of the shim and of the HIP runtime it runs on. */
const char* ek_version(void);
int ek_runtime_version(int* version);

#ifdef __cplusplus
}
#endif
#endif
