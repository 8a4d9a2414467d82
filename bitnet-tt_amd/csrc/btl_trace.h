// Phase timestamps for measurement builds (-DBTL_TRACE only; compiled out
// otherwise): lane 0 of each wave stores s_memrealtime (100 MHz, one clock
// for the whole device) at a kernel's numbered events into
// g_trace[block][wave][event]; BTL_TRACE_READ_FN(name) defines name(dst, bytes),
// which copies the table out and clears it (measurement builds).  Each
// translation unit has its own table.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifdef BTL_TRACE
namespace btl {
constexpr int kTraceBlocks = 2048, kTraceWaves = 16, kTraceEvents = 16;
static __device__ uint64_t g_trace[kTraceBlocks][kTraceWaves][kTraceEvents];
}  // namespace btl
#define BTL_TRACE_AT(ev)                                                                                   \
  do {                                                                                                     \
    if (__lane_id() == 0 && blockIdx.x < (unsigned)::btl::kTraceBlocks)                                    \
      ::btl::g_trace[blockIdx.x][threadIdx.x >> 6][(ev)] = __builtin_amdgcn_s_memrealtime();               \
  } while (0)
#define BTL_TRACE_READ_FN(name)                                                                            \
  extern "C" int name(void* dst, size_t bytes) {                                                           \
    if (bytes > sizeof(::btl::g_trace)) bytes = sizeof(::btl::g_trace);                                    \
    if (hipMemcpyFromSymbol(dst, HIP_SYMBOL(::btl::g_trace), bytes, 0, hipMemcpyDeviceToHost) != hipSuccess) \
      return 1;                                                                                            \
    static uint64_t zeros[sizeof(::btl::g_trace) / 8];                                                     \
    return hipMemcpyToSymbol(HIP_SYMBOL(::btl::g_trace), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice) != \
           hipSuccess;                                                                                     \
  }
#else
#define BTL_TRACE_AT(ev) \
  do {                   \
  } while (0)
#define BTL_TRACE_READ_FN(name)
#endif
