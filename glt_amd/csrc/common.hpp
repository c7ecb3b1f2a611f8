// Shared device/host helpers for the gfx950 graft-layer kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/glt.h"

namespace glt {

// ---------------------------------------------------------------- errors
// Sets the thread-local error text returned by glt_last_error_string().
void set_error(const char* fmt, ...);
glt_status hip_fail(hipError_t e, const char* what);

#define GLT_TRY_HIP(expr)                                   \
  do {                                                      \
    hipError_t _e = (expr);                                 \
    if (_e != hipSuccess) return ::glt::hip_fail(_e, #expr); \
  } while (0)

#define GLT_CHECK(cond, code, ...)          \
  do {                                      \
    if (!(cond)) {                          \
      ::glt::set_error(__VA_ARGS__);        \
      return (code);                        \
    }                                       \
  } while (0)

// Checks the launch that was just issued.
#define GLT_LAUNCH_CHECK(name) GLT_TRY_HIP(hipGetLastError())

// Launch timing: while glt_profile_enable(1) is in effect, prof_slot hands
// out a pair of pooled HIP events for a launch (or returns -1), and the
// launch goes through hipExtLaunchKernelGGL, which binds both events to the
// kernel dispatch itself: their elapsed time is the kernel's execution time
// (as a kernel trace reports it), without the gaps that event records
// placed on the stream around a launch add.
int prof_slot(const char* label, hipEvent_t* start, hipEvent_t* stop);  // record id or -1

// Launch with optional timing under `label`.
#define GLT_LAUNCH(label, kernel, grid, block, shmem, st, ...)                                   \
  do {                                                                                           \
    hipEvent_t _e0 = nullptr, _e1 = nullptr;                                                     \
    if (::glt::prof_slot(label, &_e0, &_e1) >= 0)                                                \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, st, _e0, _e1, 0, __VA_ARGS__);           \
    else                                                                                         \
      hipLaunchKernelGGL(kernel, grid, block, shmem, st, __VA_ARGS__);                           \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------------ bf16
// bf16 <-> f32 exactly as the reference defines them
// (reference src/kernels_elementwise_impl.inc:570-580): widening is a 16-bit
// shift; narrowing is round-to-nearest-even via the 0x7FFF + lsb bias
// (NaN payloads are not special-cased, as in the reference).
__host__ __device__ __forceinline__ float bf16_to_f32(uint16_t v) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(v) << 16);
}
__host__ __device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t bits = __builtin_bit_cast(uint32_t, f);
  bits += 0x7FFFu + ((bits >> 16) & 1u);
  return static_cast<uint16_t>(bits >> 16);
}
__host__ __device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

// ------------------------------------------------------- buffer resources
// Raw buffer loads give hardware bounds checking: an access whose byte offset
// is >= num_records returns zero. Tiles use this for M/N tails and for rows
// outside a graft slice (offset forced to kOob).
constexpr uint32_t kOob = 0x80000000u;
// Word 3 of a gfx9-family buffer descriptor (32-bit dword data format, no
// swizzle, no stride); the same value CDNA3 code generators use.
constexpr int32_t kBufferWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), /*stride=*/0,
                                           static_cast<int>(bytes), kBufferWord3);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace glt
