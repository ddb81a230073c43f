// Shared device helpers and host-side error plumbing for the gfx950 MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "janus_moe.h"

namespace janus {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---- host side -----------------------------------------------------------------------------------------------

void set_error(const char* fmt, ...);

#define JANUS_REQUIRE(cond, code, ...)   \
  do {                                   \
    if (!(cond)) {                       \
      ::janus::set_error(__VA_ARGS__);   \
      return (code);                     \
    }                                    \
  } while (0)

#define JANUS_LAUNCH_CHECK(what)                                                                   \
  do {                                                                                             \
    hipError_t _e = hipGetLastError();                                                             \
    if (_e != hipSuccess) {                                                                        \
      ::janus::set_error("%s: launch failed: %s", (what), hipGetErrorString(_e));                \
      return JANUS_MOE_ELAUNCH;                                                                    \
    }                                                                                              \
  } while (0)

// Sticky status bits the kernels set in the current device's status word (janus_moe_device_status reads and clears
// it). The word is library state: a caller's workspace is fresh memory on every call and could not keep a bit until
// it is read.
constexpr int kStatusGaveUp = 1;      // a down unit of the persistent experts launch gave up waiting for its h rows;
                                      // the output rows of its tokens are NaN
constexpr int kStatusDroppedIds = 2;  // an expert id outside [0, E) reached janus_moe_experts(_nvfp4); it was skipped

// The current device's status word (device memory), or null if the runtime cannot resolve it.
int* device_status_word();

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Carves a caller-provided workspace into 256-byte aligned pieces, in a fixed order shared by the size query and
// the call (so both walk the same layout).
struct Carver {
  char* base;
  size_t used = 0;
  explicit Carver(void* p) : base(static_cast<char*>(p)) {}
  template <typename T>
  T* take(size_t count) {
    used = align_up(used, 256);
    T* p = base ? reinterpret_cast<T*>(base + used) : nullptr;
    used += count * sizeof(T);
    return p;
  }
};

// ---- device side -------------------------------------------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// Round-to-nearest-even fp32 -> bf16 bits (the hardware conversion on gfx950; NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v;
  v[0] = static_cast<__bf16>(lo);
  v[1] = static_cast<__bf16>(hi);
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

#define JANUS_LDS __attribute__((address_space(3)))

// Barrier without the memory fence __syncthreads() adds (which would wait for every outstanding load, prefetches
// included): LDS reads and writes are completed first, and the asm keeps the compiler from moving memory accesses
// across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace janus
