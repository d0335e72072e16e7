// Shared helpers for the MALOQ MI355X (gfx950) kernels.
//
// Error model of the C ABI: every entry point returns 0 on success and a
// non-zero code on failure; maloq_last_error() returns a thread-local message.
// Entry points never synchronise the stream they are given.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#define MALOQ_OK 0
#define MALOQ_EINVAL 1
#define MALOQ_EHIP 2

namespace maloq {

void set_error(const char* fmt, ...);

// Returns MALOQ_EHIP (and records the message) if the last launch failed.
int check_launch(const char* what);

// Compute units of the current device (queried once per device; 256 if the
// query fails).
int device_cus();

__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

}  // namespace maloq

#define MALOQ_REQUIRE(cond, ...)        \
  do {                                  \
    if (!(cond)) {                      \
      maloq::set_error(__VA_ARGS__);    \
      return MALOQ_EINVAL;              \
    }                                   \
  } while (0)
