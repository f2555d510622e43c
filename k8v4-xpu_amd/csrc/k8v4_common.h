// Shared host/device helpers of the k8v4 HIP library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/k8v4_abi.h"

namespace k8v4 {

constexpr int kPage = 64;
constexpr int kGqa = 6;
constexpr int kWave = 64;

// Per-thread message of the last failed ABI call.
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define K8V4_REQUIRE(cond, ...)            \
  do {                                     \
    if (!(cond)) {                         \
      ::k8v4::set_error(__VA_ARGS__);      \
      return K8V4_ERR_ARG;                 \
    }                                      \
  } while (0)

// Checks the launch that was just enqueued.
int launch_status(const char *what);

// Compute units of the current device (cached per device; 256 if unknown).
int device_cus();

inline bool supported_heads(int hkv) { return hkv == 2 || hkv == 4; }
inline bool supported_dim(int d) { return d == 128 || d == 256; }

// Loads one element of a 16-bit float tensor as float (exact for fp16 and bf16).
__device__ __forceinline__ float half_bits_to_float(uint16_t bits, bool is_bf16) {
  if (is_bf16) return __uint_as_float(static_cast<uint32_t>(bits) << 16);
  return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

}  // namespace k8v4
