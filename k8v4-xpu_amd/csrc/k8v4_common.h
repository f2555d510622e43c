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

// Enqueues the query quantization into Q-once tiles: per sequence b < batch
// and KV head h, 64 rows of head_dim int8 codes at q8 + ((b * hkv + h) * 64 +
// r) * head_dim (row r: query token r / 6 of query head h * 6 + r % 6, zero
// past q_len tokens) and one fp32 scale per row at q_scale + (b * hkv + h) *
// 64 + r.  Token layout: query rows [batch * q_len][6 * hkv][head_dim] with
// q_tok_stride elements between tokens; padded layout (batch 1): the rows
// [hkv][64][head_dim] as they are.  Arguments are not checked here.
int q_quant_launch(const void *q, int bf16, int padded, int64_t q_tok_stride, int64_t batch, int q_len, int hkv,
                   int head_dim, int8_t *q8, float *q_scale, hipStream_t stream);

// Loads one element of a 16-bit float tensor as float (exact for fp16 and bf16).
__device__ __forceinline__ float half_bits_to_float(uint16_t bits, bool is_bf16) {
  if (is_bf16) return __uint_as_float(static_cast<uint32_t>(bits) << 16);
  return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

// One element's code under the K rule of k8v4_v030/oracle.py:22-40 (also the
// reference's query rule, oracle.py:145): q = round_half_away(x * inv) with
// inv = 1 / (amax / 127), all in float64.  |q| = floor(|x| * inv + 0.5); with
// |x| <= amax the product stays within 1e-13 of 127, so the reference's clamp
// to 127 never acts and the truncating conversion of the positive |x| * inv +
// 0.5 is its floor.  The caller passes inv = 0 for an all-zero row.  The
// multiply and the add round separately (no contraction into an fma).
__device__ __forceinline__ int32_t k_rule_code(float x, double inv) {
#pragma clang fp contract(off)
  const double ay = static_cast<double>(fabsf(x)) * inv;
  const int32_t qa = static_cast<int32_t>(ay + 0.5);
  return x < 0.f ? -qa : qa;
}

// Wave-wide scans of non-negative ints by DPP moves (register to register,
// a few cycles each; the LDS permutes a shuffle compiles to cost a round trip
// through the LDS unit per step, and the plan is on the critical path of
// every work-group's prologue).  Within each 16-lane row, row_shr 1, 2, 4, 8
// (a lane with no source in its row reads 0); then lane 15 of rows 0 and 2 is
// added to rows 1 and 3 (row_bcast:15) and lane 31 to rows 2 and 3
// (row_bcast:31).  All 64 lanes must be active.
template <bool MAX>
__device__ __forceinline__ int dpp_step(int x, int y) {
  return MAX ? max(x, y) : x + y;
}
template <bool MAX>
__device__ __forceinline__ int wave_scan_dpp(int x) {
  x = dpp_step<MAX>(x, __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false));  // row_shr:1
  x = dpp_step<MAX>(x, __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false));  // row_shr:2
  x = dpp_step<MAX>(x, __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false));  // row_shr:4
  x = dpp_step<MAX>(x, __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false));  // row_shr:8
  x = dpp_step<MAX>(x, __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false));  // row_bcast:15
  x = dpp_step<MAX>(x, __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false));  // row_bcast:31
  return x;
}
// Sum / max over the wave (x >= 0), the same value in every lane.
__device__ __forceinline__ int wave_sum(int x) { return __builtin_amdgcn_readlane(wave_scan_dpp<false>(x), kWave - 1); }
__device__ __forceinline__ int wave_max(int x) { return __builtin_amdgcn_readlane(wave_scan_dpp<true>(x), kWave - 1); }
// Inclusive prefix sum over the lanes (x >= 0).
__device__ __forceinline__ int wave_inclusive_scan(int x) { return wave_scan_dpp<false>(x); }

}  // namespace k8v4
