// Query quantization into the reference's Q-once tile: per KV head h, 64 rows
// of head_dim int8 codes (row r is query token r / 6 of query head
// h * 6 + r % 6; rows past the live ones are zero) and one fp32 scale per
// row.  Reference entry points: q_quant_once (padded [hkv, 64, D] input) and
// the pack-and-quantize step of int8k_int4v_s1_varlen_from_q (token rows
// [T, 6 * hkv, D]), k8v4_v030/native/xe2_kv_ops.cpp:205-294, :1248-1265,
// :1670-1690.  The rule is the K rule of k8v4_v030/oracle.py:22-40 in
// float64 (k_rule_code), the same code path the decode kernel's prologue
// uses for its in-kernel quantization; the stored scale is the float64
// amax / 127 rounded to fp32.
//
// Mapping: one wave per tile row, head_dim / 64 consecutive elements per
// lane, the row max by a wave reduction.  The tile is tiny (hkv * 64 rows),
// so the kernel is latency-bound by design.
#include "k8v4_common.h"

namespace k8v4 {
namespace {

struct QQuantArgs {
  const uint16_t *q;
  int bf16;
  int padded;          // 1: [hkv, 64, D] rows; 0: token rows [batch * q_len, 6 * hkv, D]
  int64_t tok_stride;  // elements between tokens (token layout)
  int64_t rows;        // tile rows: batch * hkv * 64
  int q_len;           // query tokens per sequence (token layout)
  int hkv;
  int8_t *q8;
  float *q_scale;
};

template <int D>
__global__ __launch_bounds__(256) void q_quant_kernel(QQuantArgs a) {
#pragma clang fp contract(off)
  constexpr int E = D / kWave;  // elements per lane
  const int lane = threadIdx.x & (kWave - 1);
  const int row = static_cast<int>(blockIdx.x) * 4 + static_cast<int>(threadIdx.x) / kWave;
  if (row >= a.rows) return;  // whole waves
  const int bh = row / kPage, r = row - bh * kPage;  // bh = b * hkv + h
  const int b = bh / a.hkv, h = bh - b * a.hkv;
  const uint16_t *src = nullptr;
  if (a.padded) {
    src = a.q + static_cast<int64_t>(row) * D;
  } else if (r < a.q_len * kGqa) {
    const int tok = r / kGqa;
    src = a.q + (static_cast<int64_t>(b) * a.q_len + tok) * a.tok_stride +
          static_cast<int64_t>(h * kGqa + (r - tok * kGqa)) * D;
  }
  // One load per lane (rows start 16-byte aligned: both entry points require
  // it), under one condition: per-element selects become one branch and
  // one round trip each.
  uint32_t words[E / 2] = {};
  if (src) {
    if constexpr (E == 4) {
      const uint2 w = *reinterpret_cast<const uint2 *>(src + lane * E);
      words[0] = w.x;
      words[E / 2 - 1] = w.y;
    } else {
      words[0] = *reinterpret_cast<const uint32_t *>(src + lane * E);
    }
  }
  float x[E];
#pragma unroll
  for (int e = 0; e < E; ++e)
    x[e] = half_bits_to_float(static_cast<uint16_t>(words[e >> 1] >> (16 * (e & 1))), a.bf16);
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) amax = fmaxf(amax, fabsf(x[e]));
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, kWave));
  const double scale = amax == 0.f ? 0.0 : static_cast<double>(amax) / 127.0;
  const double inv = amax == 0.f ? 0.0 : 1.0 / scale;
  uint32_t packed = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) packed |= (static_cast<uint32_t>(k_rule_code(x[e], inv)) & 0xFFu) << (8 * e);
  int8_t *dst = a.q8 + static_cast<int64_t>(row) * D + lane * E;
  if constexpr (E == 4)
    *reinterpret_cast<uint32_t *>(dst) = packed;
  else
    *reinterpret_cast<uint16_t *>(dst) = static_cast<uint16_t>(packed);
  if (lane == 0) a.q_scale[row] = static_cast<float>(scale);
}

}  // namespace

int q_quant_launch(const void *q, int bf16, int padded, int64_t q_tok_stride, int64_t batch, int q_len, int hkv,
                   int head_dim, int8_t *q8, float *q_scale, hipStream_t stream) {
  QQuantArgs a;
  a.q = static_cast<const uint16_t *>(q);
  a.bf16 = bf16;
  a.padded = padded;
  a.tok_stride = q_tok_stride;
  a.rows = batch * hkv * kPage;
  a.q_len = q_len;
  a.hkv = hkv;
  a.q8 = q8;
  a.q_scale = q_scale;
  const dim3 grid(static_cast<unsigned>((a.rows + 3) / 4));
  if (head_dim == 128)
    q_quant_kernel<128><<<grid, dim3(256), 0, stream>>>(a);
  else
    q_quant_kernel<256><<<grid, dim3(256), 0, stream>>>(a);
  return launch_status("k8v4 query quantization");
}

}  // namespace k8v4

extern "C" int k8v4_q_quant(const void *q, int q_dtype, int layout, int64_t q_tok_stride, int64_t ntok, int hkv,
                            int head_dim, int8_t *q8, float *q_scale, void *stream) {
  using namespace k8v4;
  clear_error();
  K8V4_REQUIRE(supported_heads(hkv), "unsupported per-GPU KV head count %d (this library serves 2 or 4)", hkv);
  K8V4_REQUIRE(supported_dim(head_dim), "unsupported head dim %d (this library serves 128 or 256)", head_dim);
  K8V4_REQUIRE(q_dtype == K8V4_F16 || q_dtype == K8V4_BF16, "q dtype must be fp16 or bf16");
  K8V4_REQUIRE(layout == K8V4_Q_TOKENS || layout == K8V4_Q_PADDED, "unknown query layout %d", layout);
  K8V4_REQUIRE(q && q8 && q_scale, "null pointer");
  if (layout == K8V4_Q_TOKENS) {
    K8V4_REQUIRE(ntok > 0 && ntok * kGqa <= kPage, "tq*GQA exceeds BM");
    K8V4_REQUIRE(q_tok_stride >= int64_t(hkv) * kGqa * head_dim, "q token stride shorter than HQ*D");
  }
  K8V4_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 && (layout == K8V4_Q_PADDED || q_tok_stride % 8 == 0),
               "q must be 16-byte aligned with a token stride that is a multiple of 8 elements");
  K8V4_REQUIRE(reinterpret_cast<uintptr_t>(q8) % 4 == 0 && reinterpret_cast<uintptr_t>(q_scale) % 4 == 0,
               "q8 / q_scale misaligned");
  return q_quant_launch(q, q_dtype == K8V4_BF16, layout == K8V4_Q_PADDED, q_tok_stride, 1,
                        layout == K8V4_Q_TOKENS ? static_cast<int>(ntok) : 0, hkv, head_dim, q8, q_scale,
                        static_cast<hipStream_t>(stream));
}
