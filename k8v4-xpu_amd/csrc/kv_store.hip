// KV quantize-and-write: fp16/bf16 K and V rows -> int8 K codes, packed
// int4 V codes and fp32 planes inside the paged cache.
//
// Reference: k8v4_v030/native/xe2_kv_ops.cpp:536-627 (two kernels, fp32
// arithmetic with rint) and the parity oracle k8v4_v030/oracle.py:18-69
// (float64, half-away-from-zero for K, floor(x+0.5) for V).  This kernel
// follows the oracle: scales are the same IEEE double operations in the same
// order, and every code equals the float64 rule's (an fp32 evaluation is used
// only where its error bound cannot change the result, see below), so codes
// and stored scales are bit-identical to it.  This file is compiled with
// -ffp-contract=off and the kernel body disables contraction as well, so no
// multiply-add is fused.
//
// Mapping (MI355X): K and V of one (token, kv_head) pair are handled by the
// same D/16 lanes, 16 consecutive dims per lane (two 16-byte loads of K and
// two of V).  Consecutive pairs are consecutive heads of a token, so a wave
// writes whole contiguous rows of a page: the store is one pass over the
// inputs and one pass over the outputs.  The per-pair work (float64 scale
// divisions, group reductions, scale stores) is the same for every lane of a
// group, so fewer, wider lanes per pair cut the instruction count per byte.
#include "k8v4_common.h"

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace k8v4 {
namespace {

struct StoreArgs {
  const uint16_t *k;
  const uint16_t *v;
  int64_t k_tok_stride;  // elements
  int64_t v_tok_stride;
  const int64_t *slots;
  int64_t units;  // ntok * hkv
  int8_t *k_cache;
  float *k_scale;
  uint8_t *v_cache;
  float *v_scale;
  float *v_zero;
  int64_t num_pages;
  int64_t k_ps, ks_ps, v_ps, vs_ps, vz_ps;  // page strides, bytes
  int hkv;
  int bf16;
  int vec_ok;  // 16-byte aligned rows: one vector load per lane
  int parts;   // kStoreK | kStoreV: which of K and V this launch writes
};

constexpr int kStoreK = 1, kStoreV = 2;

// E consecutive fp16/bf16 values as E / 2 words (element 2i in the low
// half of word i).  The conversion is a separate step so that the K and V
// loads are all in flight before either is used.
template <int E>
__device__ __forceinline__ void load_words(const uint16_t *src, bool vec_ok, uint32_t w[E / 2]) {
  if (vec_ok) {
#pragma unroll
    for (int c = 0; c < E / 8; ++c) {
      const uint4 v = *reinterpret_cast<const uint4 *>(src + 8 * c);
      w[4 * c] = v.x;
      w[4 * c + 1] = v.y;
      w[4 * c + 2] = v.z;
      w[4 * c + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < E / 2; ++i) w[i] = static_cast<uint32_t>(src[2 * i]) | (static_cast<uint32_t>(src[2 * i + 1]) << 16);
  }
}
template <int E>
__device__ __forceinline__ void words_to_float(const uint32_t w[E / 2], bool bf16, float out[E]) {
#pragma unroll
  for (int i = 0; i < E; ++i) out[i] = half_bits_to_float(static_cast<uint16_t>(w[i >> 1] >> (16 * (i & 1))), bf16);
}

// Max / min over the LPU lanes of one (token, head) group.
template <int LPU>
__device__ __forceinline__ float group_max(float x) {
#pragma unroll
  for (int m = 1; m < LPU; m <<= 1) x = fmaxf(x, __shfl_xor(x, m, kWave));
  return x;
}
template <int LPU>
__device__ __forceinline__ float group_min(float x) {
#pragma unroll
  for (int m = 1; m < LPU; m <<= 1) x = fminf(x, __shfl_xor(x, m, kWave));
  return x;
}

// One wave handles 64/LPU (token, head) pairs; LPU = D/16 lanes per pair.
template <int D>
__global__ __launch_bounds__(256) void kv_store_kernel(StoreArgs a) {
#pragma clang fp contract(off)
  constexpr int E = 16;  // dims per lane
  constexpr int LPU = D / E;
  constexpr int UPW = kWave / LPU;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  const int sub = lane % LPU;
  int64_t unit = wave * UPW + lane / LPU;
  const bool live = unit < a.units;
  if (!live) unit = a.units - 1;  // keep the group's shuffles on real data
  const int64_t token = unit / a.hkv;
  const int head = static_cast<int>(unit - token * a.hkv);

  // The slot first: its load then shares the round trip of the K/V loads.
  const int64_t slot = a.slots[token];
  const bool do_k = a.parts & kStoreK, do_v = a.parts & kStoreV;  // uniform over the launch
  uint32_t kwd[E / 2] = {}, vwd[E / 2] = {};
  if (do_k) load_words<E>(a.k + token * a.k_tok_stride + static_cast<int64_t>(head) * D + E * sub, a.vec_ok, kwd);
  if (do_v) load_words<E>(a.v + token * a.v_tok_stride + static_cast<int64_t>(head) * D + E * sub, a.vec_ok, vwd);
  float kx[E], vx[E];
  if (do_k) words_to_float<E>(kwd, a.bf16, kx);
  if (do_v) words_to_float<E>(vwd, a.bf16, vx);

  float amax = 0.f, lo = 0.f, hi = 0.f;
  if (do_k) {
#pragma unroll
    for (int i = 0; i < E; ++i) amax = fmaxf(amax, fabsf(kx[i]));
    amax = group_max<LPU>(amax);
  }
  if (do_v) {
    lo = hi = vx[0];
#pragma unroll
    for (int i = 0; i < E; ++i) {
      lo = fminf(lo, vx[i]);
      hi = fmaxf(hi, vx[i]);
    }
    lo = group_min<LPU>(lo);
    hi = group_max<LPU>(hi);
  }

  const int64_t page = slot >= 0 ? slot / kPage : -1;
  if (!live || page < 0 || page >= a.num_pages) return;
  const int64_t row = slot - page * kPage;
  const int64_t cell = row * a.hkv + head;

  // Codes are evaluated in fp32 first.  The fp32 value of each pre-rounding
  // quantity is within 2e-5 of the float64 one the rule defines (|y| <= 127
  // for K; |x / s| <= 16.5 wherever the V code is not clamped), so its floor is
  // the float64 floor unless it lies within 2^-12 of an integer; those
  // elements (ties such as x = amax / 254, constant rows) take the float64
  // path, step for step as the rule is written.
  constexpr float kMargin = 0x1p-12f;

  if (do_k) {
  // K: symmetric int8, scale amax/127, round half away from zero.
  const double k_scale = amax == 0.f ? 0.0 : static_cast<double>(amax) / 127.0;
  uint32_t kw[E / 4] = {};
  if (amax != 0.f) {
    const double inv = 1.0 / k_scale;
    const float inv32 = static_cast<float>(inv);
    const bool fast = inv32 <= 3.0e38f;  // a tiny bf16 amax overflows the fp32 reciprocal
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const float y32 = kx[i] * inv32;
      const float d = fabsf(y32) + 0.5f;
      float m = floorf(d);
      const float fr = d - m;
      float q;
      if (!fast || fr < kMargin || fr > 1.f - kMargin) {
        const double y = static_cast<double>(kx[i]) * inv;
        q = static_cast<float>(y >= 0.0 ? floor(y + 0.5) : ceil(y - 0.5));
      } else {
        q = y32 >= 0.f ? m : -m;
      }
      q = fminf(fmaxf(q, -127.f), 127.f);
      const uint32_t b = static_cast<uint32_t>(static_cast<int32_t>(q)) & 0xFFu;
      kw[i >> 2] |= b << (8 * (i & 3));
    }
  }
  // Code rows are written with the nontemporal policy: nothing reads them
  // back in this kernel, and streaming them past the L2 leaves no dirty lines
  // for the end-of-kernel write-back (4 x 4,224 tokens: 17.5 -> 15.3 us).
  char *kdst = reinterpret_cast<char *>(a.k_cache) + page * a.k_ps + cell * D + E * sub;
#pragma unroll
  for (int c = 0; c < E / 16; ++c)
    __builtin_nontemporal_store((u32x4){kw[4 * c], kw[4 * c + 1], kw[4 * c + 2], kw[4 * c + 3]},
                                reinterpret_cast<u32x4 *>(kdst) + c);
  if (sub == 0)
    *reinterpret_cast<float *>(reinterpret_cast<char *>(a.k_scale) + page * a.ks_ps + cell * 4) =
        static_cast<float>(k_scale);
  }
  if (!do_v) return;

  // V: affine uint4 over the whole row, floor(x + 0.5) rounding.
  const double lo_d = lo, hi_d = hi;
  const double span = (hi_d - lo_d) / 15.0;
  const double v_scale = span >= 1.0e-8 ? span : 1.0e-8;
  const double zero = fmin(fmax(floor(-lo_d / v_scale + 0.5), 0.0), 15.0);
  const float rs32 = static_cast<float>(1.0 / v_scale);
  const float z32 = static_cast<float>(zero);
  uint32_t vw[E / 8] = {};
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const float y32 = vx[i] * rs32 + z32 + 0.5f;
    float q = floorf(y32);
    const float fr = y32 - q;
    if (fr < kMargin || fr > 1.f - kMargin)
      q = static_cast<float>(floor(static_cast<double>(vx[i]) / v_scale + zero + 0.5));
    q = fminf(fmaxf(q, 0.f), 15.f);
    vw[i >> 3] |= static_cast<uint32_t>(q) << (4 * (i & 7));
  }

  char *vdst = reinterpret_cast<char *>(a.v_cache) + page * a.v_ps + cell * (D / 2) + (E / 2) * sub;
  __builtin_nontemporal_store((u32x2){vw[0], vw[1]}, reinterpret_cast<u32x2 *>(vdst));
  if (sub == 0) {
    *reinterpret_cast<float *>(reinterpret_cast<char *>(a.v_scale) + page * a.vs_ps + cell * 4) =
        static_cast<float>(v_scale);
    *reinterpret_cast<float *>(reinterpret_cast<char *>(a.v_zero) + page * a.vz_ps + cell * 4) =
        static_cast<float>(zero);
  }
}

bool aligned(const void *p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

}  // namespace
}  // namespace k8v4


namespace k8v4 {
namespace {

// The three store entry points: parts selects K, V or both.
int store_paged(int parts, const void *k, const void *v, int src_dtype, int64_t k_tok_stride, int64_t v_tok_stride,
                const int64_t *slot_mapping, int64_t ntok, int hkv, int head_dim, int8_t *k_cache, float *k_scale,
                uint8_t *v_cache, float *v_scale, float *v_zero, int64_t num_pages, int64_t k_page_stride,
                int64_t ks_page_stride, int64_t v_page_stride, int64_t vs_page_stride, int64_t vz_page_stride,
                void *stream, const char *what) {
  clear_error();
  const bool do_k = parts & kStoreK, do_v = parts & kStoreV;
  K8V4_REQUIRE(supported_heads(hkv), "unsupported per-GPU KV head count %d (this library serves 2 or 4)",
               hkv);
  K8V4_REQUIRE(supported_dim(head_dim), "unsupported head dim %d (this library serves 128 or 256)",
               head_dim);
  K8V4_REQUIRE(src_dtype == K8V4_F16 || src_dtype == K8V4_BF16, "k/v dtype must be fp16 or bf16");
  K8V4_REQUIRE(ntok >= 0 && num_pages >= 0, "negative token or page count");
  if (ntok == 0) return K8V4_OK;
  K8V4_REQUIRE(slot_mapping && (!do_k || (k && k_cache && k_scale)) && (!do_v || (v && v_cache && v_scale && v_zero)),
               "null pointer");
  K8V4_REQUIRE((!do_k || k_tok_stride >= static_cast<int64_t>(hkv) * head_dim) &&
                   (!do_v || v_tok_stride >= static_cast<int64_t>(hkv) * head_dim),
               "k/v token stride shorter than hkv*head_dim");
  K8V4_REQUIRE(aligned(slot_mapping, 8) && (!do_k || (aligned(k_cache, 16) && aligned(k_scale, 4))) &&
                   (!do_v || (aligned(v_cache, 8) && aligned(v_scale, 4) && aligned(v_zero, 4))),
               "cache region or slot pointer misaligned");
  K8V4_REQUIRE((!do_k || (k_page_stride % 16 == 0 && ks_page_stride % 4 == 0)) &&
                   (!do_v || (v_page_stride % 8 == 0 && vs_page_stride % 4 == 0 && vz_page_stride % 4 == 0)),
               "cache page strides must keep rows aligned");
  K8V4_REQUIRE((!do_k || aligned(k, 2)) && (!do_v || aligned(v, 2)), "k/v pointers misaligned");

  StoreArgs a;
  a.k = static_cast<const uint16_t *>(k);
  a.v = static_cast<const uint16_t *>(v);
  a.k_tok_stride = k_tok_stride;
  a.v_tok_stride = v_tok_stride;
  a.slots = slot_mapping;
  a.units = ntok * hkv;
  a.k_cache = k_cache;
  a.k_scale = k_scale;
  a.v_cache = v_cache;
  a.v_scale = v_scale;
  a.v_zero = v_zero;
  a.num_pages = num_pages;
  a.k_ps = k_page_stride;
  a.ks_ps = ks_page_stride;
  a.v_ps = v_page_stride;
  a.vs_ps = vs_page_stride;
  a.vz_ps = vz_page_stride;
  a.hkv = hkv;
  a.bf16 = src_dtype == K8V4_BF16;
  a.vec_ok = (!do_k || (aligned(k, 16) && k_tok_stride % 8 == 0)) && (!do_v || (aligned(v, 16) && v_tok_stride % 8 == 0));
  a.parts = parts;

  const int upw = kWave / (head_dim / 16);
  const int64_t waves = (a.units + upw - 1) / upw;
  const int64_t blocks = (waves + 3) / 4;
  K8V4_REQUIRE(blocks < (int64_t(1) << 31), "too many tokens for one launch");
  auto s = static_cast<hipStream_t>(stream);
  if (head_dim == 128)
    kv_store_kernel<128><<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(a);
  else
    kv_store_kernel<256><<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(a);
  return launch_status(what);
}

}  // namespace
}  // namespace k8v4

extern "C" int k8v4_kv_store_paged(const void *k, const void *v, int src_dtype,
                                   int64_t k_tok_stride, int64_t v_tok_stride,
                                   const int64_t *slot_mapping, int64_t ntok, int hkv,
                                   int head_dim, int8_t *k_cache, float *k_scale,
                                   uint8_t *v_cache, float *v_scale, float *v_zero,
                                   int64_t num_pages, int64_t k_page_stride,
                                   int64_t ks_page_stride, int64_t v_page_stride,
                                   int64_t vs_page_stride, int64_t vz_page_stride, void *stream) {
  return k8v4::store_paged(k8v4::kStoreK | k8v4::kStoreV, k, v, src_dtype, k_tok_stride, v_tok_stride,
                           slot_mapping, ntok, hkv, head_dim, k_cache, k_scale, v_cache, v_scale, v_zero,
                           num_pages, k_page_stride, ks_page_stride, v_page_stride, vs_page_stride,
                           vz_page_stride, stream, "k8v4_kv_store_paged");
}

extern "C" int k8v4_k_store_paged(const void *k, int src_dtype, int64_t k_tok_stride, const int64_t *slot_mapping,
                                  int64_t ntok, int hkv, int head_dim, int8_t *k_cache, float *k_scale,
                                  int64_t num_pages, int64_t k_page_stride, int64_t ks_page_stride, void *stream) {
  return k8v4::store_paged(k8v4::kStoreK, k, nullptr, src_dtype, k_tok_stride, 0, slot_mapping, ntok, hkv,
                           head_dim, k_cache, k_scale, nullptr, nullptr, nullptr, num_pages, k_page_stride,
                           ks_page_stride, 0, 0, 0, stream, "k8v4_k_store_paged");
}

extern "C" int k8v4_v_store_paged(const void *v, int src_dtype, int64_t v_tok_stride, const int64_t *slot_mapping,
                                  int64_t ntok, int hkv, int head_dim, uint8_t *v_cache, float *v_scale,
                                  float *v_zero, int64_t num_pages, int64_t v_page_stride, int64_t vs_page_stride,
                                  int64_t vz_page_stride, void *stream) {
  return k8v4::store_paged(k8v4::kStoreV, nullptr, v, src_dtype, 0, v_tok_stride, slot_mapping, ntok, hkv,
                           head_dim, nullptr, nullptr, v_cache, v_scale, v_zero, num_pages, 0, 0, v_page_stride,
                           vs_page_stride, vz_page_stride, stream, "k8v4_v_store_paged");
}
