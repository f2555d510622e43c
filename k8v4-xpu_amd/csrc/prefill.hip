// Chunked-prefill attention over the int8-K / int4-V paged cache.
//
// Reference semantics: the eager prefill k8v4_v030/dequant.py:213-242
// (gather + dequantize K = code * k_scale, V = (nibble - v_zero) * v_scale,
// then softmax(Q K^T * scale) V) with the bottom-right causal rule of
// dequant.py:245-261 / onednn_prefill.py:89-121: query row j of a q_len
// suffix is token seq_len - q_len + j and sees keys t <= that position.  Q is
// not quantized; accumulation is fp32.
//
// MI355X design:
//  * The problem of one KV head is a matrix of q_len * 6 query rows (token
//    major, the 6 GQA heads of a token adjacent) against seq_len keys.  A
//    work-group owns a block of rows of one KV head and streams every page of
//    that head once: direct-to-LDS loads stage the next page's codes while the
//    current page is computed, then the group converts them into the other
//    buffer of a two-buffer MFMA tile ring.  Each page is a 64-key tile shared
//    by all waves (all GQA rows) of the group.
//  * Dequantization is split so the per-element work is shared by the whole
//    work-group: K codes become fp16 integers (byte permute into the mantissa
//    of 1024.0, then subtract 1152) times the token's K scale and the
//    exp2-domain softmax factor (one fp16 rounding, as a bf16/fp16 dequant
//    has); V nibbles become exact fp16 subnormals (n * 2^-24 for even dims,
//    16 n * 2^-24 for odd dims) in a transposed tile, the V scale multiplies
//    P and the zero point is subtracted once per row at the end:
//      sum_t p_t (n_t - z_t) s_t = sum_t (p_t s_t) n_t - sum_t (p_t s_t) z_t.
//  * S^T = K Q^T and O^T = V^T P'^T on v_mfma_f32_32x32x16_f16 (the 32x32
//    shapes run at twice the rate of the 16x16 ones on gfx950): the query row
//    is the MFMA column, so a lane pair owns one row's softmax state and the
//    score tile is already the B operand of the PV product.
//  * Online softmax in the exp2 domain with a lazy rescale (the running max
//    only moves when a row's max grows by more than 2^2).
#include "k8v4_common.h"

#include <algorithm>

namespace k8v4 {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// Lazy-rescale threshold (log2 units): p stays <= 2^2 before a row's running
// max moves, so P' = p * v_scale stays a finite fp16 even for a V row spanning
// the whole fp16 range (4 * 2 * 65504 / 15 = 34,936).
constexpr float kThreshold = 2.0f;
constexpr uint32_t kEvenNib = 0x000F000Fu;
constexpr uint32_t kOddNib = 0x00F000F0u;

struct PrefillArgs {
  const uint16_t *q;
  int64_t q_tok_stride;  // elements; head stride is head_dim
  int q_bf16;
  const int8_t *k_cache;
  const float *k_scale;
  const uint8_t *v_cache;
  const float *v_scale;
  const float *v_zero;
  int64_t num_pages;
  int64_t k_ps, ks_ps, v_ps, vs_ps, vz_ps;  // page strides, bytes
  const int32_t *block_row;
  int ppb;
  int seq_len;
  int q_len;
  int hkv;
  float c;       // softmax scale * log2(e)
  int rows;      // query rows per block (32 per wave of a work-group)
  int nbh;       // row blocks per KV head
  int tper;      // page steps of one head: sum over its blocks of the pages each reads
  int total;     // page steps of the call (hkv * tper)
  int grid;      // persistent work-groups; work-group v takes steps [v*total/grid, (v+1)*total/grid)
  int xcd_perm;  // map ids so the work-groups of one XCD take adjacent work (grid % 8 == 0)
  float *ws;     // partial states: [grid][2][rows][D + 2] floats
  void *out;
  int out_dtype;
  int64_t out_tok_stride;  // elements
};

template <int D>
struct Tile {
  // D=128: eight waves (two per SIMD) share each converted page; D=256: four
  // waves (one per SIMD, the register file holds the wider accumulators).
  static constexpr int NW = D == 128 ? 8 : 4;        // waves per work-group, one work-group per CU
  static constexpr int WPE = NW / 4;                 // waves per SIMD
  static constexpr int THREADS = 64 * NW;
  static constexpr int ROWS = 32 * NW;               // query rows per block (one 32-row tile per wave)
  static constexpr int DS = D / 16;                  // k-steps of the QK MFMA (16 dims each)
  static constexpr int DT = D / 32;                  // 32-dim output tiles
  // MFMA tile of one page (one ring buffer).  Row paddings, not XOR
  // swizzles, keep the operand reads conflict-free, so every read address is
  // one per-lane base plus a compile-time offset.
  static constexpr int KROW = 2 * D + 16;            // K row: D fp16 codes + 16 B (8 rows hit 8 bank groups)
  static constexpr int K_BYTES = 64 * KROW;
  // V^T: row d = the 64 keys' fp16 values, key k at position k with bits 2
  // and 3 swapped, so the 8 keys one lane feeds to a 16-key MFMA step sit in
  // 16 contiguous bytes.  Rows padded to 144 B (D = 128: one aligned 16-byte
  // read per operand, 16 rows hit all 64 banks) or 136 B (D = 256, where the
  // LDS is full: two 8-byte reads).
  static constexpr int V_OFF = K_BYTES;
  static constexpr int VROW = D == 128 ? 144 : 136;
  static constexpr int S_OFF = V_OFF + D * VROW;     // ksc[64] | vs[64] | vz[64] floats
  static constexpr int BUF = S_OFF + 768;
  // Staging of the next page's raw codes: [64][D] K | V as 16-byte pieces
  // ordered [part q][key parity][key pair] (its scale planes go straight into
  // the S area of the ring buffer they belong to).
  static constexpr int SV_OFF = 64 * D;
  static constexpr int STAGE = SV_OFF + 32 * D;
  static constexpr int KDMA = D / 16;                 // 1 KB K pieces per page (one DMA each)
  static constexpr int VDMA = D / 32;                 // 1 KB V pieces per page
  static constexpr int KCHUNKS = 4 * D;               // 16-byte K code chunks per page
  static constexpr int VITEMS = 2 * D;                // (part, half, key pair) V items per page
};

typedef const __attribute__((address_space(4))) int32_t *const_i32_ptr;

__device__ __forceinline__ int64_t page_of(const PrefillArgs &a, int p) {
  const const_i32_ptr row = (const_i32_ptr)(a.block_row);
  int64_t phys = a.ppb <= 1 ? row[p] : static_cast<int64_t>(row[p / a.ppb]) * a.ppb + (p % a.ppb);
  if (phys < 0 || phys >= a.num_pages) phys = 0;  // stay in bounds on a bad table entry
  return phys;
}

// ---- page staging: direct-to-LDS loads of one page of one head (no registers
// held while the previous page is computed), then a work-group pass that
// converts the staged codes into the MFMA tile of the next ring buffer.
typedef __attribute__((address_space(3))) char lds_t;

__device__ __forceinline__ void dma16(const void *src, lds_t *dst) {
  __builtin_amdgcn_global_load_lds(src, reinterpret_cast<__attribute__((address_space(3))) void *>(dst), 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void *src, lds_t *dst) {
  __builtin_amdgcn_global_load_lds(src, reinterpret_cast<__attribute__((address_space(3))) void *>(dst), 4, 0, 0);
}

// DMA idx (taken by wave idx % NW), lane L: 16-byte K piece 64 * idx + L
// (row-major codes), V pieces likewise, and scale plane w (waves 0-2) for key
// L, the latter into the S area of the ring buffer the page is converted into.
template <int D>
__device__ __forceinline__ void stage_page(const PrefillArgs &a, int p, int h, int wave, int lane, lds_t *stage,
                                           lds_t *scales) {
  using T = Tile<D>;
  const int64_t phys = page_of(a, p);
  const char *kb = reinterpret_cast<const char *>(a.k_cache) + phys * a.k_ps + h * D;
  const char *vb = reinterpret_cast<const char *>(a.v_cache) + phys * a.v_ps + h * (D / 2);
#pragma unroll
  for (int j = 0; j < (T::KDMA + T::NW - 1) / T::NW; ++j) {
    const int idx = T::NW * j + wave;
    if (idx < T::KDMA) {
      const int c = 64 * idx + lane;
      const int key = c / (D / 16), part = c % (D / 16);
      dma16(kb + static_cast<int64_t>(key) * a.hkv * D + part * 16, stage + 1024 * idx);
    }
  }
#pragma unroll
  for (int j = 0; j < (T::VDMA + T::NW - 1) / T::NW; ++j) {
    const int idx = T::NW * j + wave;
    if (idx < T::VDMA) {
      // piece q = idx of key 2 * (lane % 32) + lane / 32
      const int key = 2 * (lane & 31) + (lane >> 5);
      dma16(vb + static_cast<int64_t>(key) * a.hkv * (D / 2) + idx * 16, stage + T::SV_OFF + 1024 * idx);
    }
  }
  if (wave < 3) {
    const float *plane = wave == 0 ? a.k_scale : wave == 1 ? a.v_scale : a.v_zero;
    const int64_t ps = wave == 0 ? a.ks_ps : wave == 1 ? a.vs_ps : a.vz_ps;
    const char *src = reinterpret_cast<const char *>(plane) + phys * ps + (static_cast<int64_t>(lane) * a.hkv + h) * 4;
    dma4(src, scales + 256 * wave);
  }
}

__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// int8 codes (4 per dword) -> exact fp16 integers.
__device__ __forceinline__ void k_codes_to_f16(uint32_t w, v2h &lo, v2h &hi) {
  const uint32_t u = w ^ 0x80808080u;  // biased: code + 128
  const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  const v2h bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  lo = __builtin_bit_cast(v2h, a) - bias;
  hi = __builtin_bit_cast(v2h, b) - bias;
}

template <int D>
__device__ __forceinline__ void convert_page(const PrefillArgs &a, int p, const char *stage, char *buf, int tid) {
  using T = Tile<D>;
#pragma unroll
  for (int j = 0; j < (T::KCHUNKS + T::THREADS - 1) / T::THREADS; ++j) {
    const int c = tid + T::THREADS * j;
    if (c >= T::KCHUNKS) break;
    const int key = c / (D / 16), part = c % (D / 16);
    const uint4 w = *reinterpret_cast<const uint4 *>(stage + 16 * c);
    // K scale times the exp2-domain softmax factor, folded into the tile (a
    // key past the sequence gets 0: its unwritten plane may hold anything).
    const float ks = reinterpret_cast<const float *>(buf + T::S_OFF)[key];
    const float kc = p * 64 + key < a.seq_len ? ks * a.c : 0.f;
    const v2h kc2 = {static_cast<_Float16>(kc), static_cast<_Float16>(kc)};
    v2h h[8];
    k_codes_to_f16(w.x, h[0], h[1]);
    k_codes_to_f16(w.y, h[2], h[3]);
    k_codes_to_f16(w.z, h[4], h[5]);
    k_codes_to_f16(w.w, h[6], h[7]);
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] *= kc2;
    char *row = buf + key * T::KROW;
    const uint4 c0 = make_uint4(__builtin_bit_cast(uint32_t, h[0]), __builtin_bit_cast(uint32_t, h[1]),
                                __builtin_bit_cast(uint32_t, h[2]), __builtin_bit_cast(uint32_t, h[3]));
    const uint4 c1 = make_uint4(__builtin_bit_cast(uint32_t, h[4]), __builtin_bit_cast(uint32_t, h[5]),
                                __builtin_bit_cast(uint32_t, h[6]), __builtin_bit_cast(uint32_t, h[7]));
    *reinterpret_cast<uint4 *>(row + 32 * part) = c0;
    *reinterpret_cast<uint4 *>(row + 32 * part + 16) = c1;
  }
  // V: item (part q, half, key pair p) reads the 16-byte pieces of keys 2p and
  // 2p + 1 (the half's 8 bytes are dims 32q + 16 half .. + 15) and writes one
  // word (both keys) into each of those 16 V^T rows.  Lanes run over key
  // pairs, so the piece reads are consecutive and the 64 row writes of one
  // instruction land in 64 distinct banks (rows 16 apart are 32 banks apart).
#pragma unroll
  for (int j = 0; j < (T::VITEMS + T::THREADS - 1) / T::THREADS; ++j) {
    const int it = tid + T::THREADS * j;
    if (it >= T::VITEMS) break;
    const int q = it >> 6, half = (it >> 5) & 1, pair = it & 31;
    const uint4 e4 = *reinterpret_cast<const uint4 *>(stage + T::SV_OFF + (q * 64 + pair) * 16);
    const uint4 o4 = *reinterpret_cast<const uint4 *>(stage + T::SV_OFF + (q * 64 + 32 + pair) * 16);
    const uint32_t ev[2] = {half ? e4.z : e4.x, half ? e4.w : e4.y};
    const uint32_t od[2] = {half ? o4.z : o4.x, half ? o4.w : o4.y};
    const int kp = 2 * pair;  // even key; its column swaps bits 2 and 3
    const int col = (kp & ~12) | ((kp & 4) << 1) | ((kp & 8) >> 1);
    char *vrow = buf + T::V_OFF + (32 * q + 16 * half) * T::VROW + 2 * col;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint32_t sel = 0x0C000C00u | ((4u + (b & 3)) << 16) | (b & 3);
      const uint32_t x = __builtin_amdgcn_perm(od[b >> 2], ev[b >> 2], sel);  // byte b of both keys
      *reinterpret_cast<uint32_t *>(vrow + (2 * b) * T::VROW) = x & kEvenNib;
      *reinterpret_cast<uint32_t *>(vrow + (2 * b + 1) * T::VROW) = x & kOddNib;
    }
  }
  if (tid < 64) {
    float *s = reinterpret_cast<float *>(buf + T::S_OFF);
    // Keys past the sequence may hold anything (unwritten planes): zero them
    // so a masked probability never meets a NaN scale.
    const bool live = p * 64 + tid < a.seq_len;
    s[64 + tid] = live ? s[64 + tid] : 0.f;
    s[128 + tid] = live ? s[128 + tid] : 0.f;
  }
}

__device__ __forceinline__ void store_out4(void *out, int dtype, int64_t idx, v4f v) {
  if (dtype == K8V4_F32) {
    *reinterpret_cast<v4f *>(static_cast<float *>(out) + idx) = v;
  } else if (dtype == K8V4_BF16) {
    __bf16 *o = static_cast<__bf16 *>(out) + idx;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = static_cast<__bf16>(v[i]);
  } else {
    const v4h h = __builtin_convertvector(v, v4h);
    *reinterpret_cast<v4h *>(static_cast<_Float16 *>(out) + idx) = h;
  }
}

// ---- balanced schedule (shared by the attention and merge kernels)
// The work of KV head h, row block rb is `block_pages(rb)` page steps; the
// blocks are laid out head-major as one line of `total` steps, and the
// persistent work-group v takes steps [v*total/grid, (v+1)*total/grid).  A
// block split between work-groups is finished by the merge kernel from the
// partial states the pieces leave in the workspace: the piece of work-group v
// goes to slot 0 if v's range starts inside the block, else to slot 1.

__device__ __forceinline__ int block_pages(const PrefillArgs &a, int rb) {
  const int tok_hi = min(a.q_len - 1, (rb * a.rows + a.rows - 1) / 6);
  return (a.seq_len - a.q_len + tok_hi + 1 + 63) / 64;
}

// Block of one head that contains step sp (0 <= sp < tper), and the steps of
// the blocks before it.  Wave-uniform.
__device__ __forceinline__ void locate_block(const PrefillArgs &a, int sp, int lane, int &rb, int &before) {
  int base = 0;
  rb = a.nbh - 1;
  before = 0;
  for (int r0 = 0; r0 < a.nbh; r0 += 64) {
    const int r = r0 + lane;
    const int n = r < a.nbh ? block_pages(a, r) : 0;
    int incl = n;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(incl, d, 64);
      if (lane >= d) incl += y;
    }
    const uint64_t hit = __ballot(r < a.nbh && base + incl > sp);
    if (hit) {
      const int L = __builtin_ctzll(hit);
      rb = __builtin_amdgcn_readfirstlane(r0 + L);
      before = __builtin_amdgcn_readfirstlane(base + __shfl(incl - n, L, 64));
      return;
    }
    base += __shfl(incl, 63, 64);
  }
}

__device__ __forceinline__ int range_start(const PrefillArgs &a, int v) {
  return static_cast<int>(static_cast<int64_t>(v) * a.total / a.grid);
}
// Work-group whose range holds step s.
__device__ __forceinline__ int range_owner(const PrefillArgs &a, int s) {
  return static_cast<int>(((static_cast<int64_t>(s) + 1) * a.grid - 1) / a.total);
}

// One segment: pages [p_lo, p_hi) of row block rb of KV head h.  `part` is
// null when the segment is the whole block (the output is written directly).
template <int D>
__device__ __forceinline__ void run_segment(const PrefillArgs &a, char *smem, int h, int rb, int p_lo, int p_hi,
                                            float *part, int tid, int wave, int lane) {
  using T = Tile<D>;
  lds_t *stage_lds = (lds_t *)(smem + 2 * T::BUF);
  const char *stage = smem + 2 * T::BUF;
  const int nrows = a.q_len * 6;
  const int row0 = rb * T::ROWS;

  // ---- query fragments (B operand of S^T = K Q^T) and the row limit.
  // Lane (r, hh): query row r = lane % 32 of the wave's tile, dims 16*ds + 8*hh.
  const int hh = lane / 32, r32 = lane % 32;
  const int row = row0 + wave * 32 + r32;
  const bool row_valid = row < nrows;
  v8h qf[T::DS];
  int lim;
  {
    const int tok = row_valid ? row / 6 : 0;
    const int qh = h * 6 + (row_valid ? row % 6 : 0);
    // A padding row sees key 0 only, which keeps its softmax finite.
    lim = row_valid ? a.seq_len - a.q_len + tok + 1 : 1;
    const uint16_t *src = a.q + static_cast<int64_t>(tok) * a.q_tok_stride + static_cast<int64_t>(qh) * D + 8 * hh;
    if (a.q_bf16) {
#pragma unroll
      for (int ds = 0; ds < T::DS; ++ds) {
        const uint4 raw = row_valid ? *reinterpret_cast<const uint4 *>(src + 16 * ds) : make_uint4(0, 0, 0, 0);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          qf[ds][2 * e] = static_cast<_Float16>(__uint_as_float(w[e] << 16));
          qf[ds][2 * e + 1] = static_cast<_Float16>(__uint_as_float(w[e] & 0xFFFF0000u));
        }
      }
    } else {
#pragma unroll
      for (int ds = 0; ds < T::DS; ++ds) {
        const uint4 raw = row_valid ? *reinterpret_cast<const uint4 *>(src + 16 * ds) : make_uint4(0, 0, 0, 0);
        qf[ds] = __builtin_bit_cast(v8h, raw);
      }
    }
  }

  // Pages that need no causal mask for any row of the block.
  const int tok_lo = row0 / 6;
  const int full_pages = (a.seq_len - a.q_len + tok_lo + 1) / 64;

  v16f O[T::DT];
#pragma unroll
  for (int dt = 0; dt < T::DT; ++dt) O[dt] = (v16f)0.f;
  float m_run = -INFINITY, lsum = 0.f, corr = 0.f;

  // Per-lane LDS read bases.  K: key 32*mt + r32, dims 16*ds + 8*hh.  V^T:
  // dim 32*dt + r32, columns 16*s + 8*hh .. + 7 of the s-th 16-key step (keys
  // 16s + 4hh + i and 16s + 8 + 4hh + i); everything else is a compile-time
  // offset.
  const int k_base = r32 * T::KROW + 16 * hh;
  const int v_base = T::V_OFF + r32 * T::VROW + 16 * hh;

  stage_page<D>(a, p_lo, h, wave, lane, stage_lds, (lds_t *)(smem + T::S_OFF));
  wait_dma();
  __syncthreads();
  convert_page<D>(a, p_lo, stage, smem, tid);
  __syncthreads();

  for (int p = p_lo; p < p_hi; ++p) {
    const int bi = (p - p_lo) & 1;
    const char *buf = smem + bi * T::BUF;
    const bool more = p + 1 < p_hi;
    if (more) stage_page<D>(a, p + 1, h, wave, lane, stage_lds, (lds_t *)(smem + (bi ^ 1) * T::BUF + T::S_OFF));

    // ---- S^T = K Q^T - m for the 64 keys of page p: lane (r, hh) reg 4j+i
    // of tile mt holds key 32*mt + 8*j + 4*hh + i of row r.  The accumulators
    // start at -m (the row's running max, 0 before the first visible key), so
    // the exp2 argument needs no subtraction.  The two 32-key tiles
    // alternate, so consecutive MFMAs never wait on each other's accumulator.
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    v16f S[2] = {(v16f)(-m_use), (v16f)(-m_use)};
#pragma unroll
    for (int ds = 0; ds < T::DS; ++ds)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const v8h kf = *reinterpret_cast<const v8h *>(buf + k_base + 32 * mt * T::KROW + 32 * ds);
        S[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[ds], S[mt], 0, 0, 0);
      }

    // ---- scores (already scaled: the K tile carries k_scale * c, and offset
    // by -m_use), masks, lazy max
    const float *sc = reinterpret_cast<const float *>(buf + T::S_OFF);
    const bool masked = p >= full_pages;
    float mx = -INFINITY;
    // The causal mask touches only the last pages of a block: a uniform
    // branch, so the common pages carry no per-score compare and select.
    if (__builtin_expect(masked, 0)) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (p * 64 + 32 * mt + 8 * j + 4 * hh + i >= lim) S[mt][4 * j + i] = -INFINITY;
    }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, S[mt][e]);
    // A row's max passes the threshold exactly when one of its two lanes'
    // does, so the cross-lane max is only taken on a rescale.  Before the
    // first visible key (m = -inf) any finite score moves the max.
    const float thr = m_run == -INFINITY ? -INFINITY : kThreshold;
    if (__ballot(mx > thr)) {
      auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      const float rmx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) + m_use;
      const float mnew = fmaxf(m_run, rmx);
      const float alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - mnew);
      m_run = mnew;
      lsum *= alpha;
      corr *= alpha;
#pragma unroll
      for (int dt = 0; dt < T::DT; ++dt) O[dt] *= alpha;
      // Move the scores to the new max (a row still without a visible key
      // keeps m = -inf and offset 0).
      const float delta = m_run == -INFINITY ? 0.f : m_run - m_use;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) S[mt] -= delta;
    }

    // ---- P' = exp2(x - m) * v_scale as the fp16 B operand; row sums and zero-point terms.
    // A row with no visible key yet (a segment that starts inside the causal
    // tail) keeps m = -inf; its masked scores then give p = 0.
    v8h pb[4];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kb = 32 * mt + 8 * j + 4 * hh;
        const v4f vsc = *reinterpret_cast<const v4f *>(sc + 64 + kb);
        const v4f vzc = *reinterpret_cast<const v4f *>(sc + 128 + kb);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pr = __builtin_amdgcn_exp2f(S[mt][4 * j + i]);
          lsum += pr;
          const float pv = pr * vsc[i];
          corr = fmaf(pv, vzc[i], corr);
          pb[2 * mt + (j >> 1)][4 * (j & 1) + i] = static_cast<_Float16>(pv);
        }
      }

    // ---- O^T += V^T P'^T (16-key steps st = 2*mt + j/2; the DT output tiles
    // alternate, so consecutive MFMAs are independent)
    const char *vbase = buf + v_base;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
#pragma unroll
      for (int dt = 0; dt < T::DT; ++dt) {
        const int blk = 32 * dt * T::VROW + 32 * st;
        v8h vf;
        if constexpr (T::VROW % 16 == 0) {
          vf = *reinterpret_cast<const v8h *>(vbase + blk);
        } else {
          const uint2 lo = *reinterpret_cast<const uint2 *>(vbase + blk);
          const uint2 hi = *reinterpret_cast<const uint2 *>(vbase + blk + 8);
          vf = __builtin_bit_cast(v8h, make_uint4(lo.x, lo.y, hi.x, hi.y));
        }
        O[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pb[st], O[dt], 0, 0, 0);
      }
    }

    if (more) {
      wait_dma();
      __syncthreads();
      convert_page<D>(a, p + 1, stage, smem + (bi ^ 1) * T::BUF, tid);
    }
    __syncthreads();
  }

  // ---- finalize: O = (acc * 2^24|2^20 - corr) / l, written as [token][head][D]
  float l = lsum, cz = corr;
  {
    auto a1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
    l = __uint_as_float(a1[0]) + __uint_as_float(a1[1]);
    auto a2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(cz), __float_as_uint(cz), false, false);
    cz = __uint_as_float(a2[0]) + __uint_as_float(a2[1]);
  }
  if (part) {
    // Partial segment: O' = acc * 2^24|2^20 - corr (before the division), m, l.
    const int lr = wave * 32 + r32;
#pragma unroll
    for (int dt = 0; dt < T::DT; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v4f o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = O[dt][4 * j + i] * ((i & 1) ? 1048576.f : 16777216.f) - cz;
        *reinterpret_cast<v4f *>(part + lr * D + 32 * dt + 8 * j + 4 * hh) = o;
      }
    if (hh == 0) {
      part[T::ROWS * D + lr] = m_run;
      part[T::ROWS * D + T::ROWS + lr] = l;
    }
    return;
  }
  if (!row_valid) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const int tok = row / 6, qh = h * 6 + row % 6;
  const int64_t ob = static_cast<int64_t>(tok) * a.out_tok_stride + static_cast<int64_t>(qh) * D + 4 * hh;
#pragma unroll
  for (int dt = 0; dt < T::DT; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v4f o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = (O[dt][4 * j + i] * ((i & 1) ? 1048576.f : 16777216.f) - cz) * inv;
      store_out4(a.out, a.out_dtype, ob + 32 * dt + 8 * j, o);
    }
}

template <int D>
__global__ __attribute__((amdgpu_flat_work_group_size(Tile<D>::THREADS, Tile<D>::THREADS),
                          amdgpu_waves_per_eu(Tile<D>::WPE, Tile<D>::WPE))) void
prefill_kernel(PrefillArgs a) {
  using T = Tile<D>;
  __shared__ __attribute__((aligned(16))) char smem[2 * T::BUF + T::STAGE];
  const int w = blockIdx.x;
  const int v = a.xcd_perm ? (w % 8) * (a.grid / 8) + w / 8 : w;
  const int s0 = range_start(a, v), s1 = range_start(a, v + 1);
  if (s0 >= s1) return;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int lane = tid % 64;
  int s = s0;
  bool first = true;
  while (s < s1) {
    const int h = s / a.tper;
    int rb, before;
    locate_block(a, s - h * a.tper, lane, rb, before);
    const int n = block_pages(a, rb);
    const int p_lo = s - h * a.tper - before;
    const int p_hi = min(n, p_lo + (s1 - s));
    float *part = nullptr;
    if (p_lo != 0 || p_hi != n)
      part = a.ws + (static_cast<int64_t>(v) * 2 + (first ? 0 : 1)) * T::ROWS * (D + 2);
    run_segment<D>(a, smem, h, rb, p_lo, p_hi, part, tid, wave, lane);
    s += p_hi - p_lo;
    first = false;
  }
}

// Finishes the blocks split between work-groups: one work-group per block,
// two threads per row, D/2 dims each.
template <int D>
__global__ __launch_bounds__(2 * Tile<D>::ROWS) void prefill_merge_kernel(PrefillArgs a) {
  constexpr int R = Tile<D>::ROWS;
  const int b = blockIdx.x;
  const int h = b / a.nbh, rb = b % a.nbh;
  const int lane = threadIdx.x % 64;
  int start = 0;
  {
    // steps before block rb of head h
    int base = 0;
    for (int r0 = 0; r0 < rb; r0 += 64) {
      const int r = r0 + lane;
      int n = r < rb ? block_pages(a, r) : 0;
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) n += __shfl_xor(n, m, 64);
      base += n;
    }
    start = h * a.tper + base;
  }
  const int n = block_pages(a, rb);
  const int va = range_owner(a, start), vb = range_owner(a, start + n - 1);
  if (va == vb) return;  // one work-group did the whole block
  const int lr = threadIdx.x / 2, half = threadIdx.x % 2;
  const int row = rb * R + lr;
  if (row >= a.q_len * 6) return;
  float M = -INFINITY;
  for (int v = va; v <= vb; ++v) {
    const int slot = range_start(a, v) >= start ? 0 : 1;
    const float *pp = a.ws + (static_cast<int64_t>(v) * 2 + slot) * R * (D + 2);
    M = fmaxf(M, pp[R * D + lr]);
  }
  float l = 0.f;
  v4f o[D / 8];
#pragma unroll
  for (int e = 0; e < D / 8; ++e) o[e] = (v4f){0.f, 0.f, 0.f, 0.f};
  for (int v = va; v <= vb; ++v) {
    const int slot = range_start(a, v) >= start ? 0 : 1;
    const float *pp = a.ws + (static_cast<int64_t>(v) * 2 + slot) * R * (D + 2);
    const float m = pp[R * D + lr];
    if (m == -INFINITY) continue;
    const float wgt = __builtin_amdgcn_exp2f(m - M);
    l += wgt * pp[R * D + R + lr];
    const v4f *src = reinterpret_cast<const v4f *>(pp + lr * D + half * (D / 2));
#pragma unroll
    for (int e = 0; e < D / 8; ++e) o[e] += wgt * src[e];
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const int tok = row / 6, qh = h * 6 + row % 6;
  const int64_t ob = static_cast<int64_t>(tok) * a.out_tok_stride + static_cast<int64_t>(qh) * D + half * (D / 2);
#pragma unroll
  for (int e = 0; e < D / 8; ++e) store_out4(a.out, a.out_dtype, ob + 4 * e, o[e] * inv);
}

}  // namespace
}  // namespace k8v4

namespace k8v4 {
namespace {

struct PrefillPlan {
  int nbh, tper, total, grid;
};

// Host mirror of the device schedule; false if the call is too large for it.
int rows_per_block(int head_dim) { return head_dim == 128 ? Tile<128>::ROWS : Tile<256>::ROWS; }

bool plan_prefill(int64_t seq_len, int64_t q_len, int hkv, int head_dim, PrefillPlan &pl) {
  const int64_t R = rows_per_block(head_dim);
  const int64_t nbh = (q_len * kGqa + R - 1) / R;
  int64_t tper = 0;
  for (int64_t rb = 0; rb < nbh; ++rb) {
    const int64_t tok_hi = std::min<int64_t>(q_len - 1, (rb * R + R - 1) / 6);
    tper += (seq_len - q_len + tok_hi + 1 + 63) / 64;
  }
  const int64_t total = tper * hkv;
  if (nbh < 1 || total < 1 || total >= (int64_t(1) << 31) / 2) return false;
  int64_t grid = std::min<int64_t>(static_cast<int64_t>(device_cus()), total);  // one work-group per CU
  if (grid >= 8) grid -= grid % 8;
  pl.nbh = static_cast<int>(nbh);
  pl.tper = static_cast<int>(tper);
  pl.total = static_cast<int>(total);
  pl.grid = static_cast<int>(grid);
  return true;
}

int64_t partial_bytes(int grid, int head_dim) {
  return static_cast<int64_t>(grid) * 2 * rows_per_block(head_dim) * (head_dim + 2) * 4;
}

}  // namespace
}  // namespace k8v4

extern "C" int64_t k8v4_prefill_workspace_bytes(int64_t seq_len, int64_t q_len, int hkv, int head_dim) {
  using namespace k8v4;
  if (!supported_heads(hkv) || !supported_dim(head_dim) || q_len < 0 || q_len > seq_len) return -1;
  if (q_len == 0) return 0;
  PrefillPlan pl;
  if (!plan_prefill(seq_len, q_len, hkv, head_dim, pl)) return -1;
  return partial_bytes(pl.grid, head_dim);
}

extern "C" int k8v4_prefill_paged(const void *q, int q_dtype, int64_t q_tok_stride, const int8_t *k_cache,
                                  const float *k_scale, const uint8_t *v_cache, const float *v_scale,
                                  const float *v_zero, int64_t num_pages, int64_t k_page_stride,
                                  int64_t ks_page_stride, int64_t v_page_stride, int64_t vs_page_stride,
                                  int64_t vz_page_stride, const int32_t *block_row, int64_t table_width,
                                  int pages_per_block, int64_t seq_len, int64_t q_len, int hkv, int head_dim,
                                  float scale, void *out, int out_dtype, int64_t out_tok_stride,
                                  void *workspace, int64_t workspace_bytes, void *stream) {
  using namespace k8v4;
  clear_error();
  K8V4_REQUIRE(supported_heads(hkv), "unsupported per-GPU KV head count %d (this library serves 2 or 4)", hkv);
  K8V4_REQUIRE(supported_dim(head_dim), "unsupported head dim %d (this library serves 128 or 256)", head_dim);
  K8V4_REQUIRE(q_len >= 0 && seq_len >= 0 && seq_len < (int64_t(1) << 30), "bad lengths");
  K8V4_REQUIRE(q_len <= seq_len, "query longer than the KV sequence");
  if (q_len == 0) return K8V4_OK;
  K8V4_REQUIRE(pages_per_block >= 1, "pages_per_block");
  K8V4_REQUIRE(num_pages >= 1, "empty cache");
  K8V4_REQUIRE(table_width >= 1 && table_width * pages_per_block * kPage >= seq_len,
               "block table row covers %lld tokens, seq_len is %lld",
               static_cast<long long>(table_width * pages_per_block * kPage), static_cast<long long>(seq_len));
  K8V4_REQUIRE(q_dtype == K8V4_F16 || q_dtype == K8V4_BF16, "q dtype must be fp16 or bf16");
  K8V4_REQUIRE(out_dtype == K8V4_F16 || out_dtype == K8V4_BF16 || out_dtype == K8V4_F32,
               "out dtype must be fp16, bf16 or fp32");
  K8V4_REQUIRE(q && k_cache && k_scale && v_cache && v_scale && v_zero && block_row && out, "null pointer");
  K8V4_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 && q_tok_stride % 8 == 0,
               "q must be 16-byte aligned with a token stride that is a multiple of 8 elements");
  K8V4_REQUIRE(q_tok_stride >= int64_t(hkv) * kGqa * head_dim, "q token stride shorter than HQ*D");
  K8V4_REQUIRE(out_tok_stride >= int64_t(hkv) * kGqa * head_dim && out_tok_stride % 4 == 0,
               "out token stride must cover HQ*D and be a multiple of 4");
  K8V4_REQUIRE(reinterpret_cast<uintptr_t>(out) % 16 == 0, "out must be 16-byte aligned");
  K8V4_REQUIRE(reinterpret_cast<uintptr_t>(k_cache) % 16 == 0 && k_page_stride % 16 == 0,
               "k_cache must keep 16-byte aligned rows");
  K8V4_REQUIRE(reinterpret_cast<uintptr_t>(v_cache) % 8 == 0 && v_page_stride % 8 == 0,
               "v_cache must keep 8-byte aligned rows");
  K8V4_REQUIRE(reinterpret_cast<uintptr_t>(k_scale) % 4 == 0 && reinterpret_cast<uintptr_t>(v_scale) % 4 == 0 &&
                   reinterpret_cast<uintptr_t>(v_zero) % 4 == 0 && ks_page_stride % 4 == 0 &&
                   vs_page_stride % 4 == 0 && vz_page_stride % 4 == 0,
               "scale planes must be 4-byte aligned");
  K8V4_REQUIRE(scale > 0.f && scale < 1e30f, "softmax scale must be positive and finite");

  PrefillArgs a;
  a.q = static_cast<const uint16_t *>(q);
  a.q_tok_stride = q_tok_stride;
  a.q_bf16 = q_dtype == K8V4_BF16;
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
  a.block_row = block_row;
  a.ppb = pages_per_block;
  a.seq_len = static_cast<int>(seq_len);
  a.q_len = static_cast<int>(q_len);
  a.hkv = hkv;
  a.c = scale * 1.4426950408889634f;
  a.out = out;
  a.out_dtype = out_dtype;
  a.out_tok_stride = out_tok_stride;

  PrefillPlan pl;
  K8V4_REQUIRE(plan_prefill(seq_len, q_len, hkv, head_dim, pl), "prefill too large for one call (q_len %lld, seq_len %lld)",
               static_cast<long long>(q_len), static_cast<long long>(seq_len));
  const int64_t need = partial_bytes(pl.grid, head_dim);
  K8V4_REQUIRE(workspace && reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
               "prefill workspace must be a 16-byte aligned device buffer");
  if (workspace_bytes < need) {
    set_error("prefill workspace holds %lld bytes, the call needs %lld", static_cast<long long>(workspace_bytes),
              static_cast<long long>(need));
    return K8V4_ERR_WORKSPACE;
  }
  a.rows = rows_per_block(head_dim);
  a.nbh = pl.nbh;
  a.tper = pl.tper;
  a.total = pl.total;
  a.grid = pl.grid;
  a.xcd_perm = pl.grid % 8 == 0 ? 1 : 0;
  a.ws = static_cast<float *>(workspace);
  auto s = static_cast<hipStream_t>(stream);
  if (head_dim == 128)
    prefill_kernel<128><<<dim3(static_cast<unsigned>(pl.grid)), dim3(Tile<128>::THREADS), 0, s>>>(a);
  else
    prefill_kernel<256><<<dim3(static_cast<unsigned>(pl.grid)), dim3(Tile<256>::THREADS), 0, s>>>(a);
  const int rc = launch_status("k8v4_prefill_paged");
  if (rc) return rc;
  const dim3 mgrid(static_cast<unsigned>(pl.nbh * hkv));
  if (head_dim == 128)
    prefill_merge_kernel<128><<<mgrid, dim3(2 * Tile<128>::ROWS), 0, s>>>(a);
  else
    prefill_merge_kernel<256><<<mgrid, dim3(2 * Tile<256>::ROWS), 0, s>>>(a);
  return launch_status("k8v4_prefill_paged merge");
}
