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
//    that head once: direct-to-LDS loads stage coming pages' codes while the
//    current page is computed, and the group dequantizes them into a ring of
//    MFMA tiles.  Each page is a 64-key tile shared by all waves (all GQA rows)
//    of the group.
//  * S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16_f16 (the 32x32
//    shape needs half the operand reads per flop of the 16x16 one): the query
//    row is the MFMA column, so a lane pair owns one row's softmax state and
//    the score tile is already the B operand of the PV product.
//  * K codes become fp16 integers (byte permute into the mantissa of 1024.0,
//    then subtract 1152) times the token's K scale and the exp2-domain
//    softmax factor (one fp16 rounding, as a bf16/fp16 dequant has).
//  * Online softmax in the exp2 domain with a lazy rescale (the running max
//    only moves when a row's max grows by more than 2^2).
//  * Head dim 128 (run_segment_pp): eight waves in two groups that alternate
//    between matrix and vector work half a page apart, so each SIMD's matrix
//    core and vector ALU run side by side.  V is dequantized into the tile
//    ((nibble - v_zero) * v_scale / 16, one fp16 rounding) and the softmax
//    row sums come from the PV product itself (an extra MFMA against a ones
//    row), so the softmax is max, exp2 and one conversion per score.
//  * Head dim 256 (run_segment): four waves (the register file holds the wider
//    accumulators) that convert each page together, then multiply.  V
//    nibbles become exact fp16 subnormals (n * 2^-24 for even dims,
//    16 n * 2^-24 for odd dims) in a transposed tile, the V scale multiplies
//    P and the zero point is subtracted once per row at the end:
//      sum_t p_t (n_t - z_t) s_t = sum_t (p_t s_t) n_t - sum_t (p_t s_t) z_t.
#include "k8v4_common.h"

#include <algorithm>
#include <vector>

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
  int head0;     // KV head of step 0 (a launch covers heads head0 .. head0 + total / tper - 1)
  const char *tiles;  // dequantized tiles of head head0, [page][PP::BUF] (D = 128) or [page][Tile<256>::TBUF] bytes (null: convert in-kernel)
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
  // Tile images dequantized beforehand (D = 256): one per page in the
  // workspace, BUF rounded up to whole 1 KB pieces, each piece one DMA of a
  // wave; the ring then holds two such images.
  static constexpr int TBUF = (BUF + 1023) / 1024 * 1024;
  static constexpr int TPIECES = TBUF / 1024;
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
//
// PRE (D = 256): the pages' tile images were dequantized beforehand
// (prefill_convert256_kernel writes each page's image to a.tiles once for
// all row blocks of the head): the ring's two buffers (TBUF apart) receive
// them by DMA, and the waves only multiply.
template <int D, bool PRE = false>
__device__ __forceinline__ void run_segment(const PrefillArgs &a, char *smem, int h, int rb, int p_lo, int p_hi,
                                            float *part, int tid, int wave, int lane) {
  using T = Tile<D>;
  constexpr int RB = PRE ? T::TBUF : T::BUF;  // ring buffer stride
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

  // PRE: wave w moves pieces w, w + NW, ... of a page's image.
  auto tile_dma = [&](int p, int bi) {
    const char *src = a.tiles + static_cast<int64_t>(p) * T::TBUF + 16 * lane;
#pragma unroll
    for (int j = 0; j < (T::TPIECES + T::NW - 1) / T::NW; ++j) {
      const int k = T::NW * j + wave;
      if (k < T::TPIECES) dma16(src + 1024 * k, (lds_t *)(smem + bi * RB + 1024 * k));
    }
  };
  if constexpr (PRE) {
    tile_dma(p_lo, 0);
    wait_dma();
    __syncthreads();
  } else {
    stage_page<D>(a, p_lo, h, wave, lane, stage_lds, (lds_t *)(smem + T::S_OFF));
    wait_dma();
    __syncthreads();
    convert_page<D>(a, p_lo, stage, smem, tid);
    __syncthreads();
  }

  for (int p = p_lo; p < p_hi; ++p) {
    const int bi = (p - p_lo) & 1;
    const char *buf = smem + bi * RB;
    const bool more = p + 1 < p_hi;
    if (more) {
      if constexpr (PRE)
        tile_dma(p + 1, bi ^ 1);
      else
        stage_page<D>(a, p + 1, h, wave, lane, stage_lds, (lds_t *)(smem + (bi ^ 1) * T::BUF + T::S_OFF));
    }

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
      if constexpr (!PRE) {
        __syncthreads();
        convert_page<D>(a, p + 1, stage, smem + (bi ^ 1) * T::BUF, tid);
      }
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

// ---- D = 128: two wave groups in ping-pong ----
// The eight waves form two groups of four, waves w and w + 4 sharing a SIMD,
// and the groups run half a page apart: while one group's waves issue the
// matrix products of a page (the PV product of the previous page with its row
// sums and the QK product of the current one, 36 MFMAs per wave), the other
// group's waves on the same SIMDs run the vector work (softmax of the page
// they last multiplied, half of the dequantization of a coming page, and the
// DMAs).  A work-group barrier ends every phase, so each SIMD always holds one
// wave in each kind of work and the matrix core and the vector ALU run side by
// side.
//
// Phases t = 0, 1, ...: group 0 runs A(i) at t = 2i and B(i) at t = 2i + 1,
// group 1 runs B(i - 1) at t = 2i and A(i) at t = 2i + 1, where
//   A(i) = PV(i - 1), QK(i), then the LDS reads of this group's next
//          conversion (tile i + 1 + g: page i + 1 + g's staged codes);
//   B(i) = dequantize half g' = 1 - g of tile i + 1 + g into the ring (from
//          those registers), group 1 also issues the DMAs of page i + 5, then
//          softmax(i).
// Tile q lives in ring slot q % 3 (written at t = 2q - 2 and 2q - 1, last read
// by PV(q) at t = 2q + 3), staged page q in slot q % 4 of the staging ring
// (DMA issued at t = 2q - 8, complete by the end of t = 2q - 5: group 1 waits
// at the end of each A phase for all but the DMAs of its last B phase; read at
// the ends of t = 2q - 3 and 2q - 2).
struct PP {
  static constexpr int D = 128;
  static constexpr int NW = 8, THREADS = 512, ROWS = 256;
  static constexpr int DS = D / 16, DT = D / 32;
  static constexpr int KROW = 2 * D + 16;  // as Tile<128>
  static constexpr int V_OFF = 64 * KROW;
  static constexpr int VROW = 144;
  static constexpr int BUF = V_OFF + D * VROW;
  // Staging slot: K codes [64][D], V pieces [part][key parity][key pair] x 16 B,
  // k_scale | v_scale | v_zero planes (64 floats each).
  static constexpr int SV_OFF = 64 * D;
  static constexpr int SS_OFF = SV_OFF + 32 * D;
  static constexpr int STAGE = SS_OFF + 768;
  static constexpr int STAGE_OFF = 3 * BUF;
  static constexpr int LDS = STAGE_OFF + 4 * STAGE;
  static_assert(ROWS == Tile<128>::ROWS && THREADS == Tile<128>::THREADS, "one block shape per head dim");
  static_assert(LDS <= 160 * 1024, "LDS");
  static_assert(BUF % 16 == 0 && STAGE % 16 == 0, "16-byte aligned slots");
};

// The DMAs of this file's ping-pong path are inline assembly in the
// scalar-base form (a wave-uniform 64-bit base in SGPRs plus a 32-bit lane
// offset).  The compiler does not see them: it neither waits for them before
// unrelated LDS reads nor tracks them, so every wait on them is explicit.  The
// statement sets M0 (the LDS destination) itself and waits the states the
// load needs after a scalar write of M0 (1) and after a vector write of an
// SGPR it reads, such as a v_readfirstlane result in its base (5).
__device__ __forceinline__ uint32_t lds_addr(const lds_t *p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}
__device__ __forceinline__ void dma16s(const void *sbase, uint32_t voff, const lds_t *dst) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase),
               "s"(lds_addr(dst))
               : "memory", "m0");
}
__device__ __forceinline__ void dma4s(const void *sbase, uint32_t voff, const lds_t *dst) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase),
               "s"(lds_addr(dst))
               : "memory", "m0");
}
// Work-group barrier after this wave's LDS writes (a bare s_barrier:
// __syncthreads() would also wait for every DMA in flight).  One statement, so
// no LDS access can move across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Per-lane constants of one segment's staging and conversion.
struct PPLane {
  uint32_t k0, k1, v, s;  // DMA source offsets: K pieces wv and wv + 4, V piece wv, scale cell of key `lane`
  int kc_src, kc_dst;     // K conversion: staged chunk, tile byte offset
  int key;                // K conversion: key of the chunk
  int v_src, v_dst;       // V conversion: staged dword of the even key, tile byte offset of its first row
  int vkey;               // V conversion: the even key of the pair
};

__device__ __forceinline__ PPLane pp_lane(const PrefillArgs &a, int gt, int khalf, int vhalf, int lane) {
  constexpr int D = PP::D;
  PPLane L;
  const int wv = gt >> 6;  // wave within the group
  const int stride = a.hkv * D;
  L.k0 = static_cast<uint32_t>((8 * wv + (lane >> 3)) * stride + (lane & 7) * 16);
  L.k1 = L.k0 + static_cast<uint32_t>(32 * stride);
  L.v = static_cast<uint32_t>((2 * (lane & 31) + (lane >> 5)) * a.hkv * (D / 2) + wv * 16);
  L.s = static_cast<uint32_t>(lane * a.hkv * 4);
  // K: chunk c = 256 * khalf + gt holds dims 16 * (c % 8) .. + 15 of key c / 8.
  const int c = 256 * khalf + gt;
  L.key = c >> 3;
  L.kc_src = 16 * c;
  L.kc_dst = (c >> 3) * PP::KROW + 32 * (c & 7);
  // V: item gt of the half reads one dword (bytes 8 hv + 4 sub .. + 3 of
  // piece q, i.e. dims 32 q + 16 hv + 8 sub .. + 7) of the key pair's two
  // keys and writes those 8 V^T rows.
  const int pair = gt & 31, sub = (gt >> 5) & 1, hv = (gt >> 6) & 1, q = 2 * vhalf + (gt >> 7);
  L.v_src = PP::SV_OFF + (q * 64 + pair) * 16 + (2 * hv + sub) * 4;
  L.vkey = 2 * pair;
  const int kp = 2 * pair;  // even key; its column swaps bits 2 and 3
  const int col = (kp & ~12) | ((kp & 4) << 1) | ((kp & 8) >> 1);
  L.v_dst = PP::V_OFF + (32 * q + 16 * hv + 8 * sub) * PP::VROW + 2 * col;
  return L;
}

// DMAs of physical page phys into a staging slot, shared by the four waves of
// group 1 (wave wv: K pieces wv and wv + 4, V piece wv, and for wv < 3 the
// scale plane whose base and page stride the caller passes).
__device__ __forceinline__ void pp_stage(const PrefillArgs &a, int64_t phys, int h, int wv, const PPLane &L,
                                         const char *plane, int64_t plane_ps, lds_t *stage) {
  constexpr int D = PP::D;
  const char *kb = reinterpret_cast<const char *>(a.k_cache) + phys * a.k_ps + h * D;
  dma16s(kb, L.k0, stage + 1024 * wv);
  dma16s(kb, L.k1, stage + 1024 * (wv + 4));
  const char *vb = reinterpret_cast<const char *>(a.v_cache) + phys * a.v_ps + h * (D / 2);
  dma16s(vb, L.v, stage + PP::SV_OFF + 1024 * wv);
  if (wv < 3) dma4s(plane + phys * plane_ps + h * 4, L.s, stage + PP::SS_OFF + 256 * wv);
}

// One lane's inputs of a conversion, read from a staging slot ahead of use:
// a K chunk (16 codes and their key's k_scale) and a V item (one dword of the
// pair's even and odd key, their v_scale and v_zero).
struct PPKIn {
  uint4 k;
  float ks;
};
struct PPVIn {
  uint32_t ev, od;
  float2 vs, vz;
};

__device__ __forceinline__ PPKIn pp_fetch_k(const char *stage, int kc_src, int key) {
  PPKIn in;
  in.k = *reinterpret_cast<const uint4 *>(stage + kc_src);
  in.ks = reinterpret_cast<const float *>(stage + PP::SS_OFF)[key];
  return in;
}
__device__ __forceinline__ PPVIn pp_fetch_v(const char *stage, const PPLane &L) {
  PPVIn in;
  in.ev = *reinterpret_cast<const uint32_t *>(stage + L.v_src);
  in.od = *reinterpret_cast<const uint32_t *>(stage + L.v_src + 32 * 16);
  in.vs = *reinterpret_cast<const float2 *>(stage + PP::SS_OFF + 256 + 4 * L.vkey);
  in.vz = *reinterpret_cast<const float2 *>(stage + PP::SS_OFF + 512 + 4 * L.vkey);
  return in;
}

// Stores of a tile image: to LDS, or (NT) to the workspace with the
// nontemporal policy, which leaves no dirty lines in L2 for the end of the
// conversion kernel to write back (the next kernel reads the tiles through
// other XCDs' caches anyway).
template <bool NT, typename T>
__device__ __forceinline__ void tile_store(char *dst, T v) {
  if constexpr (NT)
    __builtin_nontemporal_store(v, reinterpret_cast<T *>(dst));
  else
    *reinterpret_cast<T *>(dst) = v;
}

// K chunk of tile page p: fp16 codes times k_scale * c (zero past the sequence).
template <bool NT = false>
__device__ __forceinline__ void pp_emit_k(const PrefillArgs &a, int p, const PPKIn &in, char *buf, int kc_dst, int key) {
  const float kc = p * 64 + key < a.seq_len ? in.ks * a.c : 0.f;
  const v2h kc2 = {static_cast<_Float16>(kc), static_cast<_Float16>(kc)};
  v2h h[8];
  k_codes_to_f16(in.k.x, h[0], h[1]);
  k_codes_to_f16(in.k.y, h[2], h[3]);
  k_codes_to_f16(in.k.z, h[4], h[5]);
  k_codes_to_f16(in.k.w, h[6], h[7]);
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] *= kc2;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  char *row = buf + kc_dst;
  tile_store<NT>(row, (u32x4){__builtin_bit_cast(uint32_t, h[0]), __builtin_bit_cast(uint32_t, h[1]),
                              __builtin_bit_cast(uint32_t, h[2]), __builtin_bit_cast(uint32_t, h[3])});
  tile_store<NT>(row + 16, (u32x4){__builtin_bit_cast(uint32_t, h[4]), __builtin_bit_cast(uint32_t, h[5]),
                                   __builtin_bit_cast(uint32_t, h[6]), __builtin_bit_cast(uint32_t, h[7])});
}

// V item of tile page p, dequantized: each V^T entry is (nibble - v_zero) *
// v_scale / 16 rounded once to fp16 (a mixed fma on the exact fp16 value
// 1024 + nibble, or 1024 + 16 * nibble for the high nibble, with float
// factors).  The 1/16 keeps every V row of fp16 range (and 16 times more) a
// finite fp16; the output multiplies it back.  Keys past the sequence become
// zeros.
template <bool NT = false>
__device__ __forceinline__ void pp_emit_v(const PrefillArgs &a, int p, const PPVIn &in, char *buf, const PPLane &L) {
  const bool live0 = p * 64 + L.vkey < a.seq_len, live1 = p * 64 + L.vkey + 1 < a.seq_len;
  const float s0 = live0 ? in.vs.x * 0.0625f : 0.f, s1 = live1 ? in.vs.y * 0.0625f : 0.f;
  const float z0 = live0 ? in.vz.x : 0.f, z1 = live1 ? in.vz.y : 0.f;
  const float se0 = s0, se1 = s1, ce0 = -(1024.f + z0) * s0, ce1 = -(1024.f + z1) * s1;
  const float so0 = s0 * 0.0625f, so1 = s1 * 0.0625f, co0 = -(64.f + z0) * s0, co1 = -(64.f + z1) * s1;
  char *vrow = buf + L.v_dst;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const uint32_t sel = 0x0C000C00u | ((4u + b) << 16) | b;
    const uint32_t x = __builtin_amdgcn_perm(in.od, in.ev, sel);  // byte b of both keys
    const v2h xe = __builtin_bit_cast(v2h, (x & kEvenNib) | 0x64006400u);  // 1024 + n
    const v2h xo = __builtin_bit_cast(v2h, (x & kOddNib) | 0x64006400u);   // 1024 + 16 n
    v2h ye, yo;
    ye[0] = static_cast<_Float16>(__builtin_fmaf(static_cast<float>(xe[0]), se0, ce0));
    ye[1] = static_cast<_Float16>(__builtin_fmaf(static_cast<float>(xe[1]), se1, ce1));
    yo[0] = static_cast<_Float16>(__builtin_fmaf(static_cast<float>(xo[0]), so0, co0));
    yo[1] = static_cast<_Float16>(__builtin_fmaf(static_cast<float>(xo[1]), so1, co1));
    tile_store<NT>(vrow + (2 * b) * PP::VROW, ye);
    tile_store<NT>(vrow + (2 * b + 1) * PP::VROW, yo);
  }
}

// One segment (pages [p_lo, p_hi) of row block rb of KV head h) on the
// ping-pong schedule.  Same contract as run_segment.
//
// PRE: the tiles were dequantized beforehand (prefill_convert_kernel writes
// each page's tile image to a.tiles once for all row blocks): the groups
// copy them straight into a four-slot ring with DMAs and the B phases hold
// only the softmax.  Tile q lives in slot q % 4; group 1 issues its pieces of
// tile q in B(q - 3) (t = 2q - 4) and waits for them at the end of A(q - 1),
// group 0 issues its pieces in B(q - 2) (t = 2q - 3) and waits at the end of
// B(q - 1); slot q % 4 was last read by PV(q - 4) at t = 2q - 5.
template <bool PRE>
__device__ __forceinline__ void run_segment_pp(const PrefillArgs &a, char *smem, int h, int rb, int p_lo, int p_hi,
                                               float *part, int tid, int wave, int lane) {
  constexpr int D = PP::D;
  const int g = wave >> 2;   // group
  const int gt = tid & 255;  // thread within the group
  const int wv = wave & 3;   // wave within the group
  const int n = p_hi - p_lo;
  const int nrows = a.q_len * 6;
  const int row0 = rb * PP::ROWS;
  lds_t *stage_lds = (lds_t *)(smem + PP::STAGE_OFF);
  const char *stage = smem + PP::STAGE_OFF;
  // Group g dequantizes half 1 - g of each tile (K chunks and V items).
  const PPLane L = pp_lane(a, gt, 1 - g, 1 - g, lane);
  // The scale plane this wave stages (group 1, waves 0-2 of the group).
  const char *plane = reinterpret_cast<const char *>(wv == 0 ? a.k_scale : wv == 1 ? a.v_scale : a.v_zero);
  const int64_t plane_ps = wv == 0 ? a.ks_ps : wv == 1 ? a.vs_ps : a.vz_ps;

  // ---- query fragments (B operand of S^T = K Q^T) and the row limit, as run_segment.
  const int hh = lane / 32, r32 = lane % 32;
  const int row = row0 + wave * 32 + r32;
  const bool row_valid = row < nrows;
  v8h qf[PP::DS];
  int lim;
  {
    const int tok = row_valid ? row / 6 : 0;
    const int qh = h * 6 + (row_valid ? row % 6 : 0);
    lim = row_valid ? a.seq_len - a.q_len + tok + 1 : 1;
    const uint16_t *src = a.q + static_cast<int64_t>(tok) * a.q_tok_stride + static_cast<int64_t>(qh) * D + 8 * hh;
    if (a.q_bf16) {
#pragma unroll
      for (int ds = 0; ds < PP::DS; ++ds) {
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
      for (int ds = 0; ds < PP::DS; ++ds) {
        const uint4 raw = row_valid ? *reinterpret_cast<const uint4 *>(src + 16 * ds) : make_uint4(0, 0, 0, 0);
        qf[ds] = __builtin_bit_cast(v8h, raw);
      }
    }
  }
  const int tok_lo = row0 / 6;
  const int full_pages = (a.seq_len - a.q_len + tok_lo + 1) / 64;

  v16f O[PP::DT];
#pragma unroll
  for (int dt = 0; dt < PP::DT; ++dt) O[dt] = (v16f)0.f;
  float m_run = -INFINITY;
  v16f S[2];
  v8h pb[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) pb[st] = (v8h)0;
  // Row sums on the matrix core: an A operand whose row 0 is all ones puts
  // sum_k P[k][r] in row 0 of Lacc (register 0 of lanes 0-31); its other rows
  // stay zero.
  // (PRE, where the matrix core is the busier unit: fp32 sums on the vector
  // ALU instead, two per lane, and the scores start from Minit = -m in the
  // first k-step's accumulator input, rewritten only when m moves.)
  v16f Lacc = (v16f)0.f;
  const v8h ones_a = (v8h)(r32 == 0 ? (_Float16)1.0f : (_Float16)0.0f);  // row 0 (lanes 0 and 32), all 16 keys
  float lsum0 = 0.f, lsum1 = 0.f;
  v16f Minit = (v16f)0.f;
  const int k_base = r32 * PP::KROW + 16 * hh;
  const int v_base = PP::V_OFF + r32 * PP::VROW + 16 * hh;
  PPKIn kin;  // inputs of this lane's next K chunk
  PPVIn vin;  // and of its next V item

  // DMA pieces of one tile (1 KB each, 35 per tile): piece k belongs to group
  // k % 2, wave (k / 2) % 4 of it.
  static_assert(PP::BUF % 1024 == 0 && 4 * PP::BUF <= PP::LDS, "tile pieces and four-slot ring");
  const char *tsrc = PRE ? a.tiles + static_cast<int64_t>(p_lo) * PP::BUF : nullptr;
  auto tile_dma = [&](int q) {
#pragma unroll
    for (int j = 0; j < 5; ++j) {
      const int k = 2 * (wv + 4 * j) + g;
      if (k < PP::BUF / 1024)
        dma16s(tsrc + static_cast<int64_t>(q) * PP::BUF, static_cast<uint32_t>(1024 * k + 16 * lane),
               (lds_t *)(smem + (q & 3) * PP::BUF + 1024 * k));
    }
  };
  // this wave's pieces per tile: 5 for (g, wv) = (0, 0), (0, 1), (1, 0), else 4
  const bool five = wv + g < 2;
  auto wait_older = [&]() {  // all but this wave's pieces of its last tile
    if (five)
      asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  };
  if constexpr (PRE) {
    tile_dma(0);
    if (n > 1) tile_dma(1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
  }

  // ---- prologue: pages 0-3 staged, tile 0 dequantized by both groups, group
  // 1's inputs for tile 1 fetched.
  if (!PRE && g == 1) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (q < n) pp_stage(a, page_of(a, p_lo + q), h, wv, L, plane, plane_ps, stage_lds + q * PP::STAGE);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  if constexpr (!PRE) {
    lds_barrier();
    pp_emit_k(a, p_lo, pp_fetch_k(stage, L.kc_src, L.key), smem, L.kc_dst, L.key);
    pp_emit_v(a, p_lo, pp_fetch_v(stage, L), smem, L);
    if (g == 1 && n > 1) {
      kin = pp_fetch_k(stage + PP::STAGE, L.kc_src, L.key);
      vin = pp_fetch_v(stage + PP::STAGE, L);
    }
    lds_barrier();
  }

  // Physical page of group 1's next DMA (looked up in its A phase, where the
  // scalar load's latency costs no vector work).
  int64_t next_phys = 0;

  // A(i): PV(i - 1) from tile slot (i - 1) % 3 with its row sums, then QK(i)
  // from slot i % 3, as one straight run of MFMAs with the operand reads
  // eight ahead.  Both products always run: PV(-1) multiplies a finite tile
  // (the ring starts zeroed) by a zero operand, and QK(n) fills scores that
  // are never read.  Then the inputs of the next conversion are read.
  auto phase_a = [&](int i, int slot_prev, int slot_cur) {
    // With the dequantization in the vector phase, the wave feeding the matrix
    // core wins issue conflicts with its SIMD's other wave (the vector work
    // fills the remaining issue slots); with pre-converted tiles the vector
    // phase is short and equal priority measures faster.
    if constexpr (!PRE) __builtin_amdgcn_s_setprio(3);
    if (!PRE && g == 1 && i + 5 < n) next_phys = page_of(a, p_lo + i + 5);
    const char *vbase = smem + slot_prev * PP::BUF + v_base;
    const char *kbase = smem + slot_cur * PP::BUF + k_base;
    // operand k: PV (st, dt) = (k / 4, k % 4) for k < 16, QK (ds, mt) = ((k - 16) / 2, k % 2) after
    auto frag = [&](int k) -> v8h {
      if (k < 16) return *reinterpret_cast<const v8h *>(vbase + 32 * (k & 3) * PP::VROW + 32 * (k >> 2));
      const int kk = k - 16;
      return *reinterpret_cast<const v8h *>(kbase + 32 * (kk & 1) * PP::KROW + 32 * (kk >> 1));
    };
    constexpr int AHEAD = PRE ? 12 : 6;  // operand reads in flight (register budget)
    v8h f[AHEAD];
#pragma unroll
    for (int k = 0; k < AHEAD; ++k) f[k] = frag(k);
    if constexpr (!PRE) {
      const float m_use = m_run == -INFINITY ? 0.f : m_run;
      S[0] = (v16f)(-m_use);
      S[1] = (v16f)(-m_use);
    }
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      if (k < 16) {
        O[k & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[k % AHEAD], pb[k >> 2], O[k & 3], 0, 0, 0);
        if (!PRE && (k & 3) == 3) Lacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ones_a, pb[k >> 2], Lacc, 0, 0, 0);
      } else {
        const int kk = k - 16;
        S[kk & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[k % AHEAD], qf[kk >> 1],
                                                           PRE && kk < 2 ? Minit : S[kk & 1], 0, 0, 0);
      }
      if (k + AHEAD < 32) f[k % AHEAD] = frag(k + AHEAD);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, AHEAD, 0);
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      if (!PRE && (k & 3) == 3 && k < 16)
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      else
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (k + AHEAD < 32) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if constexpr (PRE) {
      // Group 1's pieces of tile i + 1 land before the barrier (all but those
      // of tile i + 2, issued in its last B phase; vector loads complete in
      // issue order).
      if (g == 1) {
        if (i + 2 < n)
          wait_older();
        else
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      return;
    }
    // Group 1's DMAs older than its last B phase's (page i + 4 and before)
    // land before the barrier (vector loads complete in issue order); group 0
    // has none in flight.
    if (g == 1 && i + 4 < n) {
      if (wv < 3)
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    // Inputs of this group's conversion in B(i): tile i + 1 + g.
    const int ct = i + 1 + g;
    if (ct < n) {
      const char *st = stage + (ct & 3) * PP::STAGE;
      kin = pp_fetch_k(st, L.kc_src, L.key);
      vin = pp_fetch_v(st, L);
    }
  };

  // Softmax of page i: P = exp2(x - m) as the fp16 B operand of the PV
  // product (whose ones row also sums these same fp16 values).
  auto softmax = [&](int i) {
    const int p = p_lo + i;
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    if (__builtin_expect(p >= full_pages, 0)) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (p * 64 + 32 * mt + 8 * j + 4 * hh + e >= lim) S[mt][4 * j + e] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, S[mt][e]);
    const float thr = m_run == -INFINITY ? -INFINITY : kThreshold;
    if (__ballot(mx > thr)) {
      auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      const float rmx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) + m_use;
      const float mnew = fmaxf(m_run, rmx);
      const float alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - mnew);
      m_run = mnew;
      if constexpr (PRE) {
        lsum0 *= alpha;
        lsum1 *= alpha;
        Minit = (v16f)(-m_run);
      } else {
        Lacc[0] *= alpha;
      }
#pragma unroll
      for (int dt = 0; dt < PP::DT; ++dt) O[dt] *= alpha;
      const float delta = m_run == -INFINITY ? 0.f : m_run - m_use;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) S[mt] -= delta;
    }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pr = __builtin_amdgcn_exp2f(S[mt][4 * j + e]);
          if constexpr (PRE) {
            if (e & 1)
              lsum1 += pr;
            else
              lsum0 += pr;
          }
          pb[2 * mt + (j >> 1)][4 * (j & 1) + e] = static_cast<_Float16>(pr);
        }
  };

  // B(i): this group's half of tile i + 1 + g from the fetched inputs, group
  // 1's DMAs of page i + 5 (four per wave, three in the fourth), then softmax(i).
  auto phase_b = [&](int i) {
    __builtin_amdgcn_s_setprio(0);
    if constexpr (PRE) {
      // Softmax, then this wave's pieces of tile i + 3 (group 1) or i + 2
      // (group 0); group 0 then waits for its pieces of tile i + 1.
      if (i >= 0 && i < n) softmax(i);
      const int q = i + 2 + g;
      if (q < n) tile_dma(q);
      if (g == 0) {
        if (q < n)
          wait_older();
        else
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      return;
    }
    const int ct = i + 1 + g;
    if (ct < n) {
      char *buf = smem + (ct % 3) * PP::BUF;
      pp_emit_k(a, p_lo + ct, kin, buf, L.kc_dst, L.key);
      pp_emit_v(a, p_lo + ct, vin, buf, L);
    }
    if (g == 1 && i + 5 < n) pp_stage(a, next_phys, h, wv, L, plane, plane_ps, stage_lds + ((i + 5) & 3) * PP::STAGE);
    if (i >= 0 && i < n) softmax(i);
  };

  // Group 1 starts half a page late: its B(-1) converts and stages only.
  if (g == 1) {
    if (!PRE && n > 4) next_phys = page_of(a, p_lo + 4);
    phase_b(-1);
    lds_barrier();
  }
  // slot = i % 3 for page i; slot_m1 = (i - 1) % 3.
  int slot = 0, slot_m1 = 2;
  for (int i = 0; i <= n; ++i) {
    if constexpr (PRE)
      phase_a(i, (i - 1) & 3, i & 3);
    else
      phase_a(i, slot_m1, slot);
    lds_barrier();
    // Group 1's B(n) would be empty; skipping it keeps both groups at 2n + 2 barriers.
    if (g == 0 || i < n) {
      phase_b(i);
      lds_barrier();
    }
    slot_m1 = slot;
    slot = slot == 2 ? 0 : slot + 1;
  }

  __builtin_amdgcn_s_setprio(0);
  // ---- finalize: O = 16 acc / l (row sums from lane r32's Lacc[0]; V^T holds V / 16).
  float l;
  if constexpr (PRE) {
    l = lsum0 + lsum1;
    auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
    l = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  } else {
    auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(Lacc[0]), __float_as_uint(Lacc[0]), false, false);
    l = hh == 0 ? Lacc[0] : __uint_as_float(sw[0]);
  }
  if (part) {
    const int lr = wave * 32 + r32;
#pragma unroll
    for (int dt = 0; dt < PP::DT; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v4f o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = 16.f * O[dt][4 * j + e];
        *reinterpret_cast<v4f *>(part + lr * D + 32 * dt + 8 * j + 4 * hh) = o;
      }
    if (hh == 0) {
      part[PP::ROWS * D + lr] = m_run;
      part[PP::ROWS * D + PP::ROWS + lr] = l;
    }
    return;
  }
  if (!row_valid) return;
  const float inv = l > 0.f ? 16.f / l : 0.f;
  const int tok = row / 6, qh = h * 6 + row % 6;
  const int64_t ob = static_cast<int64_t>(tok) * a.out_tok_stride + static_cast<int64_t>(qh) * D + 4 * hh;
#pragma unroll
  for (int dt = 0; dt < PP::DT; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v4f o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = O[dt][4 * j + e] * inv;
      store_out4(a.out, a.out_dtype, ob + 32 * dt + 8 * j, o);
    }
}

template <int D, bool PRE>
__global__ __attribute__((amdgpu_flat_work_group_size(Tile<D>::THREADS, Tile<D>::THREADS),
                          amdgpu_waves_per_eu(Tile<D>::WPE, Tile<D>::WPE))) void
prefill_kernel(PrefillArgs a) {
  using T = Tile<D>;
  constexpr int LDS_BYTES = D == 128 ? PP::LDS : (PRE ? 2 * T::TBUF : 2 * T::BUF + T::STAGE);
  __shared__ __attribute__((aligned(16))) char smem[LDS_BYTES];
  const int w = blockIdx.x;
  const int v = a.xcd_perm ? (w % 8) * (a.grid / 8) + w / 8 : w;
  const int s0 = range_start(a, v), s1 = range_start(a, v + 1);
  if (s0 >= s1) return;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int lane = tid % 64;
  if constexpr (D == 128) {
    // The ping-pong ring starts zeroed: its tiles then only ever hold finite values.
    for (int o = 16 * tid; o < 4 * PP::BUF; o += 16 * PP::THREADS) *reinterpret_cast<uint4 *>(smem + o) = make_uint4(0, 0, 0, 0);
  }
  int s = s0;
  bool first = true;
  while (s < s1) {
    const int hl = s / a.tper;
    const int h = a.head0 + hl;
    int rb, before;
    locate_block(a, s - hl * a.tper, lane, rb, before);
    const int n = block_pages(a, rb);
    const int p_lo = s - hl * a.tper - before;
    const int p_hi = min(n, p_lo + (s1 - s));
    float *part = nullptr;
    if (p_lo != 0 || p_hi != n)
      part = a.ws + (static_cast<int64_t>(v) * 2 + (first ? 0 : 1)) * T::ROWS * (D + 2);
    if constexpr (D == 128)
      run_segment_pp<PRE>(a, smem, h, rb, p_lo, p_hi, part, tid, wave, lane);
    else
      run_segment<D, PRE>(a, smem, h, rb, p_lo, p_hi, part, tid, wave, lane);
    s += p_hi - p_lo;
    first = false;
  }
}

// Dequantizes every page of KV head h once into its tile image (the LDS
// layout of run_segment_pp's ring): one work-group of 256 threads per page.
// The page's V codes and scale planes are staged in LDS with coalesced loads
// in the order the in-kernel conversion stages them; then each thread
// dequantizes two K chunks (read directly) and two V items with the same
// arithmetic as the in-kernel conversion.
__global__ __launch_bounds__(256) void prefill_convert_kernel(PrefillArgs a, char *tiles, int h) {
  constexpr int D = PP::D;
  __shared__ __attribute__((aligned(16))) char st[PP::STAGE];
  const int p = blockIdx.x, t = threadIdx.x;
  const int64_t phys = page_of(a, p);
  char *buf = tiles + static_cast<int64_t>(p) * PP::BUF;
  const char *kb = reinterpret_cast<const char *>(a.k_cache) + phys * a.k_ps + h * D;
  const char *vb = reinterpret_cast<const char *>(a.v_cache) + phys * a.v_ps + h * (D / 2);
  const int64_t krow = static_cast<int64_t>(a.hkv) * D, vrow = static_cast<int64_t>(a.hkv) * (D / 2);
  {
    // V piece q (16 bytes) of key 2 * pair + parity -> [q][parity][pair]
    const int key = t >> 2, q = t & 3;
    *reinterpret_cast<uint4 *>(st + PP::SV_OFF + (q * 64 + (key & 1) * 32 + (key >> 1)) * 16) =
        *reinterpret_cast<const uint4 *>(vb + key * vrow + 16 * q);
    if (t < 192) {
      const int plane = t >> 6, k = t & 63;
      const float *src = plane == 0 ? a.k_scale : plane == 1 ? a.v_scale : a.v_zero;
      const int64_t ps = plane == 0 ? a.ks_ps : plane == 1 ? a.vs_ps : a.vz_ps;
      reinterpret_cast<float *>(st + PP::SS_OFF)[t] =
          *reinterpret_cast<const float *>(reinterpret_cast<const char *>(src) + phys * ps + (static_cast<int64_t>(k) * a.hkv + h) * 4);
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int c = t + 256 * r;
    const int key = c >> 3, part = c & 7;
    PPKIn in;
    in.k = *reinterpret_cast<const uint4 *>(kb + key * krow + 16 * part);
    in.ks = reinterpret_cast<const float *>(st + PP::SS_OFF)[key];
    pp_emit_k<true>(a, p, in, buf, key * PP::KROW + 32 * part, key);
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const PPLane L = pp_lane(a, t, 0, r, 0);
    pp_emit_v<true>(a, p, pp_fetch_v(st, L), buf, L);
  }
}

// D = 256: every page of KV head h dequantized once into its tile image (the
// LDS layout run_segment multiplies from), one work-group of four waves per
// page: the page is staged and converted exactly as the attention kernel
// does in place, then the image leaves LDS with nontemporal 16-byte stores
// (TBUF bytes: the tail past BUF carries staged codes nothing reads).
__global__ __launch_bounds__(256) void prefill_convert256_kernel(PrefillArgs a, char *tiles, int h) {
  using T = Tile<256>;
  static_assert(T::THREADS == 256 && T::TBUF <= T::BUF + T::STAGE, "one page per work-group of four waves");
  __shared__ __attribute__((aligned(16))) char smem[T::BUF + T::STAGE];
  const int p = blockIdx.x, tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
  stage_page<256>(a, p, h, wave, lane, (lds_t *)(smem + T::BUF), (lds_t *)(smem + T::S_OFF));
  wait_dma();
  __syncthreads();
  convert_page<256>(a, p, smem + T::BUF, smem, tid);
  __syncthreads();
  char *dst = tiles + static_cast<int64_t>(p) * T::TBUF;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  for (int o = 16 * tid; o < T::TBUF; o += 16 * T::THREADS)
    tile_store<true>(dst + o, *reinterpret_cast<const u32x4 *>(smem + o));
}

// Finishes the blocks split between work-groups: kMergeSplit work-groups of
// kMergeThreads per block (a launch then fills the chip), kMergeTPR<D>
// threads per row, 32 dims each.  The pieces are folded in one pass with an
// online rescale, their states loaded kMergeU at a time (all loads of a
// round in flight together: the merge is a chain of round trips, not a
// bandwidth problem).
constexpr int kMergeSplit = 8;
constexpr int kMergeThreads = 128;
constexpr int kMergeU = 4;
template <int D>
constexpr int kMergeTPR = kMergeThreads * kMergeSplit / Tile<D>::ROWS;

// Steps of row blocks 0 .. rb - 1 of one KV head (wave-uniform).
__device__ __forceinline__ int steps_before_block(const PrefillArgs &a, int rb, int lane) {
  int base = 0;
  for (int r0 = 0; r0 < rb; r0 += 64) {
    const int r = r0 + lane;
    base += wave_sum(r < rb ? block_pages(a, r) : 0);
  }
  return base;
}

// Merges row block rb of KV head h (one sequence's fields in `sa`) whose
// steps start at `start` of the launch's step line, if work-groups split it;
// `a` holds the launch's schedule (total, grid) and workspace.
template <int D>
__device__ __forceinline__ void merge_block(const PrefillArgs &a, const PrefillArgs &sa, int h, int rb, int start,
                                            int part) {
  constexpr int R = Tile<D>::ROWS, TPR = kMergeTPR<D>, DT = D / TPR;  // DT = 32 dims per thread
  static_assert(DT == 32, "32 dims per merge thread");
  const int n = block_pages(sa, rb);
  const int va = range_owner(a, start), vb = range_owner(a, start + n - 1);
  if (va == vb) return;  // one work-group did the whole block
  const int lr = part * (R / kMergeSplit) + threadIdx.x / TPR, sub = threadIdx.x % TPR;
  const int row = rb * R + lr;
  if (row >= sa.q_len * 6) return;
  float M = -INFINITY, l = 0.f;
  v4f o[DT / 4];
#pragma unroll
  for (int e = 0; e < DT / 4; ++e) o[e] = (v4f){0.f, 0.f, 0.f, 0.f};
  for (int v0 = va; v0 <= vb; v0 += kMergeU) {
    // This round's pieces (past vb: the last piece again, dropped below).
    float mu[kMergeU], lu[kMergeU];
    v4f ou[kMergeU][DT / 4];
#pragma unroll
    for (int u = 0; u < kMergeU; ++u) {
      const int v = min(v0 + u, vb);
      const int slot = range_start(a, v) >= start ? 0 : 1;
      const float *pp = a.ws + (static_cast<int64_t>(v) * 2 + slot) * R * (D + 2);
      mu[u] = pp[R * D + lr];
      lu[u] = pp[R * D + R + lr];
      const v4f *src = reinterpret_cast<const v4f *>(pp + lr * D + sub * DT);
#pragma unroll
      for (int e = 0; e < DT / 4; ++e) ou[u][e] = src[e];
    }
    float Mn = M;
#pragma unroll
    for (int u = 0; u < kMergeU; ++u) {
      if (v0 + u > vb) mu[u] = -INFINITY;
      Mn = fmaxf(Mn, mu[u]);
    }
    if (Mn == -INFINITY) continue;  // no key seen yet by this row
    const float keep = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - Mn);
    l *= keep;
#pragma unroll
    for (int e = 0; e < DT / 4; ++e) o[e] *= keep;
#pragma unroll
    for (int u = 0; u < kMergeU; ++u) {
      // A piece that saw no key of this row (m = -inf) and the repeats past
      // vb are selected away, not multiplied by zero.
      const bool on = mu[u] != -INFINITY;
      const float wgt = __builtin_amdgcn_exp2f(mu[u] - Mn);
      l = on ? l + wgt * lu[u] : l;
#pragma unroll
      for (int e = 0; e < DT / 4; ++e) o[e] = on ? o[e] + wgt * ou[u][e] : o[e];
    }
    M = Mn;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const int tok = row / 6, qh = h * 6 + row % 6;
  const int64_t ob = static_cast<int64_t>(tok) * sa.out_tok_stride + static_cast<int64_t>(qh) * D + sub * DT;
#pragma unroll
  for (int e = 0; e < DT / 4; ++e) store_out4(sa.out, sa.out_dtype, ob + 4 * e, o[e] * inv);
}

template <int D>
__global__ __launch_bounds__(kMergeThreads) void prefill_merge_kernel(PrefillArgs a) {
  const int b = blockIdx.x / kMergeSplit;
  const int hl = b / a.nbh, rb = b % a.nbh;
  const int start = hl * a.tper + steps_before_block(a, rb, threadIdx.x % 64);
  merge_block<D>(a, a, a.head0 + hl, rb, start, blockIdx.x % kMergeSplit);
}

// ---- several sequences in one launch (the short chunks of one step)
// Their (KV head, row block) work is laid out sequence after sequence as one
// line of page steps (each sequence head-major, as above) that the persistent
// work-groups share out as for one sequence; blocks are numbered the same way
// for the merge.  The kernel argument holds one complete PrefillArgs per
// sequence (its rows of q and out, lengths, block-table row; the schedule
// fields of the launch are in every one), and a segment reads its
// sequence's through a reference into the kernel-argument segment at a
// wave-uniform offset: scalar loads on demand, as the one-sequence kernels
// read theirs (a copy in registers would not fit beside the kernels' own).
constexpr int kBatchMax = 10;
struct PrefillBatchArgs {
  PrefillArgs seq[kBatchMax];  // must stay the first member: read at kernarg offset i * sizeof(PrefillArgs)
  int n;                       // sequences of this launch
  int step0[kBatchMax + 1];    // first page step of sequence i; step0[n] = the launch's total
  int block0[kBatchMax + 1];   // first (KV head, row block) of sequence i; block0[n] = blocks of the launch
};

__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Sequence holding item x of an increasing prefix line off[0..n] (wave-uniform;
// constant indices only: a runtime index into the by-value argument would copy
// it to private memory).
__device__ __forceinline__ int batch_find(const int (&off)[kBatchMax + 1], int n, int x) {
  int i = 0;
#pragma unroll
  for (int k = 1; k < kBatchMax; ++k)
    if (k < n && off[k] <= x) i = k;
  return uni(i);
}
__device__ __forceinline__ int batch_off(const int (&off)[kBatchMax + 1], int i) {
  int v = off[0];
#pragma unroll
  for (int k = 1; k <= kBatchMax; ++k)
    if (i == k) v = off[k];
  return uni(v);
}

// Sequence i's arguments, in place in the kernel-argument segment.
__device__ __forceinline__ const PrefillArgs &batch_seq(int i) {
  typedef const __attribute__((address_space(4))) PrefillArgs const_args;
  const_args *base = (const_args *)__builtin_amdgcn_kernarg_segment_ptr();
  return *(const PrefillArgs *)(base + i);
}

template <int D>
__global__ __attribute__((amdgpu_flat_work_group_size(Tile<D>::THREADS, Tile<D>::THREADS),
                          amdgpu_waves_per_eu(Tile<D>::WPE, Tile<D>::WPE))) void
prefill_batch_kernel(PrefillBatchArgs ba) {
  using T = Tile<D>;
  constexpr int LDS_BYTES = D == 128 ? PP::LDS : 2 * T::BUF + T::STAGE;
  __shared__ __attribute__((aligned(16))) char smem[LDS_BYTES];
  const PrefillArgs &a = ba.seq[0];  // the launch's schedule
  const int w = blockIdx.x;
  const int v = a.xcd_perm ? (w % 8) * (a.grid / 8) + w / 8 : w;
  const int s0 = range_start(a, v), s1 = range_start(a, v + 1);
  if (s0 >= s1) return;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int lane = tid % 64;
  if constexpr (D == 128) {
    for (int o = 16 * tid; o < 4 * PP::BUF; o += 16 * PP::THREADS) *reinterpret_cast<uint4 *>(smem + o) = make_uint4(0, 0, 0, 0);
  }
  int s = s0;
  bool first = true;
  while (s < s1) {
    const int i = batch_find(ba.step0, ba.n, s);
    const PrefillArgs &sa = batch_seq(i);
    const int sl = s - batch_off(ba.step0, i);  // step within the sequence
    const int h = sl / sa.tper;
    int rb, before;
    locate_block(sa, sl - h * sa.tper, lane, rb, before);
    const int n = block_pages(sa, rb);
    const int p_lo = sl - h * sa.tper - before;
    const int p_hi = min(n, p_lo + (s1 - s));
    float *part = nullptr;
    if (p_lo != 0 || p_hi != n) part = a.ws + (static_cast<int64_t>(v) * 2 + (first ? 0 : 1)) * T::ROWS * (D + 2);
    if constexpr (D == 128)
      run_segment_pp<false>(sa, smem, h, rb, p_lo, p_hi, part, tid, wave, lane);
    else
      run_segment<D>(sa, smem, h, rb, p_lo, p_hi, part, tid, wave, lane);
    s += p_hi - p_lo;
    first = false;
  }
}

template <int D>
__global__ __launch_bounds__(kMergeThreads) void prefill_batch_merge_kernel(PrefillBatchArgs ba) {
  const int b = blockIdx.x / kMergeSplit;
  const int i = batch_find(ba.block0, ba.n, b);
  const PrefillArgs &sa = batch_seq(i);
  const int local = b - batch_off(ba.block0, i);
  const int h = local / sa.nbh, rb = local % sa.nbh;
  const int start = batch_off(ba.step0, i) + h * sa.tper + steps_before_block(sa, rb, threadIdx.x % 64);
  merge_block<D>(ba.seq[0], sa, h, rb, start, blockIdx.x % kMergeSplit);
}

}  // namespace
}  // namespace k8v4

namespace k8v4 {
namespace {

struct PrefillPlan {
  int nbh, tper, total, grid;
  bool tiles;  // pages dequantized once per KV head into tile images
};

// Fewest page steps per persistent work-group when a call has few (one
// 64-token chunk over 2,000 keys: 8 such calls 741 -> 339 us with 4 instead
// of 1; 8 gave no more).
constexpr int64_t kMinSteps = 4;

int rows_per_block(int head_dim) { return head_dim == 128 ? Tile<128>::ROWS : Tile<256>::ROWS; }

// Head dim 128 dequantizes each page once per KV head into the workspace when
// that work is shared by at least this many row blocks (below it the
// in-kernel conversion costs less than the extra tile traffic).
constexpr int kPreMinBlocks = 4;

// Head dim 256 (one wave per SIMD, whose conversion is cheaper in place): per
// KV head the tile path costs about 59 us of launches and pre-pass latency
// plus 62 ns per page and saves about 9 ns per (row block, page) -- measured
// against the in-place conversion over contexts of 4K-64K tokens and chunks
// of 96-4,224 tokens (two heads; per head either way).
bool tiles_pay_off(int64_t nbh, int64_t npages, int head_dim) {
  if (nbh < kPreMinBlocks) return false;
  return head_dim == 128 || (9 * nbh - 62) * npages > 58600;
}

bool use_tiles(const PrefillPlan &pl, int /*head_dim*/) { return pl.tiles; }
int64_t tile_stride(int head_dim) { return head_dim == 128 ? PP::BUF : Tile<256>::TBUF; }

// Persistent work-groups for a launch of `steps` page steps: one per CU, each
// with at least kMinSteps steps (a work-group's fixed work -- its query rows,
// its partial state, the merge's reads of it -- outweighs a page or two of
// attention), a multiple of 8 from 8 up (whole XCDs).
int64_t persistent_grid(int64_t steps) {
  int64_t grid = std::min<int64_t>(static_cast<int64_t>(device_cus()), std::max<int64_t>(1, steps / kMinSteps));
  if (grid >= 8) grid -= grid % 8;
  return grid;
}

// Host mirror of the device schedule; false if the call is too large for it.
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
  pl.nbh = static_cast<int>(nbh);
  pl.tper = static_cast<int>(tper);
  pl.total = static_cast<int>(total);
  pl.tiles = tiles_pay_off(nbh, (seq_len + kPage - 1) / kPage, head_dim);
  // The grid of the launch that runs: one per KV head over its tper steps
  // with tile images, else one over all heads.
  pl.grid = static_cast<int>(persistent_grid(use_tiles(pl, head_dim) ? tper : total));
  return true;
}

int64_t partial_bytes(int grid, int head_dim) {
  return static_cast<int64_t>(grid) * 2 * rows_per_block(head_dim) * (head_dim + 2) * 4;
}

// Workspace: partial states, then (tiles) one head's tile images, 256-byte aligned.
int64_t tiles_offset(const PrefillPlan &pl, int head_dim) { return (partial_bytes(pl.grid, head_dim) + 255) / 256 * 256; }
int64_t workspace_need(const PrefillPlan &pl, int64_t seq_len, int head_dim) {
  if (!use_tiles(pl, head_dim)) return partial_bytes(pl.grid, head_dim);
  return tiles_offset(pl, head_dim) + (seq_len + kPage - 1) / kPage * tile_stride(head_dim);
}


// Argument checks shared by the single-sequence and batched prefill entries.
int check_prefill_args(const void *q, int q_dtype, int64_t q_tok_stride, const int8_t *k_cache, const float *k_scale,
                       const uint8_t *v_cache, const float *v_scale, const float *v_zero, int64_t k_page_stride,
                       int64_t ks_page_stride, int64_t v_page_stride, int64_t vs_page_stride,
                       int64_t vz_page_stride, const int32_t *block_row, int hkv, int head_dim, float scale,
                       const void *out, int out_dtype, int64_t out_tok_stride) {
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
  return K8V4_OK;
}

// Fills the launch arguments every prefill launch shares.
PrefillArgs prefill_base_args(const void *q, int q_dtype, int64_t q_tok_stride, const int8_t *k_cache,
                              const float *k_scale, const uint8_t *v_cache, const float *v_scale,
                              const float *v_zero, int64_t num_pages, int64_t k_page_stride,
                              int64_t ks_page_stride, int64_t v_page_stride, int64_t vs_page_stride,
                              int64_t vz_page_stride, const int32_t *block_row, int pages_per_block, int hkv,
                              float scale, void *out, int out_dtype, int64_t out_tok_stride) {
  PrefillArgs a{};
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
  a.hkv = hkv;
  a.c = scale * 1.4426950408889634f;
  a.out = out;
  a.out_dtype = out_dtype;
  a.out_tok_stride = out_tok_stride;
  return a;
}
}  // namespace
}  // namespace k8v4

extern "C" int64_t k8v4_prefill_workspace_bytes(int64_t seq_len, int64_t q_len, int hkv, int head_dim) {
  using namespace k8v4;
  if (!supported_heads(hkv) || !supported_dim(head_dim) || q_len < 0 || q_len > seq_len) return -1;
  if (q_len == 0) return 0;
  PrefillPlan pl;
  if (!plan_prefill(seq_len, q_len, hkv, head_dim, pl)) return -1;
  return workspace_need(pl, seq_len, head_dim);
}

extern "C" int k8v4_prefill_uses_tiles(int64_t seq_len, int64_t q_len, int hkv, int head_dim) {
  using namespace k8v4;
  if (!supported_heads(hkv) || !supported_dim(head_dim) || q_len < 0 || q_len > seq_len) return -1;
  if (q_len == 0) return 0;
  PrefillPlan pl;
  if (!plan_prefill(seq_len, q_len, hkv, head_dim, pl)) return -1;
  return use_tiles(pl, head_dim) ? 1 : 0;
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
  {
    const int rc = check_prefill_args(q, q_dtype, q_tok_stride, k_cache, k_scale, v_cache, v_scale, v_zero,
                                      k_page_stride, ks_page_stride, v_page_stride, vs_page_stride, vz_page_stride,
                                      block_row, hkv, head_dim, scale, out, out_dtype, out_tok_stride);
    if (rc) return rc;
  }

  PrefillArgs a = prefill_base_args(q, q_dtype, q_tok_stride, k_cache, k_scale, v_cache, v_scale, v_zero, num_pages,
                                    k_page_stride, ks_page_stride, v_page_stride, vs_page_stride, vz_page_stride,
                                    block_row, pages_per_block, hkv, scale, out, out_dtype, out_tok_stride);
  a.seq_len = static_cast<int>(seq_len);
  a.q_len = static_cast<int>(q_len);

  PrefillPlan pl;
  K8V4_REQUIRE(plan_prefill(seq_len, q_len, hkv, head_dim, pl), "prefill too large for one call (q_len %lld, seq_len %lld)",
               static_cast<long long>(q_len), static_cast<long long>(seq_len));
  const int64_t need = workspace_need(pl, seq_len, head_dim);
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
  a.head0 = 0;
  a.tiles = nullptr;
  auto s = static_cast<hipStream_t>(stream);
  if (use_tiles(pl, head_dim)) {
    // One KV head at a time: its pages dequantized once into the workspace,
    // then all row blocks of the head over them, then their merge.
    char *tiles = static_cast<char *>(workspace) + tiles_offset(pl, head_dim);
    const unsigned npages = static_cast<unsigned>((seq_len + kPage - 1) / kPage);
    a.total = pl.tper;
    a.tiles = tiles;
    for (int h = 0; h < hkv; ++h) {
      a.head0 = h;
      if (head_dim == 128) {
        prefill_convert_kernel<<<dim3(npages), dim3(256), 0, s>>>(a, tiles, h);
        prefill_kernel<128, true><<<dim3(static_cast<unsigned>(a.grid)), dim3(PP::THREADS), 0, s>>>(a);
        prefill_merge_kernel<128><<<dim3(static_cast<unsigned>(pl.nbh * kMergeSplit)), dim3(kMergeThreads), 0, s>>>(a);
      } else {
        prefill_convert256_kernel<<<dim3(npages), dim3(256), 0, s>>>(a, tiles, h);
        prefill_kernel<256, true><<<dim3(static_cast<unsigned>(a.grid)), dim3(Tile<256>::THREADS), 0, s>>>(a);
        prefill_merge_kernel<256><<<dim3(static_cast<unsigned>(pl.nbh * kMergeSplit)), dim3(kMergeThreads), 0, s>>>(a);
      }
      const int rc = launch_status("k8v4_prefill_paged");
      if (rc) return rc;
    }
    return K8V4_OK;
  }
  if (head_dim == 128)
    prefill_kernel<128, false><<<dim3(static_cast<unsigned>(pl.grid)), dim3(Tile<128>::THREADS), 0, s>>>(a);
  else
    prefill_kernel<256, false><<<dim3(static_cast<unsigned>(pl.grid)), dim3(Tile<256>::THREADS), 0, s>>>(a);
  const int rc = launch_status("k8v4_prefill_paged");
  if (rc) return rc;
  const dim3 mgrid(static_cast<unsigned>(pl.nbh * hkv * kMergeSplit));
  if (head_dim == 128)
    prefill_merge_kernel<128><<<mgrid, dim3(kMergeThreads), 0, s>>>(a);
  else
    prefill_merge_kernel<256><<<mgrid, dim3(kMergeThreads), 0, s>>>(a);
  return launch_status("k8v4_prefill_paged merge");
}

extern "C" int64_t k8v4_prefill_batch_workspace_bytes(int hkv, int head_dim) {
  using namespace k8v4;
  if (!supported_heads(hkv) || !supported_dim(head_dim)) return -1;
  return partial_bytes(device_cus(), head_dim);
}

extern "C" int k8v4_prefill_paged_batch(const void *q, int q_dtype, int64_t q_tok_stride, const int8_t *k_cache,
                                        const float *k_scale, const uint8_t *v_cache, const float *v_scale,
                                        const float *v_zero, int64_t num_pages, int64_t k_page_stride,
                                        int64_t ks_page_stride, int64_t v_page_stride, int64_t vs_page_stride,
                                        int64_t vz_page_stride, const int32_t *block_table, int64_t bt_stride,
                                        int64_t table_width, int pages_per_block, int nseq, const int64_t *tok0,
                                        const int64_t *q_lens, const int64_t *seq_lens, const int64_t *rows,
                                        int hkv, int head_dim, float scale, void *out, int out_dtype,
                                        int64_t out_tok_stride, void *workspace, int64_t workspace_bytes,
                                        void *stream) {
  using namespace k8v4;
  clear_error();
  K8V4_REQUIRE(supported_heads(hkv), "unsupported per-GPU KV head count %d (this library serves 2 or 4)", hkv);
  K8V4_REQUIRE(supported_dim(head_dim), "unsupported head dim %d (this library serves 128 or 256)", head_dim);
  K8V4_REQUIRE(nseq >= 0, "negative sequence count");
  if (nseq == 0) return K8V4_OK;
  K8V4_REQUIRE(tok0 && q_lens && seq_lens && rows, "null pointer");
  K8V4_REQUIRE(pages_per_block >= 1, "pages_per_block");
  K8V4_REQUIRE(num_pages >= 1, "empty cache");
  K8V4_REQUIRE(table_width >= 1 && bt_stride >= table_width, "block table row stride shorter than its width");
  {
    const int rc = check_prefill_args(q, q_dtype, q_tok_stride, k_cache, k_scale, v_cache, v_scale, v_zero,
                                      k_page_stride, ks_page_stride, v_page_stride, vs_page_stride, vz_page_stride,
                                      block_table, hkv, head_dim, scale, out, out_dtype, out_tok_stride);
    if (rc) return rc;
  }
  for (int i = 0; i < nseq; ++i) {
    K8V4_REQUIRE(q_lens[i] >= 0 && seq_lens[i] >= 0 && seq_lens[i] < (int64_t(1) << 30),
                 "sequence %d: bad lengths", i);
    K8V4_REQUIRE(q_lens[i] <= seq_lens[i], "sequence %d: query longer than the KV sequence", i);
    K8V4_REQUIRE(tok0[i] >= 0 && rows[i] >= 0, "sequence %d: negative token offset or table row", i);
    K8V4_REQUIRE(table_width * pages_per_block * kPage >= seq_lens[i],
                 "sequence %d: block table row covers %lld tokens, seq_len is %lld", i,
                 static_cast<long long>(table_width * pages_per_block * kPage), static_cast<long long>(seq_lens[i]));
  }
  const int64_t need = partial_bytes(device_cus(), head_dim);
  K8V4_REQUIRE(workspace && reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
               "prefill workspace must be a 16-byte aligned device buffer");
  if (workspace_bytes < need) {
    set_error("prefill workspace holds %lld bytes, the call needs %lld", static_cast<long long>(workspace_bytes),
              static_cast<long long>(need));
    return K8V4_ERR_WORKSPACE;
  }
  PrefillArgs a = prefill_base_args(q, q_dtype, q_tok_stride, k_cache, k_scale, v_cache, v_scale, v_zero, num_pages,
                                    k_page_stride, ks_page_stride, v_page_stride, vs_page_stride, vz_page_stride,
                                    block_table, pages_per_block, hkv, scale, out, out_dtype, out_tok_stride);
  a.rows = rows_per_block(head_dim);
  a.ws = static_cast<float *>(workspace);
  a.head0 = 0;
  a.tiles = nullptr;
  auto s = static_cast<hipStream_t>(stream);
  // Launches of up to kBatchMax non-empty sequences each, one after another
  // on the stream (each launch reuses the workspace after the previous one).
  // All of them are planned and checked before the first is enqueued, so a
  // rejected call launches nothing.
  const int ob = out_dtype == K8V4_F32 ? 4 : 2;
  std::vector<PrefillBatchArgs> launches;
  std::vector<int64_t> merge_blocks;
  int i = 0;
  while (i < nseq) {
    PrefillBatchArgs ba{};
    int64_t steps = 0, blocks = 0;
    for (; i < nseq && ba.n < kBatchMax; ++i) {
      if (q_lens[i] == 0) continue;
      PrefillPlan pl;
      K8V4_REQUIRE(plan_prefill(seq_lens[i], q_lens[i], hkv, head_dim, pl),
                   "sequence %d too large for one call (q_len %lld, seq_len %lld)", i,
                   static_cast<long long>(q_lens[i]), static_cast<long long>(seq_lens[i]));
      const int k = ba.n++;
      PrefillArgs &sa = ba.seq[k];
      sa = a;
      sa.q = a.q + tok0[i] * q_tok_stride;
      sa.out = static_cast<char *>(out) + tok0[i] * out_tok_stride * ob;
      sa.block_row = block_table + rows[i] * bt_stride;
      sa.q_len = static_cast<int>(q_lens[i]);
      sa.seq_len = static_cast<int>(seq_lens[i]);
      sa.nbh = pl.nbh;
      sa.tper = pl.tper;
      ba.step0[k] = static_cast<int>(steps);
      ba.block0[k] = static_cast<int>(blocks);
      steps += pl.total;
      blocks += static_cast<int64_t>(pl.nbh) * hkv;
      K8V4_REQUIRE(steps < (int64_t(1) << 30) && blocks * kMergeSplit < (int64_t(1) << 30),
                   "prefill batch too large for one launch");
    }
    if (ba.n == 0) break;
    ba.step0[ba.n] = static_cast<int>(steps);
    ba.block0[ba.n] = static_cast<int>(blocks);
    const int64_t grid = persistent_grid(steps);
    for (int k = 0; k < ba.n; ++k) {
      ba.seq[k].total = static_cast<int>(steps);
      ba.seq[k].grid = static_cast<int>(grid);
      ba.seq[k].xcd_perm = grid % 8 == 0 ? 1 : 0;
    }
    launches.push_back(ba);
    merge_blocks.push_back(blocks);
  }
  for (size_t j = 0; j < launches.size(); ++j) {
    const PrefillBatchArgs &ba = launches[j];
    const dim3 grid(static_cast<unsigned>(ba.seq[0].grid));
    const dim3 mgrid(static_cast<unsigned>(merge_blocks[j] * kMergeSplit));
    if (head_dim == 128) {
      prefill_batch_kernel<128><<<grid, dim3(Tile<128>::THREADS), 0, s>>>(ba);
      prefill_batch_merge_kernel<128><<<mgrid, dim3(kMergeThreads), 0, s>>>(ba);
    } else {
      prefill_batch_kernel<256><<<grid, dim3(Tile<256>::THREADS), 0, s>>>(ba);
      prefill_batch_merge_kernel<256><<<mgrid, dim3(kMergeThreads), 0, s>>>(ba);
    }
    const int rc = launch_status("k8v4_prefill_paged_batch");
    if (rc) return rc;
  }
  return K8V4_OK;
}
