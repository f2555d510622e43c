// Paged decode / MTP-verify attention over the int8-K / int4-V cache.
//
// Reference semantics: k8v4_v030/oracle.py:100-163 (int8-quantized Q, exact
// integer QK dot, fp softmax, V dequantized as (nibble - zero) * scale) and
// the batch op k8v4_v030/native/xe2_kv_ops.cpp:1728-1775 with its stage-1
// masking (:657-791) and stage-2 merge guards (:1086-1166).
//
// MI355X design (not a translation of the reference's per-page stage 1 +
// per-row stage 2):
//  * One launch covers the whole batch.  The grid is a fixed number G of
//    split-K work-groups (about one per CU); every work-group derives, from
//    the device-resident lengths, the same balanced plan: all live pages of
//    all sequences are cut into runs of P pages that never straddle a
//    sequence, so a batch of 4 x 128K and a batch of {2K, 32K, 128K, 200K}
//    both fill the chip.  No host read of the lengths: graph-capturable.
//  * A work-group holds two waves per KV head (one per half-head with four
//    256-dim heads), two per SIMD.  The waves of a head share the 6*q_len
//    query rows of their head (int8-quantized in the prologue, padded to
//    16-row tiles) as MFMA operands in LDS, so each K/V byte is fetched from
//    HBM once and used for every GQA row.  With up to three tiles the two
//    waves take alternate chunks; with four (q_len 9-10) each takes two
//    tiles and both multiply every chunk, shared between their rings.
//  * Each wave owns a ring of LDS slots filled by direct-to-LDS loads
//    (global_load_lds, nontemporal for K and V): one slot is one 32-token
//    chunk of its head (K rows with XOR-swizzled 16-byte chunks, V rows in a
//    rotated order, the three scale planes), so the next chunks stream in
//    without holding registers and every operand read is conflict-free.
//  * Per chunk: QK^T on v_mfma_i32_16x16x64_i8 computed transposed (tokens x
//    rows) so the score tile lands in the operand layout of the P.V MFMA;
//    online softmax in the exp2 domain with a lazy rescale; V nibbles are used
//    as fp16 subnormal operands straight from the packed bytes (n * 2^-24 and
//    16 n * 2^-24 after one AND), the V scale multiplies P and the zero point
//    is one extra MFMA per tile (sum_t p_t s_t z_t), removed at the end;
//    P.V and the row sums on v_mfma_f32_16x16x32_f16 with fp32 accumulation.
//  * Each split writes (m, l, O / l in fp16) for its live rows only; a small
//    merge kernel combines the splits of each output row.
//  * Head dim 256 runs as paired halves: the cache's rows are read as those
//    of a 128-dim cache with twice the heads, two waves per SIMD; the two
//    waves of a pair score each chunk over both of their K slots and each
//    accumulates its own 128 output dims (a 256-dim wave needs all 512
//    registers of a SIMD lane, so one wave per SIMD, latency-bound).  Its
//    query is quantized by a small kernel ahead of the split kernel, once for
//    all work-groups.  Every split-kernel instance is 128-dim.
#include "k8v4_common.h"

#include <cfloat>
#include <mutex>

namespace k8v4 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kScoreBias = 0x4B400000;  // bits of 1.5 * 2^23
// Lazy-rescale threshold (log2 units): the running max m moves only when a
// score passes it by more than 4, so exp2(score - m) <= 16.  P is carried as
// exp2(score - m - 2), a quarter of the probability (row sums and outputs
// shrink alike, so their ratio is unchanged), and is multiplied by the
// token's V scale in fp16: a V row spanning the whole fp16 range has scale
// 2 * 65504 / 15, and 16 / 4 * 2 * 65504 / 15 = 34,936 stays finite.
constexpr float kRescaleThreshold = 4.0f;
constexpr float kPLog2Offset = 2.0f;

struct DecodeArgs {
  const uint16_t *q;
  int64_t q_tok_stride;  // elements; head stride is head_dim
  int q_bf16;
  // Pre-quantized query instead of q (nullable): per sequence an int8 tile
  // [hkv][64][head_dim] (row r of head h is token r / 6, query head
  // h * 6 + r % 6) and fp32 scales [hkv][64], the reference's Q-once layout.
  const int8_t *q8;
  const float *q8_scale;
  int64_t q8_seq_stride, qs_seq_stride;  // elements between sequences
  const int8_t *k_cache;
  const float *k_scale;
  const uint8_t *v_cache;
  const float *v_scale;
  const float *v_zero;
  int64_t num_pages;
  int64_t k_ps, ks_ps, v_ps, vs_ps, vz_ps;  // page strides, bytes
  const int32_t *block_table;
  int64_t bt_stride;  // elements between table rows
  int table_width;
  int ppb;
  const int32_t *seq_lens;
  // The scale planes share one page stride and lie within 2^30 bytes of
  // each other: their gathers then use the scalar-base form, with
  // d_kv = v_scale - k_scale and d_vz = v_zero - v_scale in bytes.
  int planes_fast;
  int64_t d_kv, d_vz;
  const int32_t *visible;  // nullable, [batch][vis_stride]
  int64_t vis_stride;
  int batch;
  int q_len;
  int hkv;
  char *ws;
  int64_t split_bytes;  // bytes of one split's state
  int grid;              // number of split work-groups (the plan's G)
  int min_pages;
  int merge_cs;   // column slices per output row in the merge
  int tile0;      // first 16-row query tile of this split launch (four 256-dim heads, four tiles: three, then one)
  int units;      // merge units: output rows x merge_cs
  void *out;
  int out_dtype;
  int64_t out_tok_stride;  // elements
};

// ---------------------------------------------------------------- planning
// Every work-group of both kernels evaluates the same plan from device data.

__device__ __forceinline__ int seq_len0(const DecodeArgs &a, int b) {
  return a.visible ? a.visible[static_cast<int64_t>(b) * a.vis_stride] : a.seq_lens[b];
}

__device__ __forceinline__ int seq_pages(const DecodeArgs &a, int b) {
  const int L0 = seq_len0(a, b);
  if (L0 <= 0) return 0;
  const int64_t cap = static_cast<int64_t>(a.table_width) * a.ppb;
  const int64_t n = (static_cast<int64_t>(L0) + kPage - 1) / kPage;
  return static_cast<int>(n < cap ? n : cap);
}

// Pages per split for this batch (same value in every lane and work-group).
__device__ int plan_pages_per_split(const DecodeArgs &a, int lane) {
  int total = 0, maxn = 0;
  for (int b0 = 0; b0 < a.batch; b0 += kWave) {
    const int b = b0 + lane;
    const int n = b < a.batch ? seq_pages(a, b) : 0;
    total += n;
    maxn = max(maxn, n);
  }
  total = wave_sum(total);
  maxn = wave_max(maxn);
  int P = a.grid > a.batch ? (total + (a.grid - a.batch) - 1) / (a.grid - a.batch) : maxn;
  P = max(P, a.min_pages);
  return __builtin_amdgcn_readfirstlane(max(P, 1));
}

// Split index range [first, first + count) of sequence b, or the sequence
// owning split w.  Sequences take ceil(pages / P) consecutive splits.
struct SplitRange {
  int b;
  int first;
  int count;
};

__device__ SplitRange plan_locate(const DecodeArgs &a, int P, int lane, int want_b, int want_w) {
  SplitRange r{-1, 0, 0};
  int base = 0;
  for (int b0 = 0; b0 < a.batch; b0 += kWave) {
    const int b = b0 + lane;
    const int n = b < a.batch ? seq_pages(a, b) : 0;
    const int s = (n + P - 1) / P;
    const int incl = wave_inclusive_scan(s);
    const int excl = base + incl - s;
    bool hit;
    if (want_b >= 0)
      hit = b == want_b;
    else
      hit = (s > 0) && (want_w >= excl) && (want_w < excl + s);
    const uint64_t mask = __ballot(hit);
    if (mask) {
      const int src = __builtin_ctzll(mask);
      // The results are wave-uniform; readfirstlane keeps them in SGPRs.
      r.b = __builtin_amdgcn_readfirstlane(b0 + src);
      r.first = __builtin_amdgcn_readlane(excl, src);
      r.count = __builtin_amdgcn_readlane(s, src);
      return r;
    }
    base += __builtin_amdgcn_readlane(incl, kWave - 1);
  }
  return r;
}

// The split kernel's view of the plan in one pass over the lengths when the
// batch fits one wave (the common case): pages per split P, the split range
// of work-group wg, and that sequence's page count and length.
struct SplitPlan {
  SplitRange r;
  int P;
  int npages;
  int L0;
};

__device__ SplitPlan plan_split(const DecodeArgs &a, int lane, int wg) {
  SplitPlan sp;
  if (a.batch > kWave) {
    sp.P = plan_pages_per_split(a, lane);
    sp.r = plan_locate(a, sp.P, lane, -1, wg);
    sp.npages = sp.r.b >= 0 ? seq_pages(a, sp.r.b) : 0;
    sp.L0 = sp.r.b >= 0 ? seq_len0(a, sp.r.b) : 0;
    return sp;
  }
  const int L = lane < a.batch ? seq_len0(a, lane) : 0;
  int n = 0;
  if (L > 0) {
    const int64_t cap = static_cast<int64_t>(a.table_width) * a.ppb;
    const int64_t np = (static_cast<int64_t>(L) + kPage - 1) / kPage;
    n = static_cast<int>(np < cap ? np : cap);
  }
  const int total = wave_sum(n), maxn = wave_max(n);
  int P = a.grid > a.batch ? (total + (a.grid - a.batch) - 1) / (a.grid - a.batch) : maxn;
  P = __builtin_amdgcn_readfirstlane(max(max(P, a.min_pages), 1));
  const int s = (n + P - 1) / P;
  const int excl = wave_inclusive_scan(s) - s;
  const uint64_t mask = __ballot(s > 0 && wg >= excl && wg < excl + s);
  sp.P = P;
  sp.r = SplitRange{-1, 0, 0};
  sp.npages = 0;
  sp.L0 = 0;
  if (mask) {
    const int src = __builtin_ctzll(mask);
    sp.r.b = __builtin_amdgcn_readfirstlane(src);
    sp.r.first = __builtin_amdgcn_readlane(excl, src);
    sp.r.count = __builtin_amdgcn_readlane(s, src);
    sp.npages = __builtin_amdgcn_readlane(n, src);
    sp.L0 = __builtin_amdgcn_readlane(L, src);
  }
  return sp;
}

// The merge's view of the plan: the split range of sequence want_b, in one
// pass over the lengths when the batch fits one wave (one round trip, not
// one for the pages per split and another for the scan).
__device__ SplitRange plan_sequence(const DecodeArgs &a, int lane, int want_b) {
  if (a.batch > kWave) return plan_locate(a, plan_pages_per_split(a, lane), lane, want_b, -1);
  const int n = lane < a.batch ? seq_pages(a, lane) : 0;
  const int total = wave_sum(n), maxn = wave_max(n);
  int P = a.grid > a.batch ? (total + (a.grid - a.batch) - 1) / (a.grid - a.batch) : maxn;
  P = __builtin_amdgcn_readfirstlane(max(max(P, a.min_pages), 1));
  const int s = (n + P - 1) / P;
  const int excl = wave_inclusive_scan(s) - s;
  SplitRange r;
  r.b = want_b;
  r.first = __builtin_amdgcn_readlane(excl, want_b);
  r.count = __builtin_amdgcn_readlane(s, want_b);
  return r;
}

// Block-table reads go through the constant address space: the table is
// read-only for the kernel's lifetime, so a uniform lookup becomes a scalar
// load and never waits on the vector-memory counter the LDS DMA uses.
typedef const __attribute__((address_space(4))) int32_t *const_i32_ptr;

__device__ __forceinline__ int physical_page(const DecodeArgs &a, const int32_t *bt_row, int p) {
  const const_i32_ptr row = (const_i32_ptr)(bt_row);
  if (a.ppb <= 1) return row[p];
  return row[p / a.ppb] * a.ppb + (p % a.ppb);
}

// ------------------------------------------------------------ merge
// The splits of one sequence are combined per output row (token, query
// head): a merge unit is one column slice of one row, VPR = D / 8 / merge_cs
// columns of 8 dims (at least 8 columns: 128-byte state lines are never
// shared between units), folded over the sequence's split states by the TPU
// threads (128 or 256) of one work-group.  Thread t owns column t % VPR and
// the splits t / VPR + k * SPI (SPI = TPU / VPR); it loads the (m, l, O) of
// up to MU of its splits at once and folds them online (running max,
// rescaled sums), one round trip per MU splits (the host picks TPU and
// merge_cs so that one round covers the average sequence).  The threads of a
// column are then combined with the same rescaling: within a wave by lane
// exchanges, across the waves through a few LDS words.

constexpr int kMergeMU = 8;  // splits loaded together by one merge thread

__device__ __forceinline__ void store_out(void *out, int dtype, int64_t idx, float v) {
  if (dtype == K8V4_F32)
    static_cast<float *>(out)[idx] = v;
  else if (dtype == K8V4_BF16)
    static_cast<__bf16 *>(out)[idx] = static_cast<__bf16>(v);
  else
    static_cast<_Float16 *>(out)[idx] = static_cast<_Float16>(v);
}

typedef float v8f __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// Where one merge unit's row lives.
struct MergeRow {
  int b, tok, qh, r, h, slice;
};
__device__ __forceinline__ MergeRow merge_row(const DecodeArgs &a, int unit) {
  MergeRow m;
  const int hq = kGqa * a.hkv;
  const int row_id = unit / a.merge_cs;
  m.slice = unit - row_id * a.merge_cs;
  m.qh = row_id % hq;
  m.tok = row_id / hq;  // b * q_len + j
  m.b = m.tok / a.q_len;
  m.h = m.qh / kGqa;
  m.r = (m.tok - m.b * a.q_len) * kGqa + (m.qh - m.h * kGqa);
  return m;
}

// Running (max, sum, output) of one column, folded online.
struct MergeAcc {
  float M, l;
  v8f o;
};

// One round of a merge thread: the (m, l, O) of its splits s = s0 + u * SPI
// (u < kMergeMU) below `limit`, others empty.
struct MergeRound {
  float ms[kMergeMU], ls[kMergeMU];
  v8f os[kMergeMU];
};

// Byte offsets of a unit's column inside one split state (layout written by
// the split kernel: O [hkv][rows][D] fp16, then (m, l) [hkv][rows] fp32 pairs).
struct MergeOffsets {
  int64_t o, ml;
};
template <int D>
__device__ __forceinline__ MergeOffsets merge_offsets(const DecodeArgs &a, const MergeRow &mr, int col, int VPR) {
  const int rows = a.q_len * kGqa;
  const int dcol = 8 * (mr.slice * VPR + col);
  MergeOffsets o;
  o.o = (static_cast<int64_t>(mr.h * rows + mr.r) * D + dcol) * 2;
  o.ml = static_cast<int64_t>(a.hkv) * rows * D * 2 + (mr.h * rows + mr.r) * 8;
  return o;
}

__device__ __forceinline__ void merge_load(const DecodeArgs &a, const MergeOffsets &off, const char *ws, int s0,
                                           int SPI, int limit, MergeRound &rd) {
  // All loads are issued before any is used: a split past `limit` reads the
  // state of split limit - 1 (a live one) and is masked afterwards, so no
  // load sits behind a per-split branch that would wait for it.
  const bool any = s0 < limit;
  v8h raw[kMergeMU] = {};
  float2 ml[kMergeMU] = {};
  if (any) {
#pragma unroll
    for (int u = 0; u < kMergeMU; ++u) {
      const char *st = ws + static_cast<int64_t>(min(s0 + u * SPI, limit - 1)) * a.split_bytes;
      ml[u] = *reinterpret_cast<const float2 *>(st + off.ml);
      raw[u] = *reinterpret_cast<const v8h *>(st + off.o);
    }
  }
#pragma unroll
  for (int u = 0; u < kMergeMU; ++u) {
    const bool live = s0 + u * SPI < limit;
    rd.ms[u] = live ? ml[u].x : -INFINITY;
    rd.ls[u] = live ? ml[u].y : 0.f;
    rd.os[u] = live ? __builtin_convertvector(raw[u], v8f) : (v8f){0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  }
}

__device__ __forceinline__ void merge_fold_round(MergeAcc &acc, const MergeRound &rd) {
  float mn = acc.M;
#pragma unroll
  for (int u = 0; u < kMergeMU; ++u) mn = fmaxf(mn, rd.ms[u]);
  if (mn != -INFINITY) {
    const float c = acc.M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(acc.M - mn);
    acc.l *= c;
    acc.o *= c;
#pragma unroll
    for (int u = 0; u < kMergeMU; ++u) {
      const float w = rd.ms[u] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(rd.ms[u] - mn) * rd.ls[u];
      acc.l += w;
      acc.o += (4.f * w) * rd.os[u];  // the states hold a quarter of the split's output
    }
    acc.M = mn;
  }
}

// Folds this thread's splits (sg, sg + SPI, ...) of the unit's column.
template <int D>
__device__ __forceinline__ MergeAcc merge_fold(const DecodeArgs &a, const MergeRow &mr, int col, int sg, int SPI,
                                               int VPR, int first, int count) {
  MergeAcc acc{-INFINITY, 0.f, (v8f){0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}};
  const MergeOffsets off = merge_offsets<D>(a, mr, col, VPR);
  const char *ws = a.ws + static_cast<int64_t>(first) * a.split_bytes;
  for (int s0 = sg; s0 < count; s0 += kMergeMU * SPI) {
    MergeRound rd;
    merge_load(a, off, ws, s0, SPI, count, rd);
    merge_fold_round(acc, rd);
  }
  return acc;
}

// Rescales an accumulator to the reference max Mr (Mr >= M; both -inf: empty).
__device__ __forceinline__ void merge_rescale(MergeAcc &x, float Mr) {
  const float w = x.M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(x.M - Mr);
  x.l *= w;
  x.o *= w;
  x.M = Mr;
}

// The merge kernel: one unit per work-group.
template <int D, int TPU>
__global__ __launch_bounds__(TPU) void decode_merge_kernel(DecodeArgs a) {
  constexpr int NW = TPU / kWave;
  __shared__ float red[NW > 1 ? NW * 32 * 10 : 1];  // per wave and column: M, l, o[8]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int unit = static_cast<int>(blockIdx.x);
  const MergeRow mr = merge_row(a, unit);
  const int VPR = (D / 8) / a.merge_cs;
  const int SPI = TPU / VPR;
  const int t = threadIdx.x, col = t % VPR, sg = t / VPR;
  MergeAcc acc{-INFINITY, 0.f, (v8f){0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}};
  if (a.batch == 1 && a.grid <= kMergeMU * SPI) {
    // One sequence owns splits 0 .. count - 1 of the G, and one round covers
    // all G: the states of every split that can exist are loaded before the
    // plan, so their round trip overlaps the one for the lengths; splits
    // past the plan's count (stale states) are dropped afterwards.
    MergeRound rd;
    merge_load(a, merge_offsets<D>(a, mr, col, VPR), a.ws, sg, SPI, a.grid, rd);
    const SplitRange sr = plan_sequence(a, lane, 0);
    const int count = sr.b < 0 ? 0 : sr.count;
#pragma unroll
    for (int u = 0; u < kMergeMU; ++u) {
      if (sg + u * SPI >= count) {
        rd.ms[u] = -INFINITY;
        rd.ls[u] = 0.f;
        rd.os[u] = (v8f){0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      }
    }
    merge_fold_round(acc, rd);
  } else {
    const SplitRange sr = plan_sequence(a, lane, mr.b);
    acc = merge_fold<D>(a, mr, col, sg, SPI, VPR, sr.first, sr.b < 0 ? 0 : sr.count);
  }
  // The lanes of one column in a wave are col + VPR * j: combine them.
  float Mw = acc.M;
  for (int off = VPR; off < kWave; off <<= 1) Mw = fmaxf(Mw, __shfl_xor(Mw, off, kWave));
  merge_rescale(acc, Mw);
  for (int off = VPR; off < kWave; off <<= 1) {
    acc.l += __shfl_xor(acc.l, off, kWave);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc.o[e] += __shfl_xor(acc.o[e], off, kWave);
  }
  if constexpr (NW > 1) {
    // Then the waves: each publishes its columns, wave 0 folds them.
    if (lane < VPR) {
      float *w = red + (wave * 32 + lane) * 10;
      w[0] = acc.M;
      w[1] = acc.l;
#pragma unroll
      for (int e = 0; e < 8; ++e) w[2 + e] = acc.o[e];
    }
    __syncthreads();
    if (wave != 0) return;
    float Mg = acc.M;
#pragma unroll
    for (int v = 1; v < NW; ++v) Mg = fmaxf(Mg, red[(v * 32 + (lane & 31)) * 10]);
    merge_rescale(acc, Mg);
#pragma unroll
    for (int v = 1; v < NW; ++v) {
      const float *w = red + (v * 32 + (lane & 31)) * 10;
      MergeAcc x{w[0], w[1], (v8f){w[2], w[3], w[4], w[5], w[6], w[7], w[8], w[9]}};
      merge_rescale(x, Mg);
      acc.l += x.l;
      acc.o += x.o;
    }
  }
  if (unit < 0 || lane >= VPR) return;
  const float inv = acc.l > 0.f ? 1.f / acc.l : 0.f;
  const int64_t ob = static_cast<int64_t>(mr.tok) * a.out_tok_stride + static_cast<int64_t>(mr.qh) * D +
                     8 * (mr.slice * VPR + lane);
  const v8f o = acc.o * inv;
  const uintptr_t addr = reinterpret_cast<uintptr_t>(a.out) + static_cast<uintptr_t>(ob) * (a.out_dtype == K8V4_F32 ? 4 : 2);
  if (a.out_dtype == K8V4_F16 && addr % 16 == 0) {
    *reinterpret_cast<v8h *>(addr) = __builtin_convertvector(o, v8h);
  } else if (a.out_dtype == K8V4_BF16 && addr % 16 == 0) {
    *reinterpret_cast<v8bf *>(addr) = __builtin_convertvector(o, v8bf);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) store_out(a.out, a.out_dtype, ob + e, o[e]);
  }
}

// ------------------------------------------------------------ split kernel
//
// Work-group = NWH waves per KV head.  Wave (h, w) handles KV head h and the
// chunks x0 + w, x0 + w + NWH, ... of the work-group's page run.  Each wave
// owns a ring of R LDS slots; a slot receives one 32-token chunk of its head
// (K codes, V nibble words, the three scale planes) through direct-to-LDS DMA
// loads (global_load_lds), so the next R-1 chunks stream in without holding
// registers.  The LDS image of each slot is laid out so every read the MFMA
// operands need is a linear, conflict-free ds_read.

typedef __attribute__((address_space(3))) char lds_t;

template <int D>
struct Slot {
  static constexpr int KS = D / 64;     // 64-dim k-steps of the QK MFMA
  static constexpr int DG = D / 128;    // 8-dim dword groups per lane in a V row
  static constexpr int VROW = D / 2;    // bytes of one token's V row (one head)
  static constexpr int KRP = 1024 / D;  // K rows per 1 KB DMA
  // K slot: [32 tokens][D] codes, 16-byte chunks XOR-swizzled per row.
  static constexpr int K_BYTES = 32 * D;
  // V slot: [32 tokens][VROW] V rows (rotated order), then ks[32] | vs[32] | vz[32].
  static constexpr int S_OFF = 32 * VROW;
  static constexpr int V_BYTES = S_OFF + 384;
  static constexpr int NK = 32 * D / 1024;       // 16-byte DMAs for the K rows
  static constexpr int NV = 32 * VROW / 1024;    // 16-byte DMAs for the V rows
  static constexpr int NVS = NV + 2;             // V rows + the two scale-plane DMAs
};

// K rows sit in LDS with their 16-byte chunks permuted: chunk c of row t is at
// position c ^ kswz(t).  A DMA writes lane L at byte 16*L of its 1 KB, so the
// permutation is applied on the source side; it makes the 16 rows read by one
// quarter-wave of the A-operand ds_read_b128 land in 16 distinct bank groups.
// LDS row position of the V row of chunk_token(g, i) (see lane_offsets).
template <int D>
__device__ __forceinline__ int vrow_pos(int g, int i) {
  const int half = i >> 2, ii = i & 3;
  if constexpr (D == 128) return 16 * half + 4 * g + ((ii + g) & 3);
  return 16 * half + 4 * g + ii;
}

template <int D>
__device__ __forceinline__ int kswz(int t) {
  if constexpr (D == 128) return (t & 7) ^ ((t >> 3) & 1);
  return t & 15;
}

// Token (0..31 within the chunk) held in slot i of a lane of group g: the two
// 16-token halves of the transposed QK^T output tile.
__device__ __forceinline__ int chunk_token(int g, int i) { return i < 4 ? 4 * g + i : 16 + 4 * g + (i - 4); }

// Direct-to-LDS loads.  K rows (one 128-byte line per token and head) are
// read exactly once and carry the nontemporal policy (streaming reads
// measured faster on MI355X).  A V row is half of a 128-byte line whose other
// half is the neighbouring head's row, read by another wave of the same
// work-group moments later: with the nontemporal policy that line was often
// fetched twice (HBM reads 1.08x the algorithmic bytes), with the default
// policy once (1.005x) at the same speed.  The scale planes, shared by the
// heads of a work-group, and the query rows, shared by the splits of a
// sequence, also use the default policy.
//
// The loads use the scalar-base form: a wave-uniform 64-bit base in SGPRs
// plus a 32-bit per-lane offset, so issuing one costs no vector instruction
// (the compiler's builtin forms every lane's 64-bit address with vector
// adds).  Written as inline assembly, these loads are invisible to the
// compiler's wait counting: every wait on them is explicit (wait_vm), and a
// compiler-generated wait can only be stronger than needed, never weaker
// (vector loads complete in issue order); nor does the compiler see LDS
// being written, which keeps it from waiting for every load in flight before
// each LDS read.  The compiler's hazard checks do not look inside inline
// assembly, so the statement sets M0 (the LDS destination) itself and then
// waits the states the load needs after a scalar write of M0 (1) and after a
// vector write of an SGPR it reads, such as a v_readfirstlane result in its
// base (5).
__device__ __forceinline__ uint32_t lds_addr(const lds_t *p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}
__device__ __forceinline__ void dma16s_nt(const void *sbase, uint32_t voff, const lds_t *dst) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase),
               "s"(lds_addr(dst))
               : "memory", "m0");
}
__device__ __forceinline__ void dma16s(const void *sbase, uint32_t voff, const lds_t *dst) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase),
               "s"(lds_addr(dst))
               : "memory", "m0");
}
// Per-lane 64-bit addresses (no scalar base): same statement shape.
__device__ __forceinline__ void dma4v(const void *addr, const lds_t *dst) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 4\n\tglobal_load_lds_dword %0, off" ::"v"(addr), "s"(lds_addr(dst))
               : "memory", "m0");
}
__device__ __forceinline__ void dma4s(const void *sbase, uint32_t voff, const lds_t *dst) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase),
               "s"(lds_addr(dst))
               : "memory", "m0");
}

// Split-state stores at device scope (sc1): written through the XCD's L2 to
// memory, where the merge kernel reads them.  With default stores the states
// of the work-groups that finish last are still dirty in L2 when the kernel
// ends, and the end-of-kernel write-back of them delays the merge launch
// (4 x 8,192 tokens, q = 7: 1.5 us per step).  Vector stores; they are the
// last memory operations of the kernel, so the compiler's wait counting, which
// does not see them, has nothing after them to order.  Its hazard checks do
// not see them either: a store of more than 8 bytes still reads its data
// registers after issue, so the statement itself waits the states before a
// later instruction may overwrite them (s_nop 1).
__device__ __forceinline__ void store_wt16(void *dst, v8h v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(dst), "v"(v) : "memory");
}
__device__ __forceinline__ void store_wt8(float2 *dst, float2 v) {
  typedef float v2f_t __attribute__((ext_vector_type(2)));
  const v2f_t x = {v.x, v.y};
  asm volatile("global_store_dwordx2 %0, %1, off sc1\n\ts_nop 1" ::"v"(dst), "v"(x) : "memory");
}

// Per-lane byte offsets of one chunk's DMA sources (loop-invariant).
struct LaneOffsets {
  uint32_t k[4];  // K source per DMA index mod 4: row L/(D/16) of the piece, swizzled chunk
  uint32_t v;     // V: token (lane*16)/VROW (+rows of later DMAs), 16-byte column
  uint32_t s;     // scale plane cell of token (lane & 31)
  // Scalar-base form of the two scale-plane gathers (when the three planes
  // share one page stride): offsets from the lower of the two plane bases a
  // gather reads, lanes 0-31 in the first plane, lanes 32-63 in the second.
  uint32_t sa, sb;
};

// PH (paired halves, head dim 256 served as two 128-dim halves): h and HKV
// count half-heads; the scale planes belong to the whole head h / 2 of HKV / 2.
template <int D, int HKV, bool PH = false>
__device__ __forceinline__ LaneOffsets lane_offsets(const DecodeArgs &a, int h, int lane) {
  constexpr int VROW = D / 2, KRP = 1024 / D, CPR = D / 16;
  constexpr int HS = PH ? HKV / 2 : HKV;  // heads of the scale planes
  LaneOffsets o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = j * KRP + lane / CPR;  // row of DMA j (mod 4) this lane fills
    const int c = (lane % CPR) ^ kswz<D>(t);
    o.k[j] = static_cast<uint32_t>((lane / CPR) * (HKV * D) + h * D + 16 * c);
  }
  {
    // V rows of one DMA sit in LDS rotated within groups of four rows
    // (position 4q + ((i + q) & 3) holds row 4q + i) so the eight 4-byte
    // operand reads of a chunk spread over all banks.
    const int pos = (lane * 16) / VROW;
    const int row = VROW == 64 ? 4 * (pos >> 2) + (((pos & 3) - (pos >> 2)) & 3) : pos;
    o.v = static_cast<uint32_t>(row * (HKV * VROW) + h * VROW + (lane * 16) % VROW);
  }
  o.s = static_cast<uint32_t>(((lane & 31) * HS + (PH ? h >> 1 : h)) * 4);
  const int64_t lo_kv = a.d_kv < 0 ? a.d_kv : 0, lo_vz = a.d_vz < 0 ? a.d_vz : 0;
  o.sa = o.s + static_cast<uint32_t>(lane < 32 ? -lo_kv : a.d_kv - lo_kv);
  o.sb = o.s + static_cast<uint32_t>(lane < 32 ? -lo_vz : a.d_vz - lo_vz);
  return o;
}

// Starts the DMA of chunk x (32 tokens of head h, in physical page `phys`, -1
// outside the cache) into `slot`; returns whether the page is a cache page.
// An invalid page still issues its loads (from page 0) so every chunk costs
// the same vmcnt.  K and V move in
// 16-byte-per-lane DMAs from a wave-uniform base plus a 32-bit lane offset;
// the scale planes of this head are gathered with two 4-byte DMAs (lanes
// 0-31: k_scale then v_scale, lanes 32-63: v_scale then v_zero).
template <int D, int HKV>
__device__ __forceinline__ int issue_k(const DecodeArgs &a, int phys, int x, const LaneOffsets &lo, lds_t *kslot) {
  using S = Slot<D>;
  const int half = x & 1;
  const int valid = phys >= 0 ? 1 : 0;
  if (!valid) phys = 0;
  const char *kb = reinterpret_cast<const char *>(a.k_cache) + phys * a.k_ps +
                   static_cast<int64_t>(32 * half) * HKV * D;
#pragma unroll
  for (int j = 0; j < S::NK; ++j) dma16s_nt(kb + static_cast<int64_t>(j) * S::KRP * (HKV * D), lo.k[j & 3], kslot + j * 1024);
  return valid;
}

template <int D, int HKV, bool PH = false>
__device__ __forceinline__ void issue_v(const DecodeArgs &a, int phys, int x, const LaneOffsets &lo, int lane,
                                        lds_t *vslot) {
  using S = Slot<D>;
  constexpr int HS = PH ? HKV / 2 : HKV;  // heads of the scale planes
  const int half = x & 1;
  if (phys < 0) phys = 0;
  const int tok0 = 32 * half;
  const char *vb = reinterpret_cast<const char *>(a.v_cache) + phys * a.v_ps +
                   static_cast<int64_t>(tok0) * HKV * S::VROW;
#pragma unroll
  for (int j = 0; j < S::NV; ++j) dma16s(vb + static_cast<int64_t>(j) * (1024 / S::VROW) * (HKV * S::VROW), lo.v, vslot + j * 1024);
  // Two full-wave 4-byte DMAs, no divergent branch: ks[32] | vs[32] at
  // S_OFF, then vs[32] | vz[32] at S_OFF + 128 (the v_scale cells are written
  // twice with the same values).
  const int64_t plane0 = static_cast<int64_t>(tok0) * HS * 4;
  if (a.planes_fast) {
    const int64_t lo_kv = a.d_kv < 0 ? a.d_kv : 0, lo_vz = a.d_vz < 0 ? a.d_vz : 0;
    const char *pa = reinterpret_cast<const char *>(a.k_scale) + lo_kv + phys * a.ks_ps + plane0;
    const char *pb = reinterpret_cast<const char *>(a.v_scale) + lo_vz + phys * a.vs_ps + plane0;
    dma4s(pa, lo.sa, vslot + S::S_OFF);
    dma4s(pb, lo.sb, vslot + S::S_OFF + 128);
  } else {
    const char *ksp = reinterpret_cast<const char *>(a.k_scale) + phys * a.ks_ps + plane0 + lo.s;
    const char *vsp = reinterpret_cast<const char *>(a.v_scale) + phys * a.vs_ps + plane0 + lo.s;
    const char *vzp = reinterpret_cast<const char *>(a.v_zero) + phys * a.vz_ps + plane0 + lo.s;
    dma4v(lane < 32 ? ksp : vsp, vslot + S::S_OFF);
    dma4v(lane < 32 ? vsp : vzp, vslot + S::S_OFF + 128);
  }
}

// Wait until at most `after` chunks' DMAs are still in flight.
// Wait until at most n (wave-uniform, 0..) vector-memory loads are
// outstanding.  s_waitcnt takes an immediate, so the count is dispatched;
// counts above 62 wait for 62 (more than needed, still correct).
__device__ __forceinline__ void wait_vm(int n) {
#define K8V4_WAIT_CASE(N) \
  case N:                 \
    asm volatile("s_waitcnt vmcnt(" #N ")" ::: "memory"); \
    break;
  switch (n < 62 ? n : 62) {
    K8V4_WAIT_CASE(0) K8V4_WAIT_CASE(1) K8V4_WAIT_CASE(2) K8V4_WAIT_CASE(3) K8V4_WAIT_CASE(4)
    K8V4_WAIT_CASE(5) K8V4_WAIT_CASE(6) K8V4_WAIT_CASE(7) K8V4_WAIT_CASE(8) K8V4_WAIT_CASE(9)
    K8V4_WAIT_CASE(10) K8V4_WAIT_CASE(11) K8V4_WAIT_CASE(12) K8V4_WAIT_CASE(13) K8V4_WAIT_CASE(14)
    K8V4_WAIT_CASE(15) K8V4_WAIT_CASE(16) K8V4_WAIT_CASE(17) K8V4_WAIT_CASE(18) K8V4_WAIT_CASE(19)
    K8V4_WAIT_CASE(20) K8V4_WAIT_CASE(21) K8V4_WAIT_CASE(22) K8V4_WAIT_CASE(23) K8V4_WAIT_CASE(24)
    K8V4_WAIT_CASE(25) K8V4_WAIT_CASE(26) K8V4_WAIT_CASE(27) K8V4_WAIT_CASE(28) K8V4_WAIT_CASE(29)
    K8V4_WAIT_CASE(30) K8V4_WAIT_CASE(31) K8V4_WAIT_CASE(32) K8V4_WAIT_CASE(33) K8V4_WAIT_CASE(34)
    K8V4_WAIT_CASE(35) K8V4_WAIT_CASE(36) K8V4_WAIT_CASE(37) K8V4_WAIT_CASE(38) K8V4_WAIT_CASE(39)
    K8V4_WAIT_CASE(40) K8V4_WAIT_CASE(41) K8V4_WAIT_CASE(42) K8V4_WAIT_CASE(43) K8V4_WAIT_CASE(44)
    K8V4_WAIT_CASE(45) K8V4_WAIT_CASE(46) K8V4_WAIT_CASE(47) K8V4_WAIT_CASE(48) K8V4_WAIT_CASE(49)
    K8V4_WAIT_CASE(50) K8V4_WAIT_CASE(51) K8V4_WAIT_CASE(52) K8V4_WAIT_CASE(53) K8V4_WAIT_CASE(54)
    K8V4_WAIT_CASE(55) K8V4_WAIT_CASE(56) K8V4_WAIT_CASE(57) K8V4_WAIT_CASE(58) K8V4_WAIT_CASE(59)
    K8V4_WAIT_CASE(60) K8V4_WAIT_CASE(61)
    default:
      asm volatile("s_waitcnt vmcnt(62)" ::: "memory");
      break;
  }
#undef K8V4_WAIT_CASE
}

__device__ __forceinline__ v2h pack_h2(float lo, float hi) {
  return __builtin_convertvector((v2f){lo, hi}, v2h);
}

// max(x, x from lane^16) and max(x, x from lane^32) without LDS.
__device__ __forceinline__ float xlane_max16_32(float x) {
  auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
  auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}

// (The int8 query operands live in LDS, shared by the waves of a head.)
template <int D, int NT>
struct WaveState {
  static constexpr int DG = D / 128;
  float crow[NT];   // q_scale * log2(e) / sqrt(D), > 0
  int lim[NT];      // causal end of this lane's row (S layout)
  float m_run[NT];  // running max, log2 domain (S layout)
  float thr[NT];    // (m_run + threshold) / crow: a raw score above it moves m_run
  v4f lsum[NT];     // row sums (O layout, rows 4g+i)
  v4f corr[NT];     // sum of P * v_scale * v_zero per row (O layout)
  v4f O[NT][DG][8]; // unnormalized output (O layout)
};

// TS: LDS tiles between this wave's query tiles (2 when the waves of a head
// hold alternate row tiles).
template <int D, int NT, int TS = 1>
__device__ __forceinline__ void chunk_qk(const lds_t *kslot, const lds_t *qlds, int lane, int g, v4i (&sc)[2][NT]) {
  using S = Slot<D>;
  constexpr int KS = S::KS;
  // ---- QK^T, transposed: S[ml][nt] lane (n,g) reg i = score(token 16*ml+4g+i, row 16*nt+n)
  v4i kf[2][KS];
  const int n = lane & 15;
#pragma unroll
  for (int ml = 0; ml < 2; ++ml)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int t = 16 * ml + n, c = 4 * ks + g;
      kf[ml][ks] = *reinterpret_cast<const __attribute__((address_space(3))) v4i *>(
          kslot + t * D + 16 * (c ^ kswz<D>(t)));
    }
  // k-step outermost: the 2 * NT score tiles are independent accumulators,
  // so consecutive MFMAs never wait on each other.
#pragma unroll
  for (int ml = 0; ml < 2; ++ml)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) sc[ml][nt] = (v4i){kScoreBias, kScoreBias, kScoreBias, kScoreBias};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const v4i qf =
          *reinterpret_cast<const __attribute__((address_space(3))) v4i *>(qlds + ((nt * TS * KS + ks) * kWave + lane) * 16);
#pragma unroll
      for (int ml = 0; ml < 2; ++ml) sc[ml][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf[ml][ks], qf, sc[ml][nt], 0, 0, 0);
    }
}

// QK^T of a 256-dim head from two 128-dim K slots (paired halves): dims
// 0-127 of the chunk's keys in `klo`, dims 128-255 in `khi` (the slots of the
// two waves of the pair), the query fragments of all four 64-dim k-steps in
// LDS.  Same score layout and bias as chunk_qk; |dot| <= 256 * 127 * 127 <
// 2^22 keeps the biased accumulator exact.  The two halves' K operands are
// read one half at a time (16 registers instead of 32).
template <int NT, int TS = 1>
__device__ __forceinline__ void chunk_qk_pair(const lds_t *klo, const lds_t *khi, const lds_t *qlds, int lane, int g,
                                              v4i (&sc)[2][NT]) {
  const int n = lane & 15;
#pragma unroll
  for (int ml = 0; ml < 2; ++ml)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) sc[ml][nt] = (v4i){kScoreBias, kScoreBias, kScoreBias, kScoreBias};
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    const lds_t *kslot = part ? khi : klo;
    v4i kf[2][2];
#pragma unroll
    for (int ml = 0; ml < 2; ++ml)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int t = 16 * ml + n, c = 4 * ks + g;
        kf[ml][ks] = *reinterpret_cast<const __attribute__((address_space(3))) v4i *>(
            kslot + t * 128 + 16 * (c ^ kswz<128>(t)));
      }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const v4i qf = *reinterpret_cast<const __attribute__((address_space(3))) v4i *>(
            qlds + ((nt * TS * 4 + 2 * part + ks) * kWave + lane) * 16);
#pragma unroll
        for (int ml = 0; ml < 2; ++ml) sc[ml][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf[ml][ks], qf, sc[ml][nt], 0, 0, 0);
      }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Flags of the paired-halves handshake, one word per wave in LDS.  A flag
// only grows within a launch; a wait polls its partner's word (wave-uniform)
// until it reaches the target, sleeping between polls.  The pair runs the
// same chunk sequence and neither wave waits before publishing what the
// other waits for, so every wait ends; the bound only caps a wait that a
// broken launch could otherwise make endless, and such a give-up is counted
// in a device word the host reads (k8v4_decode_fault_count), so it shows up
// in tests instead of as a silently wrong output.
typedef __attribute__((address_space(3))) int lds_int;
__device__ int g_pair_wait_timeouts;
__device__ __forceinline__ void pair_flag_set(lds_int *f, int v, int lane) {
  if (lane == 0) *reinterpret_cast<volatile lds_int *>(f) = v;
}
__device__ __forceinline__ void pair_flag_wait(const lds_int *f, int target, int lane) {
  for (int it = 0; it < (1 << 22); ++it) {
    const int v = __builtin_amdgcn_readfirstlane(*reinterpret_cast<const volatile lds_int *>(f));
    if (v >= target) return;
    __builtin_amdgcn_s_sleep(1);
  }
  if (lane == 0) __hip_atomic_fetch_add(&g_pair_wait_timeouts, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Softmax and P.V of one chunk whose scores chunk_qk produced; reads the V
// rows and scale planes of the chunk's V slot.
template <int D, int NT, bool RAISE = false>
__device__ __forceinline__ void chunk_softmax_pv(WaveState<D, NT> &st, const v4i (&sc)[2][NT],
                                                 const lds_t *vslot, int tbase, int L0, int lane, int g,
                                                 bool masked) {
  using S = Slot<D>;
  constexpr int DG = S::DG;
  // Phase fences keep the scheduler from hoisting later LDS reads into this
  // phase, which would raise register pressure past two waves per SIMD.
  __builtin_amdgcn_sched_barrier(0);
  // RAISE (the paired halves): the softmax's vector work runs at a raised
  // issue priority, so beside the other wave's matrix phases it overlaps them
  // instead of queueing behind that wave's vector instructions (reference
  // shape 40.6 -> 40.2 us; with the 128-dim kernels' progress balance it
  // measured slower at the headline, so they do not raise).
  if constexpr (RAISE) __builtin_amdgcn_s_setprio(1);
  // ---- scale planes of this lane's 8 tokens: [0..3] = tokens 4g+i, [4..7] = 16+4g+i
  typedef float v4f_l __attribute__((ext_vector_type(4)));
  const auto *sp = reinterpret_cast<const __attribute__((address_space(3))) v4f_l *>(vslot + S::S_OFF);
  v4f_l ksa = sp[g], ksb = sp[4 + g], vsa = sp[8 + g], vsb = sp[12 + g], vza = sp[16 + g], vzb = sp[20 + g];
  float ksv[8] = {ksa[0], ksa[1], ksa[2], ksa[3], ksb[0], ksb[1], ksb[2], ksb[3]};
  float vsv[8] = {vsa[0], vsa[1], vsa[2], vsa[3], vsb[0], vsb[1], vsb[2], vsb[3]};
  float vzv[8] = {vza[0], vza[1], vza[2], vza[3], vzb[0], vzb[1], vzb[2], vzb[3]};
  if (__builtin_expect(masked, 0)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (tbase + chunk_token(g, i) >= L0) {  // unwritten tail: never use its planes
        ksv[i] = 0.f;
        vsv[i] = 0.f;
        vzv[i] = 0.f;
      }
    }
  }
  // The QK accumulators start at the bits of 1.5 * 2^23, so each reads as the
  // float 12582912 + dot, exactly (|dot| <= 128 * 127 * 127 < 2^22); one fma
  // with k_bias = -12582912 * k_scale gives dot * k_scale within 0.75 of a
  // unit of the dot (the rounding of k_bias) -- against a query quantization
  // step of about 0.3 * |k| per dim.
  float kbias[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) kbias[i] = -12582912.0f * ksv[i];
  // ---- scores, chunk max, lazy rescale
  float t[2][NT][4];
  float lmx[NT];  // this lane's largest score of each row tile
  bool grow = false;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float mx = -INFINITY;
#pragma unroll
    for (int ml = 0; ml < 2; ++ml)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = fmaf(__int_as_float(sc[ml][nt][i]), ksv[4 * ml + i], kbias[4 * ml + i]);
        t[ml][nt][i] = v;
      }
    if (__builtin_expect(masked, 0)) {
#pragma unroll
      for (int ml = 0; ml < 2; ++ml)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (tbase + 16 * ml + 4 * g + i >= st.lim[nt]) t[ml][nt][i] = -INFINITY;
    }
#pragma unroll
    for (int ml = 0; ml < 2; ++ml)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, t[ml][nt][i]);
    lmx[nt] = mx;
    // A row's largest score passes the threshold exactly when one of its four
    // lanes' does, so the cross-lane max is only taken on a rescale.
    grow |= mx > st.thr[nt];
  }
  if (__ballot(grow)) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const float mnew = fmaxf(st.m_run[nt], xlane_max16_32(lmx[nt]) * st.crow[nt]);
      const float alpha = st.m_run[nt] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st.m_run[nt] - mnew);
      st.m_run[nt] = mnew;
      st.thr[nt] = (mnew + kRescaleThreshold) / st.crow[nt];
      float ai[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ai[i] = __shfl(alpha, 4 * g + i, kWave);
        st.lsum[nt][i] *= ai[i];
        st.corr[nt][i] *= ai[i];
      }
#pragma unroll
      for (int dg = 0; dg < DG; ++dg)
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) st.O[nt][dg][j][i] *= ai[i];
    }
  }
  // ---- P = exp2(score * c - m), packed fp16 in the PV A-operand layout; row sums by MFMA
  const v8h ones = {1, 1, 1, 1, 1, 1, 1, 1};
  v2h vsp[4];
  v8h bz;  // v_zero of the lane's tokens: the zero-point correction operand
  {
    const v2h z01 = pack_h2(vzv[0], vzv[1]), z23 = pack_h2(vzv[2], vzv[3]);
    const v2h z45 = pack_h2(vzv[4], vzv[5]), z67 = pack_h2(vzv[6], vzv[7]);
    bz = (v8h){z01[0], z01[1], z23[0], z23[1], z45[0], z45[1], z67[0], z67[1]};
#pragma unroll
    for (int qp = 0; qp < 4; ++qp) vsp[qp] = pack_h2(vsv[2 * qp], vsv[2 * qp + 1]);
  }
  v8h PA[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float nm = -fmaxf(st.m_run[nt], -FLT_MAX) - kPLog2Offset;
    float p[8];
#pragma unroll
    for (int ml = 0; ml < 2; ++ml)
#pragma unroll
      for (int i = 0; i < 4; ++i) p[4 * ml + i] = __builtin_amdgcn_exp2f(fmaf(t[ml][nt][i], st.crow[nt], nm));
    v2h pp[4] = {pack_h2(p[0], p[1]), pack_h2(p[2], p[3]), pack_h2(p[4], p[5]), pack_h2(p[6], p[7])};
    st.lsum[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
        (v8h){pp[0][0], pp[0][1], pp[1][0], pp[1][1], pp[2][0], pp[2][1], pp[3][0], pp[3][1]}, ones, st.lsum[nt],
        0, 0, 0);
    // P' = P * v_scale of each token (the V scale moves onto the A operand).
#pragma unroll
    for (int qp = 0; qp < 4; ++qp) pp[qp] = pp[qp] * vsp[qp];
    PA[nt] = (v8h){pp[0][0], pp[0][1], pp[1][0], pp[1][1], pp[2][0], pp[2][1], pp[3][0], pp[3][1]};
    st.corr[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(PA[nt], bz, st.corr[nt], 0, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (RAISE) __builtin_amdgcn_s_setprio(0);
  // ---- V: the packed bytes themselves are the B operand, read as fp16
  // subnormals: a byte in the low half of a 16-bit lane is (16 hi + lo) * 2^-24
  // and (x & 0x00F000F0) is hi * 2^-20.  Exact; the finalization takes the
  // even dim as the difference, rescales by 2^24 / 2^20 and subtracts the
  // zero-point correction.
#pragma unroll
  for (int dg = 0; dg < DG; ++dg) {
    uint32_t vw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      vw[i] = *reinterpret_cast<const __attribute__((address_space(3))) uint32_t *>(
          vslot + vrow_pos<D>(g, i) * S::VROW + 64 * dg + 4 * (lane & 15));
#pragma unroll
    for (int byte = 0; byte < 4; ++byte) {
      const uint32_t sel = 0x0C000C00u | (static_cast<uint32_t>(4 + byte) << 16) | static_cast<uint32_t>(byte);
      uint32_t be[4], bo[4];
#pragma unroll
      for (int qp = 0; qp < 4; ++qp) {
        const uint32_t xw = __builtin_amdgcn_perm(vw[2 * qp + 1], vw[2 * qp], sel);
        be[qp] = xw;
        bo[qp] = xw & 0x00F000F0u;
      }
      const v8h Be = __builtin_bit_cast(v8h, (v4i){static_cast<int>(be[0]), static_cast<int>(be[1]),
                                                   static_cast<int>(be[2]), static_cast<int>(be[3])});
      const v8h Bo = __builtin_bit_cast(v8h, (v4i){static_cast<int>(bo[0]), static_cast<int>(bo[1]),
                                                   static_cast<int>(bo[2]), static_cast<int>(bo[3])});
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        st.O[nt][dg][2 * byte] = __builtin_amdgcn_mfma_f32_16x16x32_f16(PA[nt], Be, st.O[nt][dg][2 * byte], 0, 0, 0);
        st.O[nt][dg][2 * byte + 1] =
            __builtin_amdgcn_mfma_f32_16x16x32_f16(PA[nt], Bo, st.O[nt][dg][2 * byte + 1], 0, 0, 0);
      }
    }
  }
}

// O = sum P' * q * 2^-24 (even dims) or 2^-20 (odd dims); the dequantized
// value is (q - zero) * scale, so the true accumulator is the rescaled sum
// minus the zero-point correction.
template <int D, int NT>
__device__ __forceinline__ void finalize_output(WaveState<D, NT> &st) {
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int dg = 0; dg < D / 128; ++dg)
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        // O[j] holds sum p' (16 hi + lo) 2^-24 (the whole byte), O[j+1] holds
        // sum p' 16 hi 2^-24: the even dim is their difference.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float whole = st.O[nt][dg][j][i], high = st.O[nt][dg][j + 1][i];
          st.O[nt][dg][j][i] = fmaf(whole - high, 16777216.0f, -st.corr[nt][i]);
          st.O[nt][dg][j + 1][i] = fmaf(high, 1048576.0f, -st.corr[nt][i]);
        }
      }
}

template <int D, int NT, int HKV, int NWH, bool PH = false, bool RS = false>
struct SplitConfig {
  // Two waves per head (NWH = 2), or paired halves (PH) with one or two
  // waves per half-head; two waves per SIMD either way.  The int8 Q operands
  // live in LDS, per head (shared by its waves; PH: all 256 dims, per whole
  // head).  Each wave owns a K ring of RK slots and a V ring of RV slots,
  // the K ring as deep as the LDS allows; a K slot is refilled as soon as
  // its QK^T product is issued, so while a wave computes one chunk up to
  // RK - 1 K slots and RV - 1 V slots are in flight.  PH: D = 128 and HKV
  // half-heads serve a 256-dim cache of HKV / 2 heads.  RS (row split, four
  // row tiles): the two waves of a head hold alternate row tiles (NT each)
  // and both multiply every chunk of the split, each chunk resident in the
  // ring of the wave that loaded it.
  static constexpr int NTQ = RS ? 2 * NT : NT;    // row tiles of a head's query
  static constexpr int DQ = PH ? 2 * D : D;       // dims of one score
  static constexpr int QHEADS = PH ? HKV / 2 : HKV;
  static constexpr int WAVES = HKV * NWH;
  static constexpr int Q_FRAG_BYTES = NTQ * (DQ / 64) * kWave * 16;       // int8 B-operand fragments
  static constexpr int Q_LDS_BYTES = Q_FRAG_BYTES + NTQ * 16 * 4;          // + per-row factors
  // 4 / HKV work-groups share a CU (the grid is about that many per CU; one
  // with eight half-head waves).
  static constexpr int LDS_MAX = HKV >= 4 ? 163840 : 163840 * HKV / 4;
  static constexpr int Q_BYTES_PER_HEAD = Q_LDS_BYTES;
  static constexpr int Q_TOTAL = QHEADS * Q_BYTES_PER_HEAD;
  // PH handshake words: per wave, the chunks whose K half is resident and
  // the chunks whose K slots it has finished reading.
  // Progress balance (two waves per head, eight waves: waves w and w + 4
  // share a SIMD): one chunk counter per wave.
  static constexpr bool BALANCE = NWH == 2 && WAVES == 8 && !PH && !RS;
  static constexpr int FLAG_BYTES = (PH || RS) ? 2 * WAVES * 4 : (BALANCE ? WAVES * 4 : 0);
  // A PH wave refills its K slot after P.V, next to the V slot: the other
  // half of its pair reads that slot during its own QK^T.
  static constexpr bool K_EARLY = !PH && !RS;
  static constexpr int RV = 2;
  static constexpr int RK_FIT = ((LDS_MAX - Q_TOTAL - FLAG_BYTES) / WAVES - RV * Slot<D>::V_BYTES) / Slot<D>::K_BYTES;
  static constexpr int RK = RK_FIT < 2 ? 2 : (RK_FIT > 4 ? 4 : RK_FIT);
  static constexpr int WAVE_BYTES = RK * Slot<D>::K_BYTES + RV * Slot<D>::V_BYTES;
  // Loads issued after a chunk's V group until that chunk is consumed, in
  // the steady state of the main loop (one K and one V group per chunk).
  static constexpr int STEADY_AFTER = (RV - 1) * (Slot<D>::NK + Slot<D>::NVS);
  static constexpr int Q_OFF = WAVES * WAVE_BYTES;
  static constexpr int FLAG_OFF = Q_OFF + Q_TOTAL;
  static constexpr int RING_BYTES = FLAG_OFF + FLAG_BYTES;
  // Partner-wave state exchange at the end (reuses the ring memory).
  static constexpr int XCHG_FLOATS = (NT * (D / 128) * 8 * 4 + NT * 4 + NT) * kWave;
  static constexpr int XCHG_BYTES = (NWH > 1 && !RS) ? HKV * XCHG_FLOATS * 4 : 0;
  static constexpr int LDS_BYTES = RING_BYTES > XCHG_BYTES ? RING_BYTES : XCHG_BYTES;
  static constexpr int OCC = HKV > 4 ? HKV * NWH / 4 : NWH;  // waves per SIMD the kernel is built for
  static_assert(LDS_BYTES <= LDS_MAX, "decode ring exceeds the LDS");
  static_assert(PH || NWH == 2, "128-dim heads run two waves each");
  static_assert(!RS || NWH == 2, "row split: two waves per (half-)head");
  // The query rows of a wave's tiles are staged in its K slots 1..RK-1 (RS:
  // loaded into registers instead; PH: read already quantized).
  static_assert(PH || RS || ((NT + NWH - 1) / NWH) * 16 * 2 * D <= (RK - 1) * Slot<D>::K_BYTES,
                "query staging does not fit the K ring");
};

// PH: paired halves.  A 256-dim cache of HKV / 2 heads is served as HKV
// 128-dim half-heads (its K rows [token][HKV/2][256] and V rows
// [token][HKV/2][128 B] are exactly the rows of a 128-dim cache of HKV
// heads): waves h = 2 hh + half load and compute on dims 128 half .. + 127 of
// head hh; the two waves of a pair build each chunk's 256-dim scores from
// both of their K slots (an LDS handshake per chunk orders the slot reads
// against the DMAs), run the same softmax and accumulate P.V over their own
// 128 output dims.  The query comes pre-quantized (256-dim rows, one scale
// per row).
template <int D, int NT, int HKV, int NWH, bool PH = false, bool RS = false>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * HKV * NWH, 64 * HKV * NWH),
                          amdgpu_waves_per_eu(SplitConfig<D, NT, HKV, NWH, PH, RS>::OCC,
                                              SplitConfig<D, NT, HKV, NWH, PH, RS>::OCC)))
void decode_split_kernel(DecodeArgs a) {
  static_assert(D == 128, "split-kernel instances are 128-dim (head dim 256 runs as paired halves)");
  using S = Slot<D>;
  using CFG = SplitConfig<D, NT, HKV, NWH, PH, RS>;
  constexpr int KS = S::KS, DG = S::DG, RK = CFG::RK, RV = CFG::RV;
  __shared__ __attribute__((aligned(16))) char lds_raw[CFG::LDS_BYTES];
  lds_t *lds = (lds_t *)(lds_raw);

  const int lane = threadIdx.x & (kWave - 1);
  // Wave-uniform by construction; readfirstlane tells the compiler so, which
  // keeps page lookups on the scalar unit.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int h = wave % HKV;   // KV head (PH: half-head)
  const int w = wave / HKV;   // position among the NWH waves of this head
  const int hq = PH ? h >> 1 : h;  // head of the query rows, scale planes and split state
  const int half = PH ? h & 1 : 0;
  const int n = lane & 15, g = lane >> 4;
  // Row tile of the launch held in this wave's tile slot j (RS: alternate
  // tiles w, w + 2; otherwise all NT).
  auto tile_of = [&](int j) { return RS ? w + 2 * j : j; };

  const int role = static_cast<int>(blockIdx.x);  // this work-group's split of the plan
  const SplitPlan plan = plan_split(a, lane, role);
  const SplitRange sr = plan.r;
  if (sr.b < 0) return;  // idle work-group (uniform over the work-group)
  const int P = plan.P;
  const int b = sr.b;
  const int npages = plan.npages;
  const int L0 = plan.L0;
  const int p0 = (role - sr.first) * P;
  const int p1 = min(npages, p0 + P);
  const int x0 = 2 * p0;
  const int x1 = min(2 * p1, (L0 + 31) / 32);
  const int32_t *bt_row = a.block_table + static_cast<int64_t>(b) * a.bt_stride;
  const int rows = a.q_len * kGqa;
  const int r0 = 16 * a.tile0;  // this launch's tiles are rows r0 .. r0 + 16 NT - 1

  // A pre-quantized query tile (k8v4_attn_batch_q8) replaces the raw rows
  // and their quantization below.
  const bool pre_q = a.q8 != nullptr;  // uniform over the launch

  WaveState<D, NT> st;
  lds_t *qlds = lds + CFG::Q_OFF + hq * CFG::Q_BYTES_PER_HEAD;
  // Causal ends, through scalar loads (they are uniform over the
  // work-group): row r (token j = r / 6) sees keys t < lim(r).
  int min_end = L0;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) st.lim[nt] = L0;
  {
    const const_i32_ptr vis = a.visible ? (const_i32_ptr)(a.visible + static_cast<int64_t>(b) * a.vis_stride + 1)
                                        : (const_i32_ptr) nullptr;
    for (int j = 0; j < a.q_len; ++j) {
      const int e = a.visible ? vis[j] : L0 - a.q_len + j + 1;
      min_end = min(min_end, e);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int r = r0 + 16 * tile_of(nt) + n;
        if (r < rows && r / kGqa == j) st.lim[nt] = min(e, L0);
      }
    }
  }

  // This wave's chunks: x0 + w + k*NWH for k < cnt.
  const int my0 = x0 + w;
  const int cnt = my0 < x1 ? (x1 - my0 + NWH - 1) / NWH : 0;
  lds_t *kring = lds + wave * CFG::WAVE_BYTES;
  lds_t *vring = kring + RK * S::K_BYTES;
  const LaneOffsets lo = lane_offsets<D, HKV, PH>(a, h, lane);
  // DMA bookkeeping (wave-uniform): `issued` counts this wave's DMA
  // instructions; mk[s] / mv[s] is the count right after the K / V group of
  // ring slot s was issued, so a chunk is resident once at most
  // issued - max(mk, mv) loads remain outstanding (loads complete in order).
  // With the query rows staged in K slots 1.., only the first chunk's K and
  // V groups go out before the quantization and the rest of the ring right
  // after it; the paired halves and the row split (no staging) fill the
  // whole ring at once.
  int issued = 0;
  // Q in LDS: this wave's query rows (its tiles nt = w, w + NWH, ...) go by
  // direct-to-LDS loads into its K slots 1.. (filled only after the
  // quantization), ahead of the block-table loads below, so the two round
  // trips overlap (the first chunk's loads need the table entries; the
  // quantization needs only these rows).  Waiting for them is then a plain
  // count of this wave's own loads.  Rows past the last query row load row 0
  // and are zeroed below.
  lds_t *qstage = kring + S::K_BYTES;
  // RS: this wave's rows (its NT alternate tiles) come into registers instead
  // (the ring's K slots are all needed), ahead of the table entries likewise;
  // lane (n, g) takes row 16 tile + n, dims 64 ks + 16 g .. + 15.
  v4i qraw[RS && !PH ? NT : 1][KS][2];
  if constexpr (RS && !PH) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qraw[j][ks][0] = qraw[j][ks][1] = (v4i){0, 0, 0, 0};
      const int r = r0 + 16 * tile_of(j) + n;
      if (r < rows && !pre_q) {
        const int jt = r / kGqa;
        const int qh = h * kGqa + (r - jt * kGqa);
        const uint16_t *src = a.q + (static_cast<int64_t>(b) * a.q_len + jt) * a.q_tok_stride +
                              static_cast<int64_t>(qh) * D;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          qraw[j][ks][0] = *reinterpret_cast<const v4i *>(src + 64 * ks + 16 * g);
          qraw[j][ks][1] = *reinterpret_cast<const v4i *>(src + 64 * ks + 16 * g + 8);
        }
      }
    }
  }
  if (!PH && !RS && !pre_q) {
    constexpr int RPD = 1024 / (2 * D);  // query rows per 1 KB load
    const char *qbase = reinterpret_cast<const char *>(a.q) + static_cast<int64_t>(b) * a.q_len * a.q_tok_stride * 2;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (nt % NWH != w) continue;
      const int ti = nt / NWH;
#pragma unroll
      for (int d = 0; d < 16 / RPD; ++d) {
        const int r = r0 + 16 * nt + RPD * d + lane / (2 * D / 16);
        const int rr = r < rows ? r : 0;
        const int j = rr / kGqa;
        const int qh = h * kGqa + (rr - j * kGqa);
        const uint32_t off = static_cast<uint32_t>((j * a.q_tok_stride + qh * D + 8 * (lane % (2 * D / 16))) * 2);
        dma16s(qbase, off, qstage + (ti * 16 + RPD * d) * 2 * D);  // shared by the splits of b: cached
        ++issued;
      }
    }
  }
  // PH: the query tile's fragments go by direct-to-LDS loads straight into
  // their operand positions (lane L of fragment (nt, ks) is 16 bytes at 16 L:
  // row 16 nt + n, dims 64 ks + 16 g), the rows' scales into the factor
  // words; no K slot stages anything, so the whole ring is filled at once.
  if constexpr (PH) {
    constexpr int DQ = CFG::DQ, KSQ = DQ / 64;
    const int8_t *tile = a.q8 + static_cast<int64_t>(b) * a.q8_seq_stride + static_cast<int64_t>(hq) * kPage * DQ;
#pragma unroll
    for (int nt = 0; nt < CFG::NTQ; ++nt) {
      if (nt % NWH != w) continue;
#pragma unroll
      for (int ks = 2 * half; ks < 2 * half + 2; ++ks) {
        dma16s(tile, static_cast<uint32_t>((r0 + 16 * nt + n) * DQ + 64 * ks + 16 * g),
               qlds + (nt * KSQ + ks) * kWave * 16);
        ++issued;
      }
    }
    if (w == 0 && half == 0) {
      const float *scales = a.q8_scale + static_cast<int64_t>(b) * a.qs_seq_stride + hq * kPage;
      if (lane < CFG::NTQ * 16) dma4s(scales, static_cast<uint32_t>((r0 + lane) * 4), qlds + CFG::Q_FRAG_BYTES);
      ++issued;
    }
  }
  const int q_done = issued;
  // Physical pages of this split's run, looked up once: lane l of ptab[i]
  // holds page p0 + 64 i + l (-1 outside the cache), read back per chunk
  // with v_readlane (no scalar-cache miss or page division in the loop).
  // Runs longer than 128 pages look their pages up as they go.
  const bool tab_vgpr = p1 - p0 <= 128;
  int ptab[2] = {-1, -1};
  if (tab_vgpr) {
    // Both entries are loaded before either is used (one round trip; a lane
    // past the run reads the run's last entry and is dropped below).
    int raw[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = min(p0 + 64 * i + lane, p1 - 1);
      raw[i] = bt_row[a.ppb <= 1 ? p : p / a.ppb];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = p0 + 64 * i + lane;
      const int ph = a.ppb <= 1 ? raw[i] : raw[i] * a.ppb + p % a.ppb;
      ptab[i] = (p < p1 && ph >= 0 && ph < a.num_pages) ? ph : -1;
    }
  }
  auto page_of = [&](int x) -> int {  // x: chunk index in the sequence (wave-uniform)
    const int p = x >> 1;
    if (tab_vgpr) {
      const int d = p - p0;
      const int lo_pg = __builtin_amdgcn_readlane(ptab[0], d & 63);
      const int hi_pg = __builtin_amdgcn_readlane(ptab[1], d & 63);
      return d < 64 ? lo_pg : hi_pg;
    }
    const int ph = physical_page(a, bt_row, p);
    return (ph >= 0 && ph < a.num_pages) ? ph : -1;
  };
  int mk[4] = {0, 0, 0, 0}, mv[4] = {0, 0, 0, 0};
  uint32_t valid_mask = 0;  // bit s: K slot s holds a chunk of a valid page
  auto fill_slot = [&](int s) {
    if (s >= cnt) return;
    const int xs = my0 + s * NWH;
    if (s < RK) {
      valid_mask |= static_cast<uint32_t>(issue_k<D, HKV>(a, page_of(xs), xs, lo, kring + s * S::K_BYTES)) << s;
      issued += S::NK;
      mk[s] = issued;
    }
    if (s < RV) {
      issue_v<D, HKV, PH>(a, page_of(xs), xs, lo, lane, vring + s * S::V_BYTES);
      issued += S::NVS;
      mv[s] = issued;
    }
  };
  // Paired halves stage no query rows in their K slots (the query comes
  // quantized), so their whole ring goes out at once; the others fill the
  // rest of theirs after the quantization.  (Issuing the whole ring first,
  // with the query rows in registers, was neutral at 4 x 131,072 tokens and
  // 0.1-0.4 us slower per step on short contexts.)
  if constexpr (RS && !PH) {
    // The query words came with the table entries: a use of them here puts
    // the compiler's wait for them before the ring loads (inline assembly it
    // does not count) instead of before the quantization.
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) asm volatile("" ::"v"(qraw[j][ks][0]), "v"(qraw[j][ks][1]));
  }
  fill_slot(0);
  if constexpr (PH || RS) {
#pragma unroll
    for (int s = 1; s < (RK > RV ? RK : RV); ++s) fill_slot(s);
  }
  wait_vm(issued - q_done);

  // Q rows of this head -> int8 B operands, quantized with the store's K rule
  // in float64 (oracle.py:22-40 applied to each query row); each wave
  // quantizes its own tiles (nt % NWH == w) and publishes them in LDS.
  if constexpr (PH) {
    // Rows past the live ones: zero operands (a caller's tile may hold
    // anything in its padding rows).
    constexpr int KSQ = CFG::DQ / 64;
#pragma unroll
    for (int nt = 0; nt < CFG::NTQ; ++nt) {
      if (nt % NWH != w || r0 + 16 * nt + n < rows) continue;
#pragma unroll
      for (int ks = 2 * half; ks < 2 * half + 2; ++ks)
        *reinterpret_cast<__attribute__((address_space(3))) v4i *>(qlds + ((nt * KSQ + ks) * kWave + lane) * 16) =
            (v4i){0, 0, 0, 0};
    }
  } else if (pre_q) {
    // The tile's codes already are the B operands: lane (n, g) of tile nt
    // takes row 16 nt + n, dims 64 ks + 16 g .. + 15; dead rows stay zero.
    // (PH: the two halves of a pair stage k-steps 2 half and 2 half + 1.)
    constexpr int DQ = CFG::DQ, KSQ = DQ / 64;
    const int8_t *tile = a.q8 + static_cast<int64_t>(b) * a.q8_seq_stride + static_cast<int64_t>(hq) * kPage * DQ;
    const float *scales = a.q8_scale + static_cast<int64_t>(b) * a.qs_seq_stride + hq * kPage;
#pragma unroll
    for (int nt = 0; nt < CFG::NTQ; ++nt) {
      if (nt % NWH != w) continue;
      const int jl = RS ? nt / NWH : nt;  // this wave's tile slot
      const int r = r0 + 16 * nt + n;
      const bool live = r < rows;
#pragma unroll
      for (int ks = 0; ks < KSQ; ++ks) {
        if (PH && (ks >> 1) != half) continue;
        const v4i frag = live ? *reinterpret_cast<const v4i *>(tile + static_cast<int64_t>(r) * DQ + 64 * ks + 16 * g)
                              : (v4i){0, 0, 0, 0};
        *reinterpret_cast<__attribute__((address_space(3))) v4i *>(qlds + ((nt * KSQ + ks) * kWave + lane) * 16) = frag;
      }
      const double c = static_cast<double>(live ? scales[r] : 0.f) * (static_cast<double>(kLog2e) / sqrt(static_cast<double>(DQ)));
      st.crow[jl] = fmaxf(static_cast<float>(c), 1e-30f);
      if (g == 0 && half == 0)
        reinterpret_cast<__attribute__((address_space(3))) float *>(qlds + CFG::Q_FRAG_BYTES)[nt * 16 + n] = st.crow[jl];
    }
  } else if constexpr (!PH) {
#pragma clang fp contract(off)
#pragma unroll
    for (int nt = 0; nt < CFG::NTQ; ++nt) {
      if (nt % NWH != w) continue;  // the partner wave quantizes this tile
      const int jl = RS ? nt / NWH : nt;  // this wave's tile slot
      const bool live = r0 + 16 * nt + n < rows;
      float x[KS][16];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const v4i zero = {0, 0, 0, 0};
        v4i w0, w1;
        if constexpr (RS) {
          w0 = live ? qraw[jl][ks][0] : zero;
          w1 = live ? qraw[jl][ks][1] : zero;
        } else {
          const lds_t *row = qstage + ((nt / NWH) * 16 + n) * 2 * D + 2 * (64 * ks + 16 * g);
          w0 = live ? *reinterpret_cast<const __attribute__((address_space(3))) v4i *>(row) : zero;
          w1 = live ? *reinterpret_cast<const __attribute__((address_space(3))) v4i *>(row + 16) : zero;
        }
        const uint32_t words[8] = {static_cast<uint32_t>(w0[0]), static_cast<uint32_t>(w0[1]),
                                   static_cast<uint32_t>(w0[2]), static_cast<uint32_t>(w0[3]),
                                   static_cast<uint32_t>(w1[0]), static_cast<uint32_t>(w1[1]),
                                   static_cast<uint32_t>(w1[2]), static_cast<uint32_t>(w1[3])};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          x[ks][2 * e] = half_bits_to_float(static_cast<uint16_t>(words[e] & 0xFFFFu), a.q_bf16);
          x[ks][2 * e + 1] = half_bits_to_float(static_cast<uint16_t>(words[e] >> 16), a.q_bf16);
        }
      }
      float amax = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(x[ks][e]));
      amax = xlane_max16_32(amax);
      const double scale = amax == 0.f ? 0.0 : static_cast<double>(amax) / 127.0;
      const double inv = amax == 0.f ? 0.0 : 1.0 / scale;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        uint32_t wq[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 16; ++e)
          wq[e >> 2] |= (static_cast<uint32_t>(k_rule_code(x[ks][e], inv)) & 0xFFu) << (8 * (e & 3));
        const v4i frag = (v4i){static_cast<int>(wq[0]), static_cast<int>(wq[1]), static_cast<int>(wq[2]),
                               static_cast<int>(wq[3])};
        *reinterpret_cast<__attribute__((address_space(3))) v4i *>(qlds + ((nt * KS + ks) * kWave + lane) * 16) = frag;
      }
      // score * log2(e) = dot * q_scale * k_scale * log2(e) / sqrt(D); kept > 0
      // so masked (-inf) scores never meet a zero factor.
      const double c = scale * (static_cast<double>(kLog2e) / sqrt(static_cast<double>(D)));
      st.crow[jl] = fmaxf(static_cast<float>(c), 1e-30f);
      if (g == 0)
        reinterpret_cast<__attribute__((address_space(3))) float *>(qlds + CFG::Q_FRAG_BYTES)[nt * 16 + n] = st.crow[jl];
    }
  }

  // Where the query rows were staged in K slots 1.., they have been read
  // (their values are quantized) and those slots can take chunk data.
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if constexpr (!PH && !RS) {
#pragma unroll
    for (int s = 1; s < (RK > RV ? RK : RV); ++s) fill_slot(s);
  }

  lds_int *flags = reinterpret_cast<lds_int *>(lds + CFG::FLAG_OFF);  // PH, RS: ready[WAVES] | done[WAVES]
  if constexpr (PH || RS) {
    pair_flag_set(flags + wave, 0, lane);
    pair_flag_set(flags + CFG::WAVES + wave, 0, lane);
  }
  {
    // Q fragments and row factors visible to both waves of the head.  A bare
    // barrier after the LDS writes: __syncthreads() would also wait for every
    // ring load in flight.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const float f =
          reinterpret_cast<const __attribute__((address_space(3))) float *>(qlds + CFG::Q_FRAG_BYTES)[tile_of(nt) * 16 + n];
      if constexpr (PH) {
        // f is the row's quantization scale (dead rows: zero operands, any factor)
        const double c = static_cast<double>(f) * (static_cast<double>(kLog2e) / sqrt(static_cast<double>(CFG::DQ)));
        st.crow[nt] = fmaxf(static_cast<float>(c), 1e-30f);
      } else {
        st.crow[nt] = f;
      }
    }
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    st.lsum[nt] = (v4f){0.f, 0.f, 0.f, 0.f};
    st.corr[nt] = (v4f){0.f, 0.f, 0.f, 0.f};
    st.m_run[nt] = -INFINITY;
    st.thr[nt] = -INFINITY;
#pragma unroll
    for (int dg = 0; dg < DG; ++dg)
#pragma unroll
      for (int j = 0; j < 8; ++j) st.O[nt][dg][j] = (v4f){0.f, 0.f, 0.f, 0.f};
  }

  // Two waves of one head share a SIMD (waves w and w + 4), and the SIMD
  // favours the older one: left alone, the first wave of each head ends its
  // loop about 15 us before the second at 4 x 131,072 tokens, which then runs
  // alone.  Each wave publishes its chunk count and yields issue priority
  // while it is ahead of its SIMD partner (90.4 -> 87.3 us there).  The
  // paired halves are coupled per chunk already and run worse with it.
  lds_int *prog = reinterpret_cast<lds_int *>(lds + CFG::FLAG_OFF);
  if constexpr (CFG::BALANCE) pair_flag_set(prog + wave, 0, lane);
  if constexpr (RS) {
    // Row split: both waves of the head (of each half-head, PH) multiply
    // every chunk of the split, in order; chunk c sits in the rings of the
    // waves with w = c % 2 (their (c / 2)-th own chunk; PH: its K halves in
    // the two half-head waves, each V half in its own).  An owner publishes a
    // chunk once its loads landed ("ready", counted in own chunks), every
    // wave publishes the chunks it has finished reading ("done"), and an
    // owner refills a slot only after every wave that reads it did, so each
    // chunk is fetched from HBM once.  No wave waits before publishing what
    // the others wait for, so every wait ends.
    const int hb = PH ? (h & ~1) : h;  // first (half-)head wave of this head
    const int nall = max(0, x1 - x0);
    for (int c = 0; c < nall; ++c) {
      const int wo = c & 1;            // w of the chunk's owners
      const bool own = wo == w;        // wave-uniform
      const int ko = c >> 1;           // the owners' chunk count
      const int sk = ko % RK, sv = ko % RV;
      if (own) {
        int mks = mk[0], mvs = mv[0];
#pragma unroll
        for (int s = 1; s < RK; ++s)
          if (sk == s) mks = mk[s];
#pragma unroll
        for (int s = 1; s < RV; ++s)
          if (sv == s) mvs = mv[s];
        wait_vm(issued - max(mks, mvs));
        pair_flag_set(flags + wave, ko + 1, lane);
      }
      const int ow = wo * HKV;         // owner waves: ow + hb (+ 1 for PH)
      if constexpr (PH) {
        pair_flag_wait(flags + ow + hb, ko + 1, lane);
        pair_flag_wait(flags + ow + hb + 1, ko + 1, lane);
      } else {
        if (!own) pair_flag_wait(flags + ow + h, ko + 1, lane);
      }
      const lds_t *vslot = lds + (ow + h) * CFG::WAVE_BYTES + RK * S::K_BYTES + sv * S::V_BYTES;
      const int x = x0 + c;
      const bool valid = page_of(x) >= 0;
      const int tbase = 32 * x;
      v4i sc[2][NT];
      if constexpr (PH) {
        const lds_t *klo = lds + (ow + hb) * CFG::WAVE_BYTES + sk * S::K_BYTES;
        const lds_t *khi = lds + (ow + hb + 1) * CFG::WAVE_BYTES + sk * S::K_BYTES;
        if (valid) chunk_qk_pair<NT, 2>(klo, khi, qlds + w * 4 * kWave * 16, lane, g, sc);
      } else {
        const lds_t *kslot = lds + (ow + h) * CFG::WAVE_BYTES + sk * S::K_BYTES;
        if (valid) chunk_qk<D, NT, 2>(kslot, qlds + w * KS * kWave * 16, lane, g, sc);
      }
      if (valid) chunk_softmax_pv<D, NT, PH>(st, sc, vslot, tbase, L0, lane, g, tbase + 32 > min_end);
      // This chunk's K and V slots have been read.
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      pair_flag_set(flags + CFG::WAVES + wave, c + 1, lane);
      if (own && (ko + RK < cnt || ko + RV < cnt)) {
        // Every reader of this wave's slots is done with chunk c: the head's
        // other w (PH: both its half-head waves) and, PH, the other half.
        const int xw = (1 - w) * HKV;
        if constexpr (PH) {
          pair_flag_wait(flags + CFG::WAVES + xw + hb, c + 1, lane);
          pair_flag_wait(flags + CFG::WAVES + xw + hb + 1, c + 1, lane);
          pair_flag_wait(flags + CFG::WAVES + (wave ^ 1), c + 1, lane);
        } else {
          pair_flag_wait(flags + CFG::WAVES + xw + h, c + 1, lane);
        }
        if (ko + RK < cnt) {
          const int xr = my0 + (ko + RK) * NWH;
          issue_k<D, HKV>(a, page_of(xr), xr, lo, kring + sk * S::K_BYTES);
          issued += S::NK;
#pragma unroll
          for (int s = 0; s < RK; ++s)
            if (sk == s) mk[s] = issued;
        }
        if (ko + RV < cnt) {
          const int xr = my0 + (ko + RV) * NWH;
          issue_v<D, HKV, PH>(a, page_of(xr), xr, lo, lane, vring + sv * S::V_BYTES);
          issued += S::NVS;
#pragma unroll
          for (int s = 0; s < RV; ++s)
            if (sv == s) mv[s] = issued;
        }
      }
    }
  } else
  for (int k = 0; k < cnt; ++k) {
    const int sk = k % RK, sv = k % RV;  // wave-uniform ring slots
    if constexpr (CFG::BALANCE) {
      pair_flag_set(prog + wave, k, lane);
      const int pk = __builtin_amdgcn_readfirstlane(*reinterpret_cast<const volatile lds_int *>(prog + (wave ^ 4)));
      if (k > pk)
        __builtin_amdgcn_s_setprio(0);
      else
        __builtin_amdgcn_s_setprio(1);
    }
    lds_t *kslot = kring + sk * S::K_BYTES;
    lds_t *vslot = vring + sv * S::V_BYTES;
    int mks = mk[0], mvs = mv[0];
#pragma unroll
    for (int s = 1; s < RK; ++s)
      if (sk == s) mks = mk[s];
#pragma unroll
    for (int s = 1; s < RV; ++s)
      if (sv == s) mvs = mv[s];
    // Steady state: the loads issued after this chunk's V group are exactly
    // those of the previous RV - 1 chunks; one compare picks that count.
    {
      const int n = issued - max(mks, mvs);
      if (n == CFG::STEADY_AFTER)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(CFG::STEADY_AFTER) : "memory");
      else
        wait_vm(n);
    }
    if constexpr (PH) {
      // This wave's half of chunk k is resident; wait for the other half.
      pair_flag_set(flags + wave, k + 1, lane);
      pair_flag_wait(flags + (wave ^ 1), k + 1, lane);
    }
    const bool valid = (valid_mask >> sk) & 1u;
    const int tbase = 32 * (my0 + k * NWH);
    v4i sc[2][NT];
    if constexpr (PH) {
      const lds_t *pslot = lds + (wave ^ 1) * CFG::WAVE_BYTES + sk * S::K_BYTES;
      if (valid) chunk_qk_pair<NT>(half ? pslot : kslot, half ? kslot : pslot, qlds, lane, g, sc);
      // Both K slots of chunk k have been read.
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      pair_flag_set(flags + CFG::WAVES + wave, k + 1, lane);
    } else {
      if (valid) chunk_qk<D, NT>(kslot, qlds, lane, g, sc);
    }
    if (CFG::K_EARLY && k + RK < cnt) {
      // The K reads of this slot have completed (their values fed the MFMAs).
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      const int xr = my0 + (k + RK) * NWH;
      const uint32_t v = static_cast<uint32_t>(issue_k<D, HKV>(a, page_of(xr), xr, lo, kslot));
      valid_mask = (valid_mask & ~(1u << sk)) | (v << sk);
      issued += S::NK;
#pragma unroll
      for (int s = 0; s < RK; ++s)
        if (sk == s) mk[s] = issued;
    }
    if (valid)
      chunk_softmax_pv<D, NT, PH>(st, sc, vslot, tbase, L0, lane, g, tbase + 32 > min_end);
    if (!CFG::K_EARLY && k + RK < cnt) {
      // The K reads of this slot have completed (their values fed the MFMAs);
      // PH: so have the other half's.
      if constexpr (PH) pair_flag_wait(flags + CFG::WAVES + (wave ^ 1), k + 1, lane);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      const int xr = my0 + (k + RK) * NWH;
      const uint32_t v = static_cast<uint32_t>(issue_k<D, HKV>(a, page_of(xr), xr, lo, kslot));
      valid_mask = (valid_mask & ~(1u << sk)) | (v << sk);
      issued += S::NK;
#pragma unroll
      for (int s = 0; s < RK; ++s)
        if (sk == s) mk[s] = issued;
    }
    if (k + RV < cnt) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      const int xr = my0 + (k + RV) * NWH;
      issue_v<D, HKV, PH>(a, page_of(xr), xr, lo, lane, vslot);
      issued += S::NVS;
#pragma unroll
      for (int s = 0; s < RV; ++s)
        if (sv == s) mv[s] = issued;
    }
  }

  finalize_output(st);

  // ---- combine the NWH waves of each head, then write the split state
  // (RS: each wave holds whole rows and writes them itself)
  if constexpr (NWH > 1 && !RS) {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __syncthreads();  // every ring is drained; reuse the LDS for the exchange
    float *xb = reinterpret_cast<float *>(lds_raw) + h * (CFG::XCHG_FLOATS);
    if (w == 1) {
      int e = 0;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        xb[(e++) * kWave + lane] = st.m_run[nt];
#pragma unroll
        for (int i = 0; i < 4; ++i) xb[(e++) * kWave + lane] = st.lsum[nt][i];
#pragma unroll
        for (int dg = 0; dg < DG; ++dg)
#pragma unroll
          for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) xb[(e++) * kWave + lane] = st.O[nt][dg][j][i];
      }
    }
    __syncthreads();
    if (w != 0) return;
    int e = 0;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const float m1 = xb[(e++) * kWave + lane];
      const float m0 = st.m_run[nt];
      const float M = fmaxf(m0, m1);
      const float a0 = m0 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m0 - M);
      const float a1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - M);
      st.m_run[nt] = M;
      float a0i[4], a1i[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a0i[i] = __shfl(a0, 4 * g + i, kWave);
        a1i[i] = __shfl(a1, 4 * g + i, kWave);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) st.lsum[nt][i] = st.lsum[nt][i] * a0i[i] + xb[(e++) * kWave + lane] * a1i[i];
#pragma unroll
      for (int dg = 0; dg < DG; ++dg)
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            st.O[nt][dg][j][i] = st.O[nt][dg][j][i] * a0i[i] + xb[(e++) * kWave + lane] * a1i[i];
    }
  }

  // Split state: O normalized by the split's row sum, times 1/4, in fp16
  // (lane rows 16nt+4g+i, dims dg*128+8n+j: one 16-byte store per row and
  // dim group), then (m, l) in fp32.  A dequantized V value is at most
  // 15 * (65504 * 2 / 15) in magnitude, so a quarter of any average of them
  // is a finite fp16; the merge multiplies by 4 again (exact).  m and l of a
  // row go together (one 8-byte load per split in the merge).
  // (PH: each half writes its 128 dims of head hq's rows; m and l once.)
  constexpr int DQ = CFG::DQ, QH = CFG::QHEADS;
  char *base = a.ws + static_cast<int64_t>(role) * a.split_bytes;
  _Float16 *obase = reinterpret_cast<_Float16 *>(base);
  float2 *mlbase = reinterpret_cast<float2 *>(base + static_cast<int64_t>(QH) * rows * DQ * 2);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = r0 + 16 * tile_of(nt) + 4 * g + i;
      const float m_r = __shfl(st.m_run[nt], 4 * g + i, kWave);  // row r's max sits in lane n = 4 g + i
      if (r < rows) {
        const float l = st.lsum[nt][i];
        const float f = l > 0.f ? 0.25f / l : 0.f;
#pragma unroll
        for (int dg = 0; dg < DG; ++dg) {
          _Float16 *dst = obase + static_cast<int64_t>(hq * rows + r) * DQ + (half + dg) * 128 + 8 * n;
          const v8h o = {static_cast<_Float16>(st.O[nt][dg][0][i] * f), static_cast<_Float16>(st.O[nt][dg][1][i] * f),
                         static_cast<_Float16>(st.O[nt][dg][2][i] * f), static_cast<_Float16>(st.O[nt][dg][3][i] * f),
                         static_cast<_Float16>(st.O[nt][dg][4][i] * f), static_cast<_Float16>(st.O[nt][dg][5][i] * f),
                         static_cast<_Float16>(st.O[nt][dg][6][i] * f), static_cast<_Float16>(st.O[nt][dg][7][i] * f)};
          store_wt16(dst, o);
        }
        if (n == 0 && half == 0) store_wt8(mlbase + hq * rows + r, make_float2(m_r, l));
      }
    }
  }
}

// Two waves per 128-dim head, each holding up to three row tiles; four
// tiles (q_len 9-10) run split by rows (each wave two alternate tiles over
// every chunk, the chunks shared between the two waves' rings).
template <int HKV>
void launch_split(DecodeArgs a, int nt, hipStream_t s) {
  const dim3 grid(a.grid), block(128 * HKV);
  a.tile0 = 0;
  switch (nt) {
    case 1: decode_split_kernel<128, 1, HKV, 2><<<grid, block, 0, s>>>(a); break;
    case 2: decode_split_kernel<128, 2, HKV, 2><<<grid, block, 0, s>>>(a); break;
    case 3: decode_split_kernel<128, 3, HKV, 2><<<grid, block, 0, s>>>(a); break;
    default: decode_split_kernel<128, 2, HKV, 2, false, true><<<grid, block, 0, s>>>(a); break;
  }
}

// Head dim 256 runs as paired halves: 2 hkv 128-dim half-heads, two waves
// per SIMD (the 256-dim kernel holds one), from a query quantized by its own
// small kernel into the workspace.
bool paired_halves(int hkv, int head_dim) { return head_dim == 256 && (hkv == 2 || hkv == 4); }

void launch_split_pairs(DecodeArgs a, int nt, int hkv, hipStream_t s) {
  const dim3 grid(a.grid);
  a.tile0 = 0;
  if (hkv == 4) {
    // Eight half-head waves, one each: two per SIMD hold at most three row
    // tiles, so four run as a launch of three (rows 0-47) and one of one
    // (rows 48-63) writing disjoint rows of the same split states.
    switch (nt) {
      case 1: decode_split_kernel<128, 1, 8, 1, true><<<grid, dim3(512), 0, s>>>(a); break;
      case 2: decode_split_kernel<128, 2, 8, 1, true><<<grid, dim3(512), 0, s>>>(a); break;
      case 3: decode_split_kernel<128, 3, 8, 1, true><<<grid, dim3(512), 0, s>>>(a); break;
      default:
        decode_split_kernel<128, 3, 8, 1, true><<<grid, dim3(512), 0, s>>>(a);
        a.tile0 = 3;
        decode_split_kernel<128, 1, 8, 1, true><<<grid, dim3(512), 0, s>>>(a);
        break;
    }
    return;
  }
  switch (nt) {
    case 1: decode_split_kernel<128, 1, 4, 2, true><<<grid, dim3(512), 0, s>>>(a); break;
    case 2: decode_split_kernel<128, 2, 4, 2, true><<<grid, dim3(512), 0, s>>>(a); break;
    case 3: decode_split_kernel<128, 3, 4, 2, true><<<grid, dim3(512), 0, s>>>(a); break;
    default: decode_split_kernel<128, 2, 4, 2, true, true><<<grid, dim3(512), 0, s>>>(a); break;
  }
}

// Workspace bytes ahead of the split states: the quantized query tiles and
// their scales of a paired-halves call (256-byte aligned parts).
int64_t query_tile_bytes(int64_t batch, int hkv, int head_dim) {
  if (!paired_halves(hkv, head_dim)) return 0;
  const int64_t rows = batch * hkv * kPage;
  return ((rows * head_dim + 255) / 256) * 256 + ((rows * 4 + 255) / 256) * 256;
}

// One split's state: per KV head and query row, D fp16 outputs, then (m, l).
int64_t split_state_bytes(int hkv, int q_len, int head_dim) {
  return static_cast<int64_t>(hkv) * q_len * kGqa * (2 * head_dim + 8);
}

// Split work-groups for one call: about one per CU (two with two 128-dim
// heads, whose work-groups hold half the waves), never more than the pages,
// capped by the workspace and by an explicit request.  hkv counts the heads
// the waves serve (the half-heads of paired halves).
int64_t choose_grid(int64_t batch, int64_t table_width, int ppb, int hkv, int64_t ws_splits, int requested) {
  int64_t g = requested > 0 ? requested : static_cast<int64_t>(device_cus()) * (hkv < 4 ? 4 / hkv : 1);
  const int64_t pages = batch * table_width * ppb;
  if (g > pages) g = pages;
  if (g > ws_splits) g = ws_splits;
  if (g < batch) g = batch;
  return g;
}

}  // namespace
}  // namespace k8v4

extern "C" int64_t k8v4_attn_workspace_bytes(int64_t batch, int64_t table_width, int pages_per_block, int q_len,
                                             int hkv, int head_dim, int num_splits) {
  using namespace k8v4;
  if (batch < 1 || table_width < 1 || pages_per_block < 1 || q_len < 1 || !supported_heads(hkv) ||
      !supported_dim(head_dim))
    return -1;
  const int wave_heads = paired_halves(hkv, head_dim) ? 2 * hkv : hkv;
  const int64_t g = choose_grid(batch, table_width, pages_per_block, wave_heads, INT64_MAX, num_splits);
  return query_tile_bytes(batch, hkv, head_dim) + g * split_state_bytes(hkv, q_len, head_dim);
}

namespace k8v4 {
namespace {

int attn_batch(const void *q, int q_dtype, int64_t q_tok_stride, const int8_t *q8, const float *q8_scale,
               int64_t q8_seq_stride, int64_t qs_seq_stride, const int8_t *k_cache, const float *k_scale,
               const uint8_t *v_cache, const float *v_scale, const float *v_zero, int64_t num_pages,
               int64_t k_page_stride, int64_t ks_page_stride, int64_t v_page_stride, int64_t vs_page_stride,
               int64_t vz_page_stride, const int32_t *block_table, int64_t bt_stride, int64_t table_width,
               int pages_per_block, const int32_t *seq_lens, const int32_t *visible_lens, int64_t vis_stride,
               int64_t batch, int q_len, int hkv, int head_dim, void *out, int out_dtype,
               int64_t out_tok_stride, void *workspace, int64_t workspace_bytes, int num_splits,
               void *stream, hipEvent_t split_done, int stages) {
  clear_error();
  K8V4_REQUIRE(stages >= 1 && stages <= 3, "stages must be 1 (split), 2 (merge) or 3 (both)");
  K8V4_REQUIRE(supported_heads(hkv), "unsupported per-GPU KV head count %d (this library serves 2 or 4)", hkv);
  K8V4_REQUIRE(supported_dim(head_dim), "unsupported head dim %d (this library serves 128 or 256)", head_dim);
  K8V4_REQUIRE(q_len >= 1 && q_len * kGqa <= kPage, "q_len*GQA exceeds BM (q_len=%d)", q_len);
  K8V4_REQUIRE(pages_per_block >= 1, "pages_per_block");
  K8V4_REQUIRE(num_pages >= 1, "empty cache");
  K8V4_REQUIRE(batch >= 1 && batch < (1 << 24), "empty batch");
  K8V4_REQUIRE(table_width >= 1 && table_width * pages_per_block < (int64_t(1) << 30), "block_table width");
  if (q8) {
    K8V4_REQUIRE(q8_scale, "null pointer");
    K8V4_REQUIRE(reinterpret_cast<uintptr_t>(q8) % 16 == 0 && q8_seq_stride % 16 == 0 &&
                     q8_seq_stride >= int64_t(hkv) * kPage * head_dim && qs_seq_stride >= int64_t(hkv) * kPage,
                 "q8 must be 16-byte aligned [batch][hkv][64][head_dim] tiles with [batch][hkv][64] scales");
  } else {
    K8V4_REQUIRE(q_dtype == K8V4_F16 || q_dtype == K8V4_BF16, "q dtype must be fp16 or bf16");
  }
  K8V4_REQUIRE(out_dtype == K8V4_F16 || out_dtype == K8V4_BF16 || out_dtype == K8V4_F32,
               "out dtype must be fp16, bf16 or fp32");
  K8V4_REQUIRE((q || q8) && k_cache && k_scale && v_cache && v_scale && v_zero && block_table && seq_lens &&
                   out && workspace,
               "null pointer");
  if (!q8) {
    K8V4_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 && q_tok_stride % 8 == 0,
                 "q must be 16-byte aligned with a token stride that is a multiple of 8 elements");
    K8V4_REQUIRE(q_tok_stride >= int64_t(hkv) * kGqa * head_dim, "q token stride shorter than HQ*D");
    K8V4_REQUIRE(q_tok_stride * q_len < (int64_t(1) << 30), "q token stride too large");
  }
  K8V4_REQUIRE(out_tok_stride >= int64_t(hkv) * kGqa * head_dim, "out token stride shorter than HQ*D");
  K8V4_REQUIRE(bt_stride >= table_width, "block_table row stride shorter than its width");
  K8V4_REQUIRE(reinterpret_cast<uintptr_t>(k_cache) % 16 == 0 && k_page_stride % 16 == 0,
               "k_cache must keep 16-byte aligned rows");
  K8V4_REQUIRE(reinterpret_cast<uintptr_t>(v_cache) % 4 == 0 && v_page_stride % 4 == 0,
               "v_cache must keep 4-byte aligned rows");
  K8V4_REQUIRE(reinterpret_cast<uintptr_t>(k_scale) % 8 == 0 && reinterpret_cast<uintptr_t>(v_scale) % 8 == 0 &&
                   reinterpret_cast<uintptr_t>(v_zero) % 8 == 0 && ks_page_stride % 8 == 0 &&
                   vs_page_stride % 8 == 0 && vz_page_stride % 8 == 0,
               "scale planes must be 8-byte aligned");
  K8V4_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "workspace must be 16-byte aligned");
  if (visible_lens) K8V4_REQUIRE(vis_stride >= 1 + q_len, "visible_lens [B, 1+q_len]");

  const bool pairs = paired_halves(hkv, head_dim);
  const int64_t qt_bytes = query_tile_bytes(batch, hkv, head_dim);
  const int64_t split_bytes = split_state_bytes(hkv, q_len, head_dim);
  const int64_t ws_splits = workspace_bytes > qt_bytes ? (workspace_bytes - qt_bytes) / split_bytes : 0;
  const int64_t grid = choose_grid(batch, table_width, pages_per_block, pairs ? 2 * hkv : hkv, ws_splits, num_splits);
  if (grid > ws_splits) {
    set_error("K8/V4 workspace holds %lld split states, the batch needs at least %lld (%lld bytes each)",
              static_cast<long long>(ws_splits), static_cast<long long>(grid),
              static_cast<long long>(split_bytes));
    return K8V4_ERR_WORKSPACE;
  }

  DecodeArgs a;
  a.q = static_cast<const uint16_t *>(q);
  a.q_tok_stride = q_tok_stride;
  a.q_bf16 = q_dtype == K8V4_BF16;
  a.q8 = q8;
  a.q8_scale = q8_scale;
  a.q8_seq_stride = q8_seq_stride;
  a.qs_seq_stride = qs_seq_stride;
  a.k_cache = k_cache;
  a.k_scale = k_scale;
  a.v_cache = v_cache;
  a.v_scale = v_scale;
  a.v_zero = v_zero;
  a.num_pages = num_pages;
  {
    const int64_t dkv = reinterpret_cast<intptr_t>(v_scale) - reinterpret_cast<intptr_t>(k_scale);
    const int64_t dvz = reinterpret_cast<intptr_t>(v_zero) - reinterpret_cast<intptr_t>(v_scale);
    const int64_t lim = int64_t(1) << 30;
    a.planes_fast = ks_page_stride == vs_page_stride && vs_page_stride == vz_page_stride && dkv > -lim &&
                    dkv < lim && dvz > -lim && dvz < lim;
    a.d_kv = a.planes_fast ? dkv : 0;
    a.d_vz = a.planes_fast ? dvz : 0;
  }
  a.k_ps = k_page_stride;
  a.ks_ps = ks_page_stride;
  a.v_ps = v_page_stride;
  a.vs_ps = vs_page_stride;
  a.vz_ps = vz_page_stride;
  a.block_table = block_table;
  a.bt_stride = bt_stride;
  a.table_width = static_cast<int>(table_width);
  a.ppb = pages_per_block;
  a.seq_lens = seq_lens;
  a.visible = visible_lens;
  a.vis_stride = vis_stride;
  a.batch = static_cast<int>(batch);
  a.q_len = q_len;
  a.hkv = hkv;
  a.ws = static_cast<char *>(workspace) + qt_bytes;
  a.split_bytes = split_bytes;
  a.grid = static_cast<int>(grid);
  a.min_pages = 1;
  // Merge units: one work-group of TPU threads per column slice of an
  // output row.  The fewest slices (at least 8 columns of 8 dims each) and
  // the smaller work-group with which one thread folds at most one round of
  // kMergeMU splits of a sequence with the average split count G / batch
  // (one long sequence can own all G splits); otherwise the most threads per
  // column.
  const int nt = (q_len * kGqa + 15) / 16;
  int merge_tpu = 256;
  {
    const int vpr_max = head_dim / 8;
    const int64_t avg = (a.grid + batch - 1) / batch;
    int cs = vpr_max / 8;
    bool found = false;
    for (int tpu : {128, 256}) {
      for (int c = 1; vpr_max / c >= 8 && !found; c *= 2) {
        const int spi = tpu / (vpr_max / c);
        if ((avg + spi - 1) / spi <= kMergeMU) {
          cs = c;
          merge_tpu = tpu;
          found = true;
        }
      }
      if (found) break;
    }
    a.merge_cs = cs;
  }
  K8V4_REQUIRE(batch * q_len * kGqa * hkv * a.merge_cs <= INT32_MAX / 2, "batch too large for one merge launch");
  a.units = static_cast<int>(batch * q_len * kGqa * hkv * a.merge_cs);
  a.out = out;
  a.out_dtype = out_dtype;
  a.out_tok_stride = out_tok_stride;

  auto s = static_cast<hipStream_t>(stream);
  if (stages & 1) {
    if (pairs && !q8) {
      // The query tiles at the head of the workspace (query_tile_bytes).
      int8_t *tiles = static_cast<int8_t *>(workspace);
      float *scales = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                                ((batch * hkv * kPage * head_dim + 255) / 256) * 256);
      const int rc = q_quant_launch(q, a.q_bf16, 0, q_tok_stride, batch, q_len, hkv, head_dim, tiles, scales, s);
      if (rc) return rc;
      a.q8 = tiles;
      a.q8_scale = scales;
      a.q8_seq_stride = int64_t(hkv) * kPage * head_dim;
      a.qs_seq_stride = int64_t(hkv) * kPage;
    }
    if (pairs) {
      launch_split_pairs(a, nt, hkv, s);
    } else if (hkv == 4) {
      launch_split<4>(a, nt, s);
    } else {
      launch_split<2>(a, nt, s);
    }
    const int rc = launch_status("k8v4_attn_batch split");
    if (rc) return rc;
  }
  if (split_done) {
    const hipError_t e = hipEventRecord(split_done, s);
    if (e != hipSuccess) {
      set_error("k8v4_attn_batch: hipEventRecord: %s", hipGetErrorString(e));
      return K8V4_ERR_HIP;
    }
  }
  if (!(stages & 2)) return K8V4_OK;
  const dim3 mgrid(static_cast<unsigned>(a.units));
  if (merge_tpu == 128) {
    if (head_dim == 128)
      decode_merge_kernel<128, 128><<<mgrid, dim3(128), 0, s>>>(a);
    else
      decode_merge_kernel<256, 128><<<mgrid, dim3(128), 0, s>>>(a);
  } else {
    if (head_dim == 128)
      decode_merge_kernel<128, 256><<<mgrid, dim3(256), 0, s>>>(a);
    else
      decode_merge_kernel<256, 256><<<mgrid, dim3(256), 0, s>>>(a);
  }
  return launch_status("k8v4_attn_batch merge");
}

}  // namespace
}  // namespace k8v4

extern "C" int k8v4_attn_batch(const void *q, int q_dtype, int64_t q_tok_stride, const int8_t *k_cache,
                               const float *k_scale, const uint8_t *v_cache, const float *v_scale,
                               const float *v_zero, int64_t num_pages, int64_t k_page_stride,
                               int64_t ks_page_stride, int64_t v_page_stride, int64_t vs_page_stride,
                               int64_t vz_page_stride, const int32_t *block_table, int64_t bt_stride,
                               int64_t table_width, int pages_per_block, const int32_t *seq_lens,
                               const int32_t *visible_lens, int64_t vis_stride, int64_t batch, int q_len,
                               int hkv, int head_dim, void *out, int out_dtype, int64_t out_tok_stride,
                               void *workspace, int64_t workspace_bytes, int num_splits, void *stream) {
  return k8v4::attn_batch(q, q_dtype, q_tok_stride, nullptr, nullptr, 0, 0, k_cache, k_scale, v_cache, v_scale,
                          v_zero, num_pages, k_page_stride, ks_page_stride, v_page_stride, vs_page_stride,
                          vz_page_stride, block_table, bt_stride, table_width, pages_per_block, seq_lens,
                          visible_lens, vis_stride, batch, q_len, hkv, head_dim, out, out_dtype, out_tok_stride,
                          workspace, workspace_bytes, num_splits, stream, nullptr, 3);
}

// ------------------------------------------------- allocation-free entry point
// Split states of k8v4_attn_batch_noalloc: a library-owned device array (one
// copy per GPU the library runs on, held until the process ends).  Host code
// reaches it only through the device address hipGetSymbolAddress returns for
// the current device; the array's name is not a device address on the host.
// Every call on a GPU shares its copy: calls that overlap on one GPU race.
// Nothing in it must start at zero (each call writes every split state it
// reads before reading it).
constexpr int64_t kNoAllocScratchBytes = int64_t(32) << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace k8v4 {
namespace {

std::mutex g_scratch_mu;
void *g_scratch_ptr[64];

// The device address of `scratch` on the current device, resolved once per device.
int scratch_address(void **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64) {
    set_error("k8v4_attn_batch_noalloc: no usable current device (%s)", hipGetErrorString(e));
    return K8V4_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("k8v4_attn_batch_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
      return K8V4_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return K8V4_OK;
}

}  // namespace
}  // namespace k8v4

extern "C" int64_t k8v4_attn_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int64_t k8v4_decode_fault_count(void) {
  using namespace k8v4;
  clear_error();
  int n = 0;
  const hipError_t e = hipMemcpyFromSymbol(&n, HIP_SYMBOL(g_pair_wait_timeouts), sizeof(n));
  if (e != hipSuccess) {
    set_error("k8v4_decode_fault_count: %s", hipGetErrorString(e));
    return -1;
  }
  return n;
}

extern "C" int k8v4_attn_batch_noalloc(const void *q, int q_dtype, int64_t q_tok_stride, const int8_t *k_cache,
                                       const float *k_scale, const uint8_t *v_cache, const float *v_scale,
                                       const float *v_zero, int64_t num_pages, int64_t k_page_stride,
                                       int64_t ks_page_stride, int64_t v_page_stride, int64_t vs_page_stride,
                                       int64_t vz_page_stride, const int32_t *block_table, int64_t bt_stride,
                                       int64_t table_width, int pages_per_block, const int32_t *seq_lens,
                                       const int32_t *visible_lens, int64_t vis_stride, int64_t batch, int q_len,
                                       int hkv, int head_dim, void *out, int out_dtype, int64_t out_tok_stride,
                                       int num_splits, void *stream) {
  using namespace k8v4;
  clear_error();
  const int64_t need =
      k8v4_attn_workspace_bytes(batch, table_width, pages_per_block, q_len, hkv, head_dim, num_splits);
  K8V4_REQUIRE(supported_heads(hkv), "unsupported per-GPU KV head count %d (this library serves 2 or 4)", hkv);
  K8V4_REQUIRE(need >= 0, "bad shape for the decode workspace");
  if (need > kNoAllocScratchBytes) {
    set_error("k8v4_attn_batch_noalloc: the call needs %lld bytes of split states (and, at head dim 256 with "
              "two KV heads, the quantized query tile), the library-owned buffer holds %lld (use "
              "k8v4_attn_batch with a caller workspace)",
              static_cast<long long>(need), static_cast<long long>(kNoAllocScratchBytes));
    return K8V4_ERR_WORKSPACE;
  }
  void *ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc) return rc;
  return attn_batch(q, q_dtype, q_tok_stride, nullptr, nullptr, 0, 0, k_cache, k_scale, v_cache, v_scale, v_zero,
                    num_pages, k_page_stride, ks_page_stride, v_page_stride, vs_page_stride, vz_page_stride,
                    block_table, bt_stride, table_width, pages_per_block, seq_lens, visible_lens, vis_stride, batch,
                    q_len, hkv, head_dim, out, out_dtype, out_tok_stride, ws, kNoAllocScratchBytes, num_splits,
                    stream, nullptr, 3);
}

extern "C" int k8v4_attn_batch_q8(const int8_t *q8, const float *q_scale, int64_t q8_seq_stride,
                                  int64_t qs_seq_stride, const int8_t *k_cache, const float *k_scale,
                                  const uint8_t *v_cache, const float *v_scale, const float *v_zero,
                                  int64_t num_pages, int64_t k_page_stride, int64_t ks_page_stride,
                                  int64_t v_page_stride, int64_t vs_page_stride, int64_t vz_page_stride,
                                  const int32_t *block_table, int64_t bt_stride, int64_t table_width,
                                  int pages_per_block, const int32_t *seq_lens, const int32_t *visible_lens,
                                  int64_t vis_stride, int64_t batch, int q_len, int hkv, int head_dim, void *out,
                                  int out_dtype, int64_t out_tok_stride, void *workspace, int64_t workspace_bytes,
                                  int num_splits, void *stream) {
  if (!q8) {
    k8v4::clear_error();
    k8v4::set_error("null pointer");
    return K8V4_ERR_ARG;
  }
  return k8v4::attn_batch(nullptr, K8V4_F16, 0, q8, q_scale, q8_seq_stride, qs_seq_stride, k_cache, k_scale,
                          v_cache, v_scale, v_zero, num_pages, k_page_stride, ks_page_stride, v_page_stride,
                          vs_page_stride, vz_page_stride, block_table, bt_stride, table_width, pages_per_block,
                          seq_lens, visible_lens, vis_stride, batch, q_len, hkv, head_dim, out, out_dtype,
                          out_tok_stride, workspace, workspace_bytes, num_splits, stream, nullptr, 3);
}

extern "C" int k8v4_attn_batch_profiled(const void *q, int q_dtype, int64_t q_tok_stride, const int8_t *k_cache,
                                        const float *k_scale, const uint8_t *v_cache, const float *v_scale,
                                        const float *v_zero, int64_t num_pages, int64_t k_page_stride,
                                        int64_t ks_page_stride, int64_t v_page_stride, int64_t vs_page_stride,
                                        int64_t vz_page_stride, const int32_t *block_table, int64_t bt_stride,
                                        int64_t table_width, int pages_per_block, const int32_t *seq_lens,
                                        const int32_t *visible_lens, int64_t vis_stride, int64_t batch,
                                        int q_len, int hkv, int head_dim, void *out, int out_dtype,
                                        int64_t out_tok_stride, void *workspace, int64_t workspace_bytes,
                                        int num_splits, void *stream, void *split_done_event, int stages) {
  return k8v4::attn_batch(q, q_dtype, q_tok_stride, nullptr, nullptr, 0, 0, k_cache, k_scale, v_cache, v_scale,
                          v_zero, num_pages, k_page_stride, ks_page_stride, v_page_stride, vs_page_stride,
                          vz_page_stride, block_table, bt_stride, table_width, pages_per_block, seq_lens,
                          visible_lens, vis_stride, batch, q_len, hkv, head_dim, out, out_dtype, out_tok_stride,
                          workspace, workspace_bytes, num_splits, stream, static_cast<hipEvent_t>(split_done_event),
                          stages);
}
