/*
 * C ABI of the MI355X (gfx950) k8v4 quantized paged-KV attention library.
 *
 * Plain pointers and sizes only.  Every device pointer is a HIP device
 * address; `stream` is a hipStream_t passed as void* (NULL = the default
 * stream).  Every call only enqueues work on `stream`: no host sync, no device
 * allocation, no device->host read, so each entry point can be captured in a
 * HIP graph.  Calls return K8V4_OK or an error code; k8v4_last_error() gives
 * the message of the calling thread's last failure.
 *
 * Cache description (all entry points): the five regions of the reference
 * page format (k8v4_v030/layout.py:213-256) are passed as base pointers plus
 * a page stride in BYTES each.  Within a page every region is
 * [64 tokens][hkv heads][...] with fixed inner strides:
 *   k_cache  int8   [.., 64, hkv, head_dim]
 *   v_cache  uint8  [.., 64, hkv, head_dim/2]   (low nibble = even dim)
 *   k_scale, v_scale, v_zero  float32 [.., 64, hkv]
 * When the five views come from one allocation (cache_views.bind_regions) all
 * five page strides equal the page size in bytes.
 *
 * Supported shapes: hkv in {2, 4}, query heads = 6 * hkv, head_dim in {128, 256}.
 */
#ifndef K8V4_ABI_H
#define K8V4_ABI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Version 3: at head dim 256 with four KV heads too, the decode workspace
 * holds the quantized query tile ahead of the split states (k8v4_attn_batch
 * runs every 256-dim cache as paired 128-dim halves).  Version 2: the same
 * at head dim 256 with two KV heads, and k8v4_attn_workspace_bytes counts it
 * (a workspace sized as splits x state bytes alone holds fewer splits).
 * Version 1: the first release.
 */
#define K8V4_ABI_VERSION 3

enum {
  K8V4_OK = 0,
  K8V4_ERR_ARG = 1,       /* bad shape, stride, dtype, head count or null pointer */
  K8V4_ERR_WORKSPACE = 2, /* caller workspace smaller than the call needs */
  K8V4_ERR_HIP = 3        /* a HIP runtime call or kernel launch failed */
};

enum { K8V4_F16 = 0, K8V4_BF16 = 1, K8V4_F32 = 2 };

/* Query layouts of k8v4_q_quant. */
enum {
  K8V4_Q_TOKENS = 0, /* token rows [ntok, 6*hkv, head_dim], token stride q_tok_stride */
  K8V4_Q_PADDED = 1  /* the padded tile [hkv, 64, head_dim] itself */
};

int k8v4_abi_version(void);

/* Message of this thread's last failed call ("" if none). */
const char *k8v4_last_error(void);

/*
 * Quantize-and-write (replaces torch.ops.xe2_kv.kv_store_paged,
 * k8v4_v030/native/xe2_kv_ops.cpp:1411-1442, and its two kernels :536-627).
 *
 * k, v: [ntok, hkv, head_dim] of `src_dtype` (K8V4_F16 or K8V4_BF16), head
 * stride head_dim, dim stride 1, token stride k_tok_stride / v_tok_stride in
 * ELEMENTS.  slot_mapping: int64 [ntok].  Token t is written to page
 * slot/64, row slot%64; slot < 0 or page >= num_pages writes nothing.
 * Codes and scales follow k8v4_v030/oracle.py:18-69 bit for bit (float64
 * arithmetic, scales stored as fp32 round-to-nearest-even).
 */
int k8v4_kv_store_paged(const void *k, const void *v, int src_dtype, int64_t k_tok_stride,
                        int64_t v_tok_stride, const int64_t *slot_mapping, int64_t ntok, int hkv,
                        int head_dim, int8_t *k_cache, float *k_scale, uint8_t *v_cache,
                        float *v_scale, float *v_zero, int64_t num_pages, int64_t k_page_stride,
                        int64_t ks_page_stride, int64_t v_page_stride, int64_t vs_page_stride,
                        int64_t vz_page_stride, void *stream);

/*
 * K-only and V-only quantize-and-write (replace torch.ops.xe2_kv.k_store_paged
 * and v_store_paged, k8v4_v030/native/xe2_kv_ops.cpp:1371-1409): the K half or
 * the V half of k8v4_kv_store_paged, same rules, same skipped slots.
 */
int k8v4_k_store_paged(const void *k, int src_dtype, int64_t k_tok_stride, const int64_t *slot_mapping,
                       int64_t ntok, int hkv, int head_dim, int8_t *k_cache, float *k_scale, int64_t num_pages,
                       int64_t k_page_stride, int64_t ks_page_stride, void *stream);
int k8v4_v_store_paged(const void *v, int src_dtype, int64_t v_tok_stride, const int64_t *slot_mapping,
                       int64_t ntok, int hkv, int head_dim, uint8_t *v_cache, float *v_scale, float *v_zero,
                       int64_t num_pages, int64_t v_page_stride, int64_t vs_page_stride, int64_t vz_page_stride,
                       void *stream);

/*
 * Query quantization into the int8 Q-once tile (replaces torch.ops.xe2_kv.q_quant_once
 * and the pack-and-quantize step of int8k_int4v_s1_varlen_from_q,
 * k8v4_v030/native/xe2_kv_ops.cpp:205-294, :1248-1265, :1670-1690).
 * q8: int8 [hkv][64][head_dim]; q_scale: fp32 [hkv][64].  Row r of head h is
 * query token r / 6 of query head h*6 + r % 6 (K8V4_Q_TOKENS, ntok*6 <= 64;
 * rows from ntok*6 on get zero codes and scale) or row r of the padded input
 * (K8V4_Q_PADDED).  Codes follow the K rule of k8v4_v030/oracle.py:22-40 in
 * float64, the rule the decode kernels apply to fp16/bf16 queries.
 */
int k8v4_q_quant(const void *q, int q_dtype, int layout, int64_t q_tok_stride, int64_t ntok, int hkv,
                 int head_dim, int8_t *q8, float *q_scale, void *stream);

/*
 * Paged decode / MTP verify for a batch with one common query length
 * (replaces torch.ops.xe2_kv.int8k_int4v_attn_batch,
 * k8v4_v030/native/xe2_kv_ops.cpp:1728-1775, with its stage-1 kernel :629-845
 * and stage-2 merge :1057-1220).
 *
 * q:   [batch*q_len, 6*hkv, head_dim] (K8V4_F16 or K8V4_BF16), head stride
 *      head_dim, dim stride 1, token stride q_tok_stride elements (multiple
 *      of 8, base 16-byte aligned).  Row b*q_len + j is query token j of
 *      sequence b.  Each row is int8-quantized with the K rule in the kernel.
 * block_table: int32 [batch][bt_stride], first table_width entries used;
 *      entry e covers kernel pages e*pages_per_block .. +pages_per_block-1.
 * seq_lens: int32 [batch] (device).  visible_lens: NULL or int32
 *      [batch][vis_stride] with [0] = page-valid length and [1+j] = causal
 *      end of token j; without it the end of token j is
 *      seq_len - q_len + j + 1.  A row with no visible key outputs zeros.
 * out: [batch*q_len, 6*hkv, head_dim] of out_dtype, token stride out_tok_stride.
 * workspace: caller-owned device scratch (16-byte aligned) of
 *      workspace_bytes; k8v4_attn_workspace_bytes() gives what a call needs:
 *      the split states and, for head_dim 256, ahead of them the
 *      query quantized by a first kernel (per sequence and KV head 64 rows of
 *      256 int8 codes, then the rows' fp32 scales).
 * num_splits: split-K work-groups (0 = about one per CU).
 * Requires 1 <= q_len and q_len*6 <= 64.
 */
int k8v4_attn_batch(const void *q, int q_dtype, int64_t q_tok_stride, const int8_t *k_cache,
                    const float *k_scale, const uint8_t *v_cache, const float *v_scale,
                    const float *v_zero, int64_t num_pages, int64_t k_page_stride,
                    int64_t ks_page_stride, int64_t v_page_stride, int64_t vs_page_stride,
                    int64_t vz_page_stride, const int32_t *block_table, int64_t bt_stride,
                    int64_t table_width, int pages_per_block, const int32_t *seq_lens,
                    const int32_t *visible_lens, int64_t vis_stride, int64_t batch, int q_len,
                    int hkv, int head_dim, void *out, int out_dtype, int64_t out_tok_stride,
                    void *workspace, int64_t workspace_bytes, int num_splits, void *stream);

/*
 * k8v4_attn_batch over pre-quantized queries (replaces torch.ops.xe2_kv.
 * int8k_int4v_s1_paged and int8k_int4v_s1_varlen_paged, k8v4_v030/native/
 * xe2_kv_ops.cpp:1628-1660, which take the Q-once tile k8v4_q_quant writes).
 * q8 / q_scale: per sequence one tile as k8v4_q_quant writes it, sequences
 * q8_seq_stride / qs_seq_stride elements apart (q8 16-byte aligned, stride a
 * multiple of 16).  Every other argument as k8v4_attn_batch.
 */
int k8v4_attn_batch_q8(const int8_t *q8, const float *q_scale, int64_t q8_seq_stride, int64_t qs_seq_stride,
                       const int8_t *k_cache, const float *k_scale, const uint8_t *v_cache, const float *v_scale,
                       const float *v_zero, int64_t num_pages, int64_t k_page_stride, int64_t ks_page_stride,
                       int64_t v_page_stride, int64_t vs_page_stride, int64_t vz_page_stride,
                       const int32_t *block_table, int64_t bt_stride, int64_t table_width, int pages_per_block,
                       const int32_t *seq_lens, const int32_t *visible_lens, int64_t vis_stride, int64_t batch,
                       int q_len, int hkv, int head_dim, void *out, int out_dtype, int64_t out_tok_stride,
                       void *workspace, int64_t workspace_bytes, int num_splits, void *stream);

/*
 * k8v4_attn_batch for timing its two kernels apart.  `split_done_event`
 * (a hipEvent_t as void*, or NULL) is recorded on `stream` after the split-K
 * kernel.  `stages` selects the kernels: 1 = split-K only (fills the
 * workspace, leaves `out` untouched), 2 = merge only (reads the workspace a
 * previous stages=1 call with the same arguments filled), 3 = both, which is
 * exactly k8v4_attn_batch.  No counterpart in the reference (its S1/S2
 * timing was an environment-driven host-synchronising log inside the op,
 * k8v4_v030/native/xe2_kv_ops.cpp:1603-1621).
 */
int k8v4_attn_batch_profiled(const void *q, int q_dtype, int64_t q_tok_stride,
                             const int8_t *k_cache, const float *k_scale, const uint8_t *v_cache,
                             const float *v_scale, const float *v_zero, int64_t num_pages,
                             int64_t k_page_stride, int64_t ks_page_stride, int64_t v_page_stride,
                             int64_t vs_page_stride, int64_t vz_page_stride,
                             const int32_t *block_table, int64_t bt_stride, int64_t table_width,
                             int pages_per_block, const int32_t *seq_lens,
                             const int32_t *visible_lens, int64_t vis_stride, int64_t batch,
                             int q_len, int hkv, int head_dim, void *out, int out_dtype,
                             int64_t out_tok_stride, void *workspace, int64_t workspace_bytes,
                             int num_splits, void *stream, void *split_done_event, int stages);

/*
 * Chunked prefill of one sequence over the quantized cache (replaces the
 * prefill paths of k8v4_v030: eager_prefill, dequant.py:213-242;
 * head_major_prefill, onednn_prefill.py:188-241; and the fused fp16 SDPA it
 * calls, torch.ops.k8v4_sdpa.sdpa_len, native/k8v4_sdpa.cpp:232-238).
 *
 * q:   [q_len, 6*hkv, head_dim] (K8V4_F16 or K8V4_BF16, bf16 is rounded to
 *      fp16 first), token stride q_tok_stride elements (multiple of 8, base
 *      16-byte aligned); not quantized.
 * block_row: int32 [table_width] table row of the sequence (entry e covers
 *      kernel pages e*pages_per_block .. +pages_per_block-1).
 * Query row j is token seq_len - q_len + j and attends to keys
 * t <= seq_len - q_len + j (bottom-right causal); K and V are the cache's
 * codes dequantized as dequant.py:96-106 (K as code * k_scale rounded once
 * to fp16 on the MFMA tile, V exact); softmax(scale * q.k), fp32
 * accumulation.
 * out: [q_len, 6*hkv, head_dim] of out_dtype, token stride out_tok_stride
 *      (multiple of 4, base 16-byte aligned).
 * workspace: caller-owned device scratch (16-byte aligned) of workspace_bytes
 *      >= k8v4_prefill_workspace_bytes(seq_len, q_len, hkv, head_dim): partial
 *      softmax states of the row blocks the balanced schedule splits between
 *      work-groups and, for head_dim 128 with q_len * 6 > 768 query rows per
 *      KV head, one head's pages dequantized into MFMA tile images (35,840
 *      bytes per 64-token page; the heads run one after another over it).
 * q_len == 0 is a no-op; q_len > seq_len is an error.
 */
int k8v4_prefill_paged(const void *q, int q_dtype, int64_t q_tok_stride, const int8_t *k_cache,
                       const float *k_scale, const uint8_t *v_cache, const float *v_scale,
                       const float *v_zero, int64_t num_pages, int64_t k_page_stride,
                       int64_t ks_page_stride, int64_t v_page_stride, int64_t vs_page_stride,
                       int64_t vz_page_stride, const int32_t *block_row, int64_t table_width,
                       int pages_per_block, int64_t seq_len, int64_t q_len, int hkv, int head_dim,
                       float scale, void *out, int out_dtype, int64_t out_tok_stride,
                       void *workspace, int64_t workspace_bytes, void *stream);

/*
 * k8v4_prefill_paged over several sequences at once: the prefill chunks of
 * one engine step (replaces the reference's per-request loop in the
 * backend, backend.py:376-409 calling dequant.py:213-242 once per request).
 * Sequence i has q_lens[i] query rows at token tok0[i] of q and out (same
 * layouts and strides as k8v4_prefill_paged, shared by all sequences),
 * seq_lens[i] keys, and its block-table row at block_table + rows[i] *
 * bt_stride (table_width entries of pages_per_block pages).  tok0, q_lens,
 * seq_lens and rows are HOST arrays of nseq entries.  Per launch the kernels
 * take up to 10 non-empty sequences, whose (KV head, row block) work shares
 * the persistent work-groups of one launch; more sequences take more
 * launches, in order, on the stream.  Pages are dequantized in the kernel
 * (no per-head tile pre-pass), which suits short chunks: a long chunk is
 * faster through k8v4_prefill_paged.  The same bottom-right causal rule,
 * numerics and errors per sequence as k8v4_prefill_paged; q_lens[i] == 0
 * sequences are skipped; nseq == 0 is a no-op.  The library sees neither
 * the table's row count nor the token count of q and out: the caller keeps
 * rows[i] a row of the table and tok0[i] + q_lens[i] within q and out (the
 * Python op checks both against the tensors' shapes).
 * workspace: >= k8v4_prefill_batch_workspace_bytes(hkv, head_dim) bytes.
 */
int k8v4_prefill_paged_batch(const void *q, int q_dtype, int64_t q_tok_stride, const int8_t *k_cache,
                             const float *k_scale, const uint8_t *v_cache, const float *v_scale,
                             const float *v_zero, int64_t num_pages, int64_t k_page_stride,
                             int64_t ks_page_stride, int64_t v_page_stride, int64_t vs_page_stride,
                             int64_t vz_page_stride, const int32_t *block_table, int64_t bt_stride,
                             int64_t table_width, int pages_per_block, int nseq, const int64_t *tok0,
                             const int64_t *q_lens, const int64_t *seq_lens, const int64_t *rows, int hkv,
                             int head_dim, float scale, void *out, int out_dtype, int64_t out_tok_stride,
                             void *workspace, int64_t workspace_bytes, void *stream);

/* Workspace bytes k8v4_prefill_paged_batch needs (-1 on bad arguments):
 * the partial states of one launch, whatever its sequences.  No counterpart
 * in the reference. */
int64_t k8v4_prefill_batch_workspace_bytes(int hkv, int head_dim);

/*
 * k8v4_attn_batch without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * split states (and, at head dim 256, the quantized query
 * tile ahead of them) go to a library-owned device buffer of
 * k8v4_attn_noalloc_max_bytes() bytes (32 MiB) per GPU, held until the
 * process ends; a call whose k8v4_attn_workspace_bytes exceeds it returns
 * K8V4_ERR_WORKSPACE without launching anything.  The call allocates nothing
 * (no hipMalloc, no allocating library routine).  All calls on one GPU share
 * that buffer: calls that overlap on one GPU (other streams, other threads)
 * race and must not be issued.  Every other argument as k8v4_attn_batch.
 */
int k8v4_attn_batch_noalloc(const void *q, int q_dtype, int64_t q_tok_stride, const int8_t *k_cache,
                            const float *k_scale, const uint8_t *v_cache, const float *v_scale,
                            const float *v_zero, int64_t num_pages, int64_t k_page_stride,
                            int64_t ks_page_stride, int64_t v_page_stride, int64_t vs_page_stride,
                            int64_t vz_page_stride, const int32_t *block_table, int64_t bt_stride,
                            int64_t table_width, int pages_per_block, const int32_t *seq_lens,
                            const int32_t *visible_lens, int64_t vis_stride, int64_t batch, int q_len,
                            int hkv, int head_dim, void *out, int out_dtype, int64_t out_tok_stride,
                            int num_splits, void *stream);

/* Bytes of the library-owned buffer of k8v4_attn_batch_noalloc (split states
 * and, at head dim 256, the query tile). */
int64_t k8v4_attn_noalloc_max_bytes(void);

/*
 * Diagnostics, no counterpart in the reference: how many in-kernel waits of
 * the decode kernels on the current device gave up since the library was
 * loaded (the paired-halves handshake of head dim 256 caps
 * each wait; a give-up means a wrong output).  Synchronizes with the device
 * (a copy from device memory); -1 on a HIP error.  Zero in a correct run.
 */
int64_t k8v4_decode_fault_count(void);

/* Workspace bytes k8v4_prefill_paged needs (0 for q_len == 0, -1 on bad
 * arguments).  No counterpart in the reference (its prefill allocated its
 * gathered K/V per head inside the call, onednn_prefill.py:226-239). */
int64_t k8v4_prefill_workspace_bytes(int64_t seq_len, int64_t q_len, int hkv, int head_dim);

/* Whether k8v4_prefill_paged serves this shape from per-KV-head tile images
 * (each page dequantized once per head; 1), or converts pages in place as
 * k8v4_prefill_paged_batch does (0); -1 on bad arguments.  No counterpart in
 * the reference: a caller batching a step's chunks sends the former alone. */
int k8v4_prefill_uses_tiles(int64_t seq_len, int64_t q_len, int hkv, int head_dim);

/* Workspace bytes k8v4_attn_batch needs for this shape (-1 on bad arguments).
 * No counterpart in the reference (its caller sized [nprog, 64, D] fp32
 * partials, k8v4_v030/scratch.py:34-45, which is always at least this). */
int64_t k8v4_attn_workspace_bytes(int64_t batch, int64_t table_width, int pages_per_block,
                                  int q_len, int hkv, int head_dim, int num_splits);

#ifdef __cplusplus
}
#endif

#endif /* K8V4_ABI_H */
