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

#define K8V4_ABI_VERSION 1

enum {
  K8V4_OK = 0,
  K8V4_ERR_ARG = 1,       /* bad shape, stride, dtype, head count or null pointer */
  K8V4_ERR_WORKSPACE = 2, /* caller workspace smaller than the call needs */
  K8V4_ERR_HIP = 3        /* a HIP runtime call or kernel launch failed */
};

enum { K8V4_F16 = 0, K8V4_BF16 = 1, K8V4_F32 = 2 };

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

#ifdef __cplusplus
}
#endif

#endif /* K8V4_ABI_H */
