"""MI355X-native k8v4 quantized paged-KV attention (int8 K, packed int4 V).

Host surface of the reference package ``k8v4_v030`` (layout, cache_views,
plan, scratch, ops_api) over hand-written gfx950 HIP kernels reached through
the C ABI in ``include/k8v4_abi.h``.
"""
from .layout import CACHE_DTYPE, D, GQA, PAGE, PageLayout

__all__ = ["CACHE_DTYPE", "D", "GQA", "PAGE", "PageLayout"]
