"""KV cache spec (vllm/v1/kv_cache_interface.py)."""
from __future__ import annotations

import dataclasses


@dataclasses.dataclass(frozen=True)
class AttentionSpec:
    block_size: int
    num_kv_heads: int
    head_size: int
    dtype: object = None
    state_content_bytes: int | None = None
