"""Backend registry (vllm/v1/attention/backends/registry.py)."""
import enum


class AttentionBackendEnum(enum.Enum):
    FLASH_ATTN = "flash_attn"
    ROCM_ATTN = "rocm_attn"
    CUSTOM = "custom"


REGISTRY: dict = {}


def register_backend(member):
    def deco(cls):
        REGISTRY[member] = cls
        return cls

    return deco
