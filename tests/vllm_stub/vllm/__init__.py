"""Minimal stand-in for the parts of vLLM 0.30's attention interface that the
K8/V4 backend imports (vllm/v1/attention/backend.py, backends/registry.py,
kv_cache_interface.py, logger.py).  Test infrastructure only: vLLM is not
installed in this image, and the tests put this directory on sys.path only
when ``import vllm`` fails."""
