"""MI355X (gfx950) int8-KV paged attention: the `_gfx906_pth_dec` decode operator and the
`_gfx906_fa_pth` chunked-prefill operator of 0c33/mi50-vllm-lab rebuilt for CDNA4, the KV-cache
writer that produces their rows, and the vLLM routing shim.

The directory name is not a Python identifier; load it with `load_package()` from
`__graft_entry__` / `tests/conftest.py`, which registers it as `mi50_vllm_lab_amd`.
"""
from . import kvcache, pth_dec, vllm_shim  # noqa: F401
from .pth_dec import cache_write, decode, forward_pth, supported_layout  # noqa: F401

__all__ = ["cache_write", "decode", "forward_pth", "supported_layout", "kvcache", "pth_dec", "vllm_shim"]
