"""MI355X (gfx950) int8-KV paged decode attention: the `_gfx906_pth_dec` operator of
0c33/mi50-vllm-lab rebuilt for CDNA4.

The directory name is not a Python identifier; load it with `load_package()` from
`__graft_entry__` / `tests/conftest.py`, which registers it as `mi50_vllm_lab_amd`.
"""
from . import kvcache, pth_dec  # noqa: F401
from .pth_dec import decode, supported_layout  # noqa: F401

__all__ = ["decode", "supported_layout", "kvcache", "pth_dec"]
