"""vLLM's int8 per-token-head paged KV cache on the host side: the layout views the operators
take, cache allocation and copies, and the per-token-head quantiser.

Cache layout (one row per (block, slot, kv head), 520 bytes):
    [ K int8 x 256 | k_scale f32 | V int8 x 256 | v_scale f32 ]
Physical order is HND ([blocks, Hkv, block_size, 520]) or NHD ([blocks, block_size, Hkv, 520]).
The views handed to the operator follow kernels/pth_dec/test_dec.py:34-50: key_cache and
value_cache are int8 [blocks, block_size, Hkv, 260] (value_cache = key_cache + 260 bytes),
k_scale / v_scale are f32 [blocks, block_size, Hkv] aliasing bytes 256 / 516 of every row.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

HEAD_DIM = 256
HALF_ROW = 260    # K part: 256 int8 + f32 scale
ROW_BYTES = 520   # K part + V part
NAN_WORD = 0x7FC00000


@dataclass
class PagedKVCache:
    kv: torch.Tensor           # int8 [blocks, Hkv, block_size, 520] (strides give the physical order)
    key_cache: torch.Tensor    # int8 [blocks, block_size, Hkv, 260]
    value_cache: torch.Tensor  # int8 [blocks, block_size, Hkv, 260], 260 bytes after key_cache
    k_scale: torch.Tensor      # f32  [blocks, block_size, Hkv]
    v_scale: torch.Tensor      # f32  [blocks, block_size, Hkv]
    layout: str

    @property
    def num_blocks(self) -> int:
        return self.kv.shape[0]

    @property
    def num_kv_heads(self) -> int:
        return self.kv.shape[1]

    @property
    def block_size(self) -> int:
        return self.kv.shape[2]

    def nbytes(self) -> int:
        return self.kv.numel()


def cache_views(kv: torch.Tensor, layout: str) -> PagedKVCache:
    """Operator views over a raw int8 cache kv [blocks, Hkv, block_size, 520] (test_dec.py:44-50)."""
    assert kv.dtype == torch.int8 and kv.dim() == 4 and kv.shape[3] == ROW_BYTES and kv.storage_offset() == 0
    nblk, hkv, bs, _ = kv.shape
    f32 = torch.tensor([], dtype=torch.float32, device=kv.device).set_(kv.untyped_storage())
    st = [s // 4 for s in kv.stride()]
    ks = torch.as_strided(f32, (nblk, bs, hkv), (st[0], st[2], st[1]), HEAD_DIM // 4)
    vs = torch.as_strided(f32, (nblk, bs, hkv), (st[0], st[2], st[1]), (HALF_ROW + HEAD_DIM) // 4)
    kc, vc = kv.transpose(1, 2).split(HALF_ROW, dim=-1)
    return PagedKVCache(kv, kc, vc, ks, vs, layout)


def allocate_cache(num_blocks: int, block_size: int, num_kv_heads: int, layout: str = "HND",
                   device="cpu") -> PagedKVCache:
    if layout == "HND":
        kv = torch.zeros((num_blocks, num_kv_heads, block_size, ROW_BYTES), dtype=torch.int8, device=device)
    elif layout == "NHD":
        kv = torch.zeros((num_blocks, block_size, num_kv_heads, ROW_BYTES), dtype=torch.int8,
                         device=device).transpose(1, 2)
    else:
        raise ValueError(f"unknown layout {layout}")
    return cache_views(kv, layout)


def clone_cache(c: PagedKVCache, device=None) -> PagedKVCache:
    """Same bytes in a new buffer (same physical order), optionally on another device."""
    dev = device if device is not None else c.kv.device
    if c.layout == "HND":
        kv = c.kv.to(dev, copy=True).contiguous()
    else:
        kv = c.kv.transpose(1, 2).to(dev, copy=True).contiguous().transpose(1, 2)
    return cache_views(kv, c.layout)


def quantize_per_token_head(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric int8 per (token, kv head): scale = absmax / 127, q = clamp(round(x / scale), -127, 127).
    x: float [..., 256]. Rows that are all zero get scale 0 and q 0."""
    x = x.float()
    amax = x.abs().amax(dim=-1)
    scale = amax / 127.0
    safe = torch.where(scale > 0, scale, torch.ones_like(scale))
    q = torch.round(x / safe[..., None]).clamp_(-127, 127).to(torch.int8)
    q = torch.where((scale > 0)[..., None], q, torch.zeros_like(q))
    return q, scale
