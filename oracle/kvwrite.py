"""CPU oracle for the KV-cache writer / quantiser. TEST INFRASTRUCTURE ONLY.

Only tests/ and __graft_entry__.smoke() may use this module, and only as the checker; the
operator never calls it and has no CPU fallback.

The int8 per-token-head row (vLLM's format, kernels/pth_dec/pth_dec.cpp:25-41) is
[K int8 x256 | k_scale f32 | V int8 x256 | v_scale f32]. vLLM's cache update that produces it
(do_kv_cache_update, called at upstream/pr-dflash2/0002-...patch:81-87) lives in the un-vendored
fork KIntegrated/vllm-gfx906-mobydick 0.30.0 and is not in the reference; this restates the
closed form the rows are defined by (per (token, kv head), symmetric absmax / 127):
    scale = absmax(x) / 127        (float32; 0 for an all-zero row)
    q     = clamp(rint(x / scale), -127, 127), x / scale correctly rounded in float32,
            rint rounding half to even; q = 0 when scale == 0
Slots follow vLLM's slot_mapping: slot = block * block_size + offset; negative slots (padding)
are not written.

Parity status: pinned by tests/test_kvwrite_oracle.py (closed forms, ties, the round-trip bound,
agreement with the independent torch quantiser in mi50-vllm-lab_amd/kvcache.py). vLLM's own
writer cannot run here (vLLM is absent): parity with it is unpinned.
"""
from __future__ import annotations

import numpy as np

HEAD_DIM = 256


def _np(x):
    if hasattr(x, "detach"):
        return x.detach().cpu().numpy()
    return np.asarray(x)


def quantize_rows(x) -> tuple[np.ndarray, np.ndarray]:
    """int8 q [..., 256] and float32 scale [...] of float rows x [..., 256]."""
    xf = _np(x).astype(np.float32)
    amax = np.max(np.abs(xf), axis=-1)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    safe = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)
    with np.errstate(invalid="ignore"):
        q = np.clip(np.rint(xf / safe[..., None]), -127, 127)
    q = np.where((scale > 0)[..., None], q, 0).astype(np.int8)
    return q, scale


def write_rows(key, value, key_cache, value_cache, k_scale, v_scale, slot_mapping) -> None:
    """Quantise key/value [T, Hkv, 256] and write them into the cache views (CPU tensors or arrays,
    modified in place) at slot_mapping [T]; negative slots and slots past the cache are skipped."""
    kc, vc, ks, vs = _np(key_cache), _np(value_cache), _np(k_scale), _np(v_scale)
    kq, kscale = quantize_rows(key)
    vq, vscale = quantize_rows(value)
    nblk, bs = kc.shape[0], kc.shape[1]
    slots = _np(slot_mapping).astype(np.int64)
    for t, slot in enumerate(slots):
        if slot < 0 or slot >= nblk * bs:
            continue
        blk, off = int(slot // bs), int(slot % bs)
        kc[blk, off, :, :HEAD_DIM] = kq[t]
        vc[blk, off, :, :HEAD_DIM] = vq[t]
        ks[blk, off, :] = kscale[t]
        vs[blk, off, :] = vscale[t]
