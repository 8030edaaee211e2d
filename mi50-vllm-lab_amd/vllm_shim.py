"""Routing shim between vLLM's Triton attention backend and the gfx950 int8-KV operators.

Restates the reference's backend patch (patches/vllm/triton_attn.patch) for this library, in a
form that does not import vLLM (absent here): the backend keeps its own objects and passes the
few fields the routing reads.

- Loaders (triton_attn.patch:15-70): the library is loaded once per process and cached; an
  environment switch turns each path off, and a load failure logs a warning and leaves the
  backend on Triton. Both operators live in one library (libpthdec.so).
- Gating (triton_attn.patch:91-114): int8 per-token-head KV, ROCm, decoder attention, head
  size 256, no sinks / alibi / softcap / chunked lookback / TD, on gfx950. Prefill also needs no
  sliding window. Decode accepts a left sliding window (the operator implements the window
  rule) and any GQA group with qmax * G <= 48, where the reference required GQA 6 and no window.
- forward_pth_dec (triton_attn.patch:116-174): the cache layout is checked once; the call falls
  back (returns False) without the softmax segment buffers, with more query tokens than segment
  rows, or with query / output strides the operator does not take. nsplit = min(splits,
  segment count). With host-side sequence lengths (vLLM's seq_lens_cpu) the count is chosen by a
  makespan model of the partial kernel (one workgroup per CU; see decode_splits); without them a
  sliding window (every sequence sees at most window + qmax keys) caps it at CUs / (kv heads x
  sequences), so that the partial kernel runs in a single round.
- forward_pth_fa (triton_attn.patch:176-262): the sequences with >= MIN_Q query tokens must form
  a suffix of the batch; the rows before it go to the decode operator when every prefix sequence
  has <= 4 (8 with DFlash) query tokens, else to the caller's Triton function. Each suffix
  sequence runs the prefill operator once (no padding to a tile ladder is needed);
  VLLM_GFX950_PTH_FA_EXACT=1 selects its exact entry (pth_fa_forward_exact: the decode's
  numerics, for caches with very large per-token scales, at ~26 % more time).
- route (triton_attn.patch:272-308): prefill first when max_seqlen_q >= MIN_Q, then decode
  when max_seqlen_q <= MAX_Q; causal only, no multimodal prefix, no RSWA prefix, no output
  scale. Returns False when the caller must run its own path.
"""
from __future__ import annotations

import logging
import math
import os
from dataclasses import dataclass
from typing import Any, Callable, Optional

import numpy as np
import torch

from . import pth_dec as _pd

logger = logging.getLogger(__name__)

PTH_FA_MIN_Q = int(os.environ.get("VLLM_GFX950_PTH_FA_MIN_Q", "64"))
PTH_DEC_MAX_Q = int(os.environ.get("VLLM_GFX950_PTH_DEC_MAX_Q", "4"))
PTH_DEC_SPLITS = int(os.environ.get("VLLM_GFX950_PTH_DEC_SPLITS", "64"))
PTH_DEC_CUS = int(os.environ.get("VLLM_GFX950_PTH_DEC_CUS", "0"))  # 0: the device's CU count
PTH_FA_EXACT = os.environ.get("VLLM_GFX950_PTH_FA_EXACT", "0") == "1"  # prefill through pth_fa_forward_exact
MAX_ROWS_PER_KV_HEAD = 48  # qmax * G the decode operator takes

_dec_mod = None
_fa_mod = None
_cus = {}


def cu_count(device) -> int:
    """Compute units of `device` (cached; host-side query, no synchronisation). 256 for a CPU
    device (tests) unless VLLM_GFX950_PTH_DEC_CUS is set."""
    if PTH_DEC_CUS > 0:
        return PTH_DEC_CUS
    device = torch.device(device)
    if device.type != "cuda":
        return 256
    key = device.index if device.index is not None else torch.cuda.current_device()
    if key not in _cus:
        _cus[key] = torch.cuda.get_device_properties(key).multi_processor_count
    return _cus[key]


# Makespan model of the decode partial kernel (grid splits x kv heads x sequences, one
# workgroup per CU), fitted to MI355X measurements: a workgroup costs ~12 us of set-up and merge
# plus ~3.3 us per 32-key tile of its busiest wave (4 waves share a split's tiles); a split
# with no tiles ~2 us. The combine after it reads every split's partial row (1,032 bytes per
# (token, q head, split)) at ~4 TB/s: ~0.25 us per MB on top of a fixed cost that no split count
# changes.
SPLIT_FIXED_US, SPLIT_TILE_US, SPLIT_EMPTY_US = 12.0, 3.3, 2.0
COMBINE_US_PER_MB = 0.25
PARTIAL_ROW_BYTES = 1032

# The operator runs a windowed GQA group of more than 16 rows as 16-row slices, one workgroup
# each, when splits x kv heads x sequences x slices fits the CUs and sequences x window is at
# most SLICE_KEYS (pd_decode.hip, launch_partial). Measured on MI355X (24 q / 4 kv heads, us per
# layer, sliced at the best such split count against the best unsliced count): 4 x 8 rows over
# 2,048-key windows 19.7 (5) against 24.1 (16); 1 x 8 rows 13.2 (21) against 17.7 (32); 4 x 4
# rows 17.1 (8) against 19.1 (16); 2 x 8 rows over 4,096 keys 19.3 (10) against 25.2 (32);
# 8 x 8 rows over 1,024 keys 23.1 (2) against 26.8 (8); 1 x 8 rows over 8,192 keys 19.0 (21)
# against 24.8 (32), over 16,384 keys 24.9 (21) against 27.9 (64). Past SLICE_KEYS it lost: 4 x 8
# rows over 8,192 keys 41.4 (4) against 34.4 (16), 16 x 8 rows over 2,048 keys 46.8 (1) against
# 45.3 (4). The largest fitting count is taken when it is at least 2.
SLICE_KEYS = 16384


def sliced_splits(window: int, max_q: int, group: int, num_kv_heads: int, num_seqs: int, cus: int,
                  cap: int) -> int:
    """The split count at which the operator slices this windowed batch into one round of 16-row
    workgroups, or 0 when it would not (no window, sequences x window above SLICE_KEYS, at most
    16 rows per group, or fewer than 2 splits would fit)."""
    rows = max(1, max_q) * group
    if window <= 0 or window * max(1, num_seqs) > SLICE_KEYS or rows <= 16:
        return 0
    slices = -(-rows // 16)
    s = min(cap, cus // max(1, num_kv_heads * num_seqs * slices))
    return s if s >= 2 else 0


def decode_splits(nseg: int, window: int, num_kv_heads: int, num_seqs: int, device, seq_lens_host=None,
                  max_q: int = 1, num_q_heads: Optional[int] = None) -> int:
    """Splits per sequence for the decode operator, at most min(VLLM_GFX950_PTH_DEC_SPLITS, nseg).

    With the host-side sequence lengths, the candidate (powers of two and the cap) with the
    smallest modelled time: the partial kernel's makespan max(total workgroup time / CUs, longest
    workgroup) plus the combine's reading of the partials (num_seqs x max_q x num_q_heads rows,
    6 q heads per kv head when not given). Few splits for many sequences, many for one long
    sequence. Without the lengths: a sliding window bounds every sequence to about window + qmax
    keys, so the grid is sized to one workgroup per CU; otherwise the cap (the reference's
    rule). Before either: windowed groups of more than 16 rows take the count at which the
    operator slices them into one round of 16-row workgroups (sliced_splits), when that is at
    least 2."""
    cap = max(1, min(PTH_DEC_SPLITS, nseg))
    cus = cu_count(device)
    group = num_q_heads // num_kv_heads if num_q_heads else 6
    sliced = sliced_splits(window, max_q, group, num_kv_heads, num_seqs, cus, cap)
    if sliced:
        return sliced
    if seq_lens_host is None:
        if window > 0:
            return max(1, min(cap, cus // max(1, num_kv_heads * num_seqs)))
        return cap
    lens = np.asarray(seq_lens_host, dtype=np.int64).reshape(-1)[:num_seqs]
    if window > 0:
        lens = np.minimum(lens, window + max_q)
    tiles = (lens + 31) // 32 + (lens > 0)  # visible keys in 32-key tiles (+1: alignment)
    live = tiles > 0
    if not live.any():
        return 1
    rows = num_seqs * max(1, max_q) * (num_q_heads if num_q_heads else 6 * num_kv_heads)
    cands = sorted({1 << k for k in range(int(math.log2(cap)) + 1)} | {cap})
    best_s, best_t = cap, float("inf")
    for s in cands:
        per = np.maximum(-(-tiles // s), 1)              # tiles per split
        n = np.where(live, -(-tiles // per), 0)         # splits holding tiles
        t = SPLIT_FIXED_US + SPLIT_TILE_US * -(-per // 4)
        total = num_kv_heads * float(np.sum(n * t + (s - n) * SPLIT_EMPTY_US))
        span = max(total / cus, float(t[live].max()))
        span += COMBINE_US_PER_MB * rows * s * PARTIAL_ROW_BYTES / 1e6
        if span < best_t - 1e-9:
            best_s, best_t = s, span
    return best_s


def _capturing(device) -> bool:
    """True while a HIP graph is being captured on the current stream of `device`."""
    if torch.device(device).type != "cuda":
        return False
    return bool(torch.cuda.is_current_stream_capturing())


class _Operators:
    """The operator entry points the shim calls (the reference's torch-extension modules)."""

    def __init__(self, path: Optional[str]):
        _pd.load_library(path)
        self.supported_layout = _pd.supported_layout
        self.decode = _pd.decode
        self.forward_pth = _pd.forward_pth


def _load(env_switch: str, env_lib: str, what: str):
    path = os.environ.get(env_lib) or None
    if os.environ.get(env_switch, "1") != "1":
        return None
    if path is not None and not os.path.exists(path):
        logger.warning("gfx950: %s not found; %s stays on Triton", path, what)
        return None
    try:
        return _Operators(path)
    except Exception as e:  # keep serving on the Triton path
        logger.warning("gfx950: could not load %s (%s); %s stays on Triton", path or _pd.LIB_PATH, e, what)
        return None


def load_pth_dec():
    """The decode operator, or None (VLLM_GFX950_PTH_DEC=0 or load failure). Cached."""
    global _dec_mod
    if _dec_mod is None:
        _dec_mod = _load("VLLM_GFX950_PTH_DEC", "VLLM_GFX950_PTH_DEC_LIB", "decode") or False
    return _dec_mod or None


def load_pth_fa():
    """The prefill operator, or None (VLLM_GFX950_PTH_FA=0 or load failure). Cached."""
    global _fa_mod
    if _fa_mod is None:
        _fa_mod = _load("VLLM_GFX950_PTH_FA", "VLLM_GFX950_PTH_FA_LIB", "prefill") or False
    return _fa_mod or None


def reset_loaders() -> None:
    """Forget the cached loaders (tests)."""
    global _dec_mod, _fa_mod
    _dec_mod = None
    _fa_mod = None


@dataclass
class AttnMeta:
    """The fields of vLLM's TritonAttentionMetadata the routing reads."""
    query_start_loc: torch.Tensor            # int32 [B + 1], device
    query_start_loc_cpu: Any                 # the same offsets on the host (list or tensor)
    seq_lens: torch.Tensor                   # int32 [B], device
    block_table: torch.Tensor                # int32 [B, max_blocks], device
    max_seq_len: int = 0
    causal: bool = True
    softmax_segm_output: Optional[torch.Tensor] = None   # fp32 [T, Hq, nseg, 256]
    softmax_segm_max: Optional[torch.Tensor] = None      # fp32 [T, Hq, nseg]
    softmax_segm_expsum: Optional[torch.Tensor] = None   # fp32 [T, Hq, nseg]
    seq_lens_cpu: Optional[Any] = None                   # the same lengths on the host, if known
    mm_prefix_range_tensor: Optional[torch.Tensor] = None
    rswa_prefix_lens: Optional[torch.Tensor] = None


class Gfx950Int8Attention:
    """Per-layer routing state (the part of TritonAttentionImpl the patch adds)."""

    def __init__(self, *, num_heads: int, num_kv_heads: int, head_size: int, scale: float,
                 kv_quant_int8_per_token_head: bool, is_rocm: bool, is_decoder: bool,
                 sliding_window=(-1, -1), sinks=None, alibi_slopes=None, logits_soft_cap=0.0,
                 chunk_lookback: int = -1, use_td: bool = False, on_gfx950: bool = True,
                 max_q: int = PTH_DEC_MAX_Q):
        self.scale = float(scale)
        self.num_heads, self.num_kv_heads = num_heads, num_kv_heads
        self.pth_fa = None
        self.pth_dec = None
        self.layout_ok: Optional[bool] = None  # cache layout, checked on first use
        self.max_q = max_q
        # left window W: vLLM's sliding_window (W - 1, 0); -1 = none
        self.window = sliding_window[0] + 1 if sliding_window[0] >= 0 else -1
        common = (kv_quant_int8_per_token_head and is_rocm and is_decoder and head_size == 256 and sinks is None
                  and alibi_slopes is None and not logits_soft_cap and chunk_lookback == -1 and not use_td
                  and on_gfx950)
        if not common:
            return
        if self.window < 0 and sliding_window[1] < 0:
            self.pth_fa = load_pth_fa()
        G = num_heads // num_kv_heads if num_kv_heads > 0 else 0
        if num_heads % max(num_kv_heads, 1) == 0 and 1 <= max_q * G <= MAX_ROWS_PER_KV_HEAD and sliding_window[1] < 0:
            self.pth_dec = load_pth_dec()

    # -------------------------------------------------------------------------------------
    def forward_pth_dec(self, query, key_cache, value_cache, k_scale_cache, v_scale_cache, block_table, seq_lens,
                        query_start_loc, output, max_q: int, meta: AttnMeta, seq_lens_host=None) -> bool:
        """Sequences with <= max_q query tokens through the decode operator. Launch only (no host
        sync, no allocation): safe in graphs. False: the caller runs its own path."""
        if self.layout_ok is None:
            self.layout_ok = bool(self.pth_dec.supported_layout(key_cache, value_cache, k_scale_cache,
                                                                v_scale_cache))
            if not self.layout_ok:
                logger.warning("gfx950: unexpected int8 KV cache layout; decode stays on Triton")
        segm_o = meta.softmax_segm_output
        if (not self.layout_ok or segm_o is None or meta.softmax_segm_max is None or meta.softmax_segm_expsum is None
                or query.shape[0] > segm_o.shape[0] or query.dim() != 3 or output.dim() != 3
                or query.stride(1) != query.shape[2] or query.stride(2) != 1 or output.stride(2) != 1):
            return False
        # Under graph capture the host lengths describe the capture's dummy batch, not the batches
        # the graph will replay: size the split without them (the cap, or one round of workgroups
        # for windowed rows).
        if seq_lens_host is not None and _capturing(query.device):
            seq_lens_host = None
        self.pth_dec.decode(query, key_cache, value_cache, k_scale_cache, v_scale_cache, block_table, seq_lens,
                            query_start_loc, output, self.scale, segm_o, meta.softmax_segm_max,
                            meta.softmax_segm_expsum, seq_lens.shape[0], max(1, max_q),
                            decode_splits(segm_o.shape[2], self.window, self.num_kv_heads, seq_lens.shape[0],
                                          query.device, seq_lens_host, max(1, max_q), query.shape[1]),
                            window=self.window, causal=True)
        return True

    # -------------------------------------------------------------------------------------
    def forward_pth_fa(self, query, key_cache, value_cache, k_scale_cache, v_scale_cache, meta: AttnMeta, output,
                       triton_fallback: Callable[..., None]) -> bool:
        """The suffix of sequences with >= PTH_FA_MIN_Q query tokens through the prefill
        operator; the rows before it through the decode operator or `triton_fallback(start, end,
        seq_begin, seq_end, max_q)`. False when there is no such suffix."""
        qsl = [int(x) for x in (meta.query_start_loc_cpu.tolist() if hasattr(meta.query_start_loc_cpu, "tolist")
                                else meta.query_start_loc_cpu)]
        n = len(qsl) - 1
        p = n
        while p > 0 and qsl[p] - qsl[p - 1] >= PTH_FA_MIN_Q:
            p -= 1
        if p == n:
            return False
        max_q_prefix = max((qsl[i + 1] - qsl[i] for i in range(p)), default=0)
        if p > 0 and not (
            self.pth_dec is not None and max_q_prefix <= self.max_q
            and self.forward_pth_dec(query[:qsl[p]], key_cache, value_cache, k_scale_cache, v_scale_cache,
                                     meta.block_table[:p], meta.seq_lens[:p], meta.query_start_loc[:p + 1],
                                     output[:qsl[p]], max_q_prefix, meta,
                                     None if meta.seq_lens_cpu is None else meta.seq_lens_cpu[:p])):
            triton_fallback(0, qsl[p], 0, p, max_q_prefix)
        # The split count of each prefill is planned for the keys its sequence sees: the host length
        # when it is known and no graph is being captured (vLLM's block table is as wide as the
        # model's maximum length, so the table alone would plan every chunk for the longest context),
        # else the batch's max_seq_len, else the table width.
        lens_host = meta.seq_lens_cpu if meta.seq_lens_cpu is not None and not _capturing(query.device) else None
        for i in range(p, n):
            start, nq = qsl[i], qsl[i + 1] - qsl[i]
            q = query[start:start + nq].transpose(0, 1).unsqueeze(0).float().contiguous()  # [1, Hq, nq, D]
            seq_len = meta.seq_lens[i:i + 1]
            if lens_host is not None:
                max_keys = int(lens_host[i])
            elif meta.max_seq_len > 0 and not _capturing(query.device):
                max_keys = int(meta.max_seq_len)
            else:
                max_keys = None
            out = self.pth_fa.forward_pth(q, key_cache, value_cache, meta.block_table[i:i + 1], seq_len, self.scale,
                                          seq_len - nq, max_keys=max_keys,
                                          **({"exact": True} if PTH_FA_EXACT else {}))
            output[start:start + nq] = out[0].to(output.dtype)
        return True

    # -------------------------------------------------------------------------------------
    def route(self, query, key_cache, value_cache, k_scale_cache, v_scale_cache, meta: AttnMeta, output,
              max_seqlen_q: int, num_actual_tokens: int, triton_fallback: Callable[..., None],
              output_scale=None) -> bool:
        """The forward() glue: True when one of the operators handled the batch."""
        plain = (meta.causal is True and meta.mm_prefix_range_tensor is None and meta.rswa_prefix_lens is None
                 and output_scale is None)
        if (self.pth_fa is not None and max_seqlen_q >= PTH_FA_MIN_Q and plain
                and self.forward_pth_fa(query, key_cache, value_cache, k_scale_cache, v_scale_cache, meta, output,
                                        triton_fallback)):
            return True
        if (self.pth_dec is not None and max_seqlen_q <= self.max_q and plain
                and self.forward_pth_dec(query[:num_actual_tokens], key_cache, value_cache, k_scale_cache,
                                         v_scale_cache, meta.block_table, meta.seq_lens, meta.query_start_loc,
                                         output[:num_actual_tokens], max_seqlen_q, meta, meta.seq_lens_cpu)):
            return True
        return False
