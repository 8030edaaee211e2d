"""Seeded synthetic decode and prefill workloads over vLLM's int8 per-token-head paged cache,
and the algorithmic byte / FLOP counts of a workload: test and benchmark support, not part of
the operator package.

The cache primitives (views, allocation, quantiser) come from mi50_vllm_lab_amd.kvcache and are
re-exported here, so `import workload as kvc` gives tests one namespace. Everything random is
drawn from a CPU torch.Generator, so a workload is bit-identical on any machine and device;
tensors are moved to the target device afterwards.
"""
from __future__ import annotations

import importlib.util
import math
import os
import sys
from dataclasses import dataclass, field

import torch

_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _package_kvcache():
    """mi50_vllm_lab_amd.kvcache, importing the package directory (its name is not an identifier)."""
    if "mi50_vllm_lab_amd" not in sys.modules:
        pkg_dir = os.path.join(_ROOT, "mi50-vllm-lab_amd")
        spec = importlib.util.spec_from_file_location("mi50_vllm_lab_amd", os.path.join(pkg_dir, "__init__.py"),
                                                      submodule_search_locations=[pkg_dir])
        mod = importlib.util.module_from_spec(spec)
        sys.modules["mi50_vllm_lab_amd"] = mod
        spec.loader.exec_module(mod)
    return sys.modules["mi50_vllm_lab_amd"].kvcache


_kv = _package_kvcache()
HEAD_DIM, HALF_ROW, ROW_BYTES, NAN_WORD = _kv.HEAD_DIM, _kv.HALF_ROW, _kv.ROW_BYTES, _kv.NAN_WORD
PagedKVCache = _kv.PagedKVCache
cache_views, allocate_cache, clone_cache = _kv.cache_views, _kv.allocate_cache, _kv.clone_cache
quantize_per_token_head = _kv.quantize_per_token_head


def write_tokens(cache: PagedKVCache, block_table_row: torch.Tensor, positions: torch.Tensor,
                 k_q: torch.Tensor, k_s: torch.Tensor, v_q: torch.Tensor, v_s: torch.Tensor) -> None:
    """Scatter quantised rows for logical token positions into their pages.
    k_q / v_q int8 [n, Hkv, 256]; k_s / v_s f32 [n, Hkv]."""
    bs = cache.block_size
    pos = positions.long()
    blk = block_table_row.long()[pos // bs]
    slot = pos % bs
    cache.key_cache[blk, slot, :, :HEAD_DIM] = k_q
    cache.value_cache[blk, slot, :, :HEAD_DIM] = v_q
    cache.k_scale[blk, slot] = k_s.float()
    cache.v_scale[blk, slot] = v_s.float()


def poison_block(cache: PagedKVCache, block: int) -> None:
    """Fill every row of a physical block with the f32 NaN pattern (scales become NaN)."""
    words = cache.kv[block].view(torch.int32) if cache.layout == "HND" else None
    if words is not None:
        words.fill_(NAN_WORD)
    else:  # NHD: rows of this block are strided; write through the byte view
        pattern = torch.tensor([NAN_WORD], dtype=torch.int32).view(torch.int8)
        cache.kv[block].copy_(pattern.repeat(ROW_BYTES // 4).expand_as(cache.kv[block]))


@dataclass
class DecodeCase:
    """One decode batch: queries, cache, and the vLLM metadata the operator reads."""
    q: torch.Tensor                 # fp16 [T, Hq, 256]
    cache: PagedKVCache
    block_table: torch.Tensor       # int32 [B, max_blocks]
    seq_lens: torch.Tensor          # int32 [B]
    query_start_loc: torch.Tensor   # int32 [B + 1]
    ctxs: list
    qlens: list
    num_q_heads: int
    scale: float
    window: int = -1
    causal: bool = True
    poisoned_pages: int = 0
    meta: dict = field(default_factory=dict)

    @property
    def seqs(self) -> list:
        return [c + q for c, q in zip(self.ctxs, self.qlens)]

    @property
    def num_tokens(self) -> int:
        return self.q.shape[0]

    @property
    def num_seqs(self) -> int:
        return len(self.ctxs)

    @property
    def qmax(self) -> int:
        return max(1, max(self.qlens))

    def visible_range(self, b: int) -> tuple[int, int]:
        """[lo, seq_len): the keys any query row of sequence b can see."""
        seq, ql = self.seqs[b], self.qlens[b]
        lo = max(0, seq - ql - self.window + 1) if self.window > 0 else 0
        return lo, seq

    def to(self, device) -> "DecodeCase":
        cache = clone_cache(self.cache, device)
        q = self.q.to(device)
        if self.q.stride(1) != self.q.shape[2] or not self.q.is_contiguous():
            # keep a non-contiguous token stride: rebuild the padded parent on the device
            parent = torch.zeros((self.q.shape[0], self.q.stride(0) // self.q.shape[2], self.q.shape[2]),
                                 dtype=self.q.dtype, device=device)
            off = self.q.storage_offset() // self.q.shape[2] - 0
            parent[:, off:off + self.q.shape[1]] = q
            q = parent[:, off:off + self.q.shape[1]]
        return DecodeCase(q, cache, self.block_table.to(device), self.seq_lens.to(device),
                          self.query_start_loc.to(device), list(self.ctxs), list(self.qlens), self.num_q_heads,
                          self.scale, self.window, self.causal, self.poisoned_pages, dict(self.meta))


def make_case(ctxs, qlens, *, num_q_heads: int = 24, num_kv_heads: int = 4, block_size: int = 16,
              layout: str = "HND", seed: int = 0, layout_seed: int | None = None, kv_mode: str = "normal",
              scale_hi: float = 0.02, outlier_frac: float = 0.0, outlier_mult: float = 50.0,
              q_noncontig: bool = False, window: int = -1, causal: bool = True, poison: bool = False,
              spare_blocks: int = 3, softmax_scale: float | None = None) -> DecodeCase:
    """Seeded synthetic decode batch on the CPU (move it with .to(device)).

    ctxs[b] cached tokens + qlens[b] new tokens (already in the cache) per sequence; qlens may
    contain 0 (padded graph slot). kv_mode "normal": K, V ~ N(0, 1), then quantised per (token,
    kv head) with absmax/127 (a fraction outlier_frac of the rows is scaled by outlier_mult first);
    kv_mode "uniform": int8 values uniform in [-128, 127] and scales uniform in [0.002,
    0.002 + scale_hi] (kernels/pth_dec/test_dec.py:41-49). The block table maps each sequence to
    a random permutation of physical pages, with spare pages and padded columns. With poison=True
    (needs window > 0) every page wholly outside all rows' windows points at a NaN-filled page.
    """
    assert len(ctxs) == len(qlens)
    g = torch.Generator().manual_seed(seed)
    gl = torch.Generator().manual_seed(seed + 7919 if layout_seed is None else layout_seed)
    seqs = [c + q for c, q in zip(ctxs, qlens)]
    bs = block_size
    per = [max(1, (s + bs - 1) // bs) for s in seqs]
    nblk = sum(per) + spare_blocks + (1 if poison else 0)
    cache = allocate_cache(nblk, bs, num_kv_heads, layout)
    # arbitrary bytes everywhere first: pad bytes and unused slots hold noise
    cache.kv.copy_(torch.randint(-128, 128, cache.kv.shape, dtype=torch.int8, generator=gl))
    perm = torch.randperm(nblk, generator=gl).to(torch.int32)
    poison_blk = int(perm[-1]) if poison else -1
    maxb = max(per) + 2
    bt = torch.zeros((len(seqs), maxb), dtype=torch.int32)
    o = 0
    for b, n in enumerate(per):
        bt[b, :n] = perm[o:o + n]
        o += n
    for b, seq in enumerate(seqs):
        if seq <= 0:
            continue
        if kv_mode == "normal":
            k = torch.randn((seq, num_kv_heads, HEAD_DIM), generator=g)
            v = torch.randn((seq, num_kv_heads, HEAD_DIM), generator=g)
            if outlier_frac > 0:
                for x in (k, v):
                    sel = torch.rand((seq, num_kv_heads), generator=g) < outlier_frac
                    x[sel] *= outlier_mult
            kq, ks = quantize_per_token_head(k)
            vq, vs = quantize_per_token_head(v)
        elif kv_mode == "uniform":
            kq = torch.randint(-128, 128, (seq, num_kv_heads, HEAD_DIM), dtype=torch.int8, generator=g)
            vq = torch.randint(-128, 128, (seq, num_kv_heads, HEAD_DIM), dtype=torch.int8, generator=g)
            ks = torch.rand((seq, num_kv_heads), generator=g) * scale_hi + 0.002
            vs = torch.rand((seq, num_kv_heads), generator=g) * scale_hi + 0.002
        else:
            raise ValueError(kv_mode)
        write_tokens(cache, bt[b], torch.arange(seq), kq, ks, vq, vs)
    poisoned = 0
    if poison:
        assert window > 0, "poisoning needs a window"
        poison_block(cache, poison_blk)
        for b, (seq, ql) in enumerate(zip(seqs, qlens)):
            lo = max(0, seq - ql - window + 1)
            for lb in range(lo // bs):  # pages whose last key is before every row's window
                bt[b, lb] = poison_blk
                poisoned += 1
    T = sum(qlens)
    if q_noncontig:
        big = torch.randn((T, num_q_heads + 4, HEAD_DIM), generator=g).to(torch.float16)
        q = big[:, 2:2 + num_q_heads]
    else:
        q = torch.randn((T, num_q_heads, HEAD_DIM), generator=g).to(torch.float16)
    qsl = torch.tensor([0] + list(torch.tensor(qlens, dtype=torch.int64).cumsum(0).tolist()), dtype=torch.int32)
    sl = torch.tensor(seqs, dtype=torch.int32)
    sc = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(HEAD_DIM)
    return DecodeCase(q, cache, bt, sl, qsl, list(ctxs), list(qlens), num_q_heads, sc, window, causal, poisoned,
                      {"seed": seed, "kv_mode": kv_mode, "layout": layout, "block_size": bs})


def partial_buffers(max_tokens: int, num_q_heads: int, nseg: int, device) -> tuple:
    """vLLM's softmax segment buffers: part_o [T, Hq, NSEG, 256], part_m / part_l [T, Hq, NSEG]."""
    part_o = torch.empty((max_tokens, num_q_heads, nseg, HEAD_DIM), dtype=torch.float32, device=device)
    part_m = torch.empty((max_tokens, num_q_heads, nseg), dtype=torch.float32, device=device)
    part_l = torch.empty((max_tokens, num_q_heads, nseg), dtype=torch.float32, device=device)
    return part_o, part_m, part_l


def visible_kv_bytes(case: DecodeCase) -> int:
    """Bytes of KV rows any query row can see: the algorithmic KV traffic of one decode call."""
    hkv = case.cache.num_kv_heads
    return sum((hi - lo) for lo, hi in (case.visible_range(b) for b in range(case.num_seqs))) * hkv * ROW_BYTES


def algorithmic_bytes(case: DecodeCase) -> int:
    """KV rows + Q + out (fp16) + block-table entries of touched pages + seq_lens / query_start_loc."""
    kv = visible_kv_bytes(case)
    qo = 2 * case.num_tokens * case.num_q_heads * HEAD_DIM * 2
    bs = case.cache.block_size
    pages = 0
    for b in range(case.num_seqs):
        lo, hi = case.visible_range(b)
        if hi > lo:
            pages += (hi - 1) // bs - lo // bs + 1
    meta = 4 * case.num_seqs + 4 * (case.num_seqs + 1)
    return kv + qo + 4 * pages + meta


def algorithmic_flops(case: DecodeCase) -> int:
    """4 * D * sum over query rows of visible keys (QK and PV)."""
    G = case.num_q_heads // case.cache.num_kv_heads
    total = 0
    for b, (seq, ql) in enumerate(zip(case.seqs, case.qlens)):
        for j in range(ql):
            p = seq - ql + j
            hi = p + 1 if case.causal else seq
            lo = max(0, p - case.window + 1) if case.window > 0 else 0
            total += max(0, hi - lo)
    return 4 * HEAD_DIM * G * total * case.cache.num_kv_heads


def prefill_query(case: DecodeCase) -> torch.Tensor:
    """The case's query tokens as the prefill operator takes them: fp32 [B, Hq, Sq, 256] contiguous.

    Every sequence of the case must have the same number of new tokens Sq (kernels/fa_pth/pth_fa.cpp:35).
    """
    sq = case.qlens[0] if case.qlens else 0
    assert all(q == sq for q in case.qlens), "prefill needs the same chunk length for every sequence"
    B, hq = case.num_seqs, case.num_q_heads
    return case.q.reshape(B, sq, hq, HEAD_DIM).permute(0, 2, 1, 3).float().contiguous()


def prefill_flops(seq_lens, q_abs, sq: int, num_q_heads: int) -> int:
    """4 * D * Hq * sum over query rows of visible keys: the reference's FLOP count for a chunk
    (kernels/fa_pth/test_pth.py:128 for q_abs = seq_len - Sq)."""
    total = 0
    for seq, qa in zip(seq_lens, q_abs):
        for i in range(sq):
            total += max(0, min(int(seq), int(qa) + i + 1))
    return 4 * HEAD_DIM * num_q_heads * total


def fp16_half_ulp(x):
    """Half the spacing of fp16 numbers at |x| (numpy, elementwise): the rounding error of a
    correctly rounded fp16 result (2^-25 below the normal range)."""
    import numpy as np
    a = np.maximum(np.abs(np.asarray(x, dtype=np.float64)), 2.0 ** -14)
    return 0.5 * np.exp2(np.floor(np.log2(a)) - 10)


def fp16_output_errors(out, ref, tol_max=2e-3, tol_mean=2e-4):
    """Errors of an fp16 output against the float64 oracle, with the tolerance applied to the
    value computed before the final rounding to fp16.

    An fp16 result of magnitude >= 8 cannot be within 2e-3 of the exact answer: its spacing there
    is 2^-7. So element by element |out - ref| may exceed tol_max by half an fp16 spacing at that
    magnitude, taking the larger of |out| and |ref|, which covers a rounding across a power of two.
    The mean-abs error may exceed that of the correctly rounded answer fp16(ref) by tol_mean.
    Below |ref| = 1 the allowance is at most 2^-12 (2.4e-4).

    Returns (max-abs, mean-abs, worst excess over the element bound, mean-abs excess over fp16(ref)).
    The output passes when both excesses are <= 0 and tol_mean respectively.
    """
    import numpy as np
    o = np.asarray(out, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    if o.size == 0:
        return 0.0, 0.0, -tol_max, 0.0
    e = np.abs(o - r)
    bound = tol_max + fp16_half_ulp(np.maximum(np.abs(o), np.abs(r)))
    r16 = r.astype(np.float16).astype(np.float64)
    return float(e.max()), float(e.mean()), float((e - bound).max()), float(e.mean() - np.abs(r16 - r).mean())
