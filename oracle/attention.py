"""CPU oracle for int8 per-token-head paged decode attention. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use this module, and
only as the checker or the CPU baseline; the operator never calls it and has no CPU fallback.

`paged_decode` restates, in float64 numpy, the reference's dequantise-then-attend path
(kernels/pth_dec/test_dec.py:70-88): for every sequence gather its pages through the block
table, dequantise int8 x per-(token, kv head) scale, then softmax(q k^T * scale + mask) v per
query head. The mask rule for query row j of a sequence (absolute position
p_j = seq_len - q_len + j) and key k:
    k < seq_len
    and (not causal or k <= p_j)                      kernels/pth_dec/pth_dec.cu:186
    and (window <= 0 or p_j - k < window)             kernels/fa_pth/kernel/fattn-q8-paged.cuh:219-229,
                                                      patches/vllm/gfx906_fa_paged.patch:7-20
For non-causal rows with a window this is the "left window only" rule the reference's test
checks row by row (upstream/pr-dflash2/0002-...patch:109-118): row j sees keys
[seq_len - q_len + j - window + 1, seq_len).

Only pages that hold a key some row can see are read: pages wholly outside every row's window
(freed pages, possibly NaN-poisoned) are never touched, as in the reference's window clip.

`paged_decode_loops` is an independent, loop-form restatement (per row, per key, per dim, no
vectorisation) for tiny inputs; the tests use it to pin `paged_decode`.

`paged_prefill` restates the reference's prefill check (kernels/fa_pth/test_pth.py:71-82, the
`exact` float64 path) for the forward_pth interface (kernels/fa_pth/pth_fa.cpp:35-41): q is
[B, Hq, Sq, 256], query row i of sequence b sits at absolute position q_abs_offset[b] + i and
sees keys k < seq_lens[b] with k <= that position; the output is [B, Sq, Hq, 256].
`paged_prefill_loops` is its loop-form twin for tiny inputs.

Parity status: pinned by the checks in tests/test_oracle.py (brute force, closed forms,
torch scaled_dot_product_attention in float64, permutation invariance, the reference's
windowed-row formula). vLLM's Triton kernel, which the reference also prints, cannot run here:
parity with it is unpinned and not claimed.
"""
from __future__ import annotations

import math

import numpy as np

HEAD_DIM = 256


def _np(x):
    """numpy view of a torch CPU tensor (any strides) or an array."""
    if hasattr(x, "detach"):
        return x.detach().cpu().numpy()
    return np.asarray(x)


def visible_mask(seq_len: int, q_len: int, lo: int, causal: bool, window: int) -> np.ndarray:
    """bool [q_len, seq_len - lo]: row j sees key lo + i."""
    pos = seq_len - q_len + np.arange(q_len)[:, None]
    k = lo + np.arange(seq_len - lo)[None, :]
    m = k < seq_len
    if causal:
        m = m & (k <= pos)
    if window > 0:
        m = m & (pos - k < window)
    return m


def gather_dequant(key_cache, value_cache, k_scale, v_scale, bt_row, lo: int, hi: int):
    """float64 K, V [hi - lo, Hkv, 256] of logical tokens [lo, hi) (test_dec.py:76-80)."""
    kc, vc, ks, vs = _np(key_cache), _np(value_cache), _np(k_scale), _np(v_scale)
    bt = _np(bt_row).astype(np.int64)
    bs = kc.shape[1]
    t = np.arange(lo, hi)
    blk, slot = bt[t // bs], t % bs
    k = kc[blk, slot, :, :HEAD_DIM].astype(np.float64) * ks[blk, slot][..., None].astype(np.float64)
    v = vc[blk, slot, :, :HEAD_DIM].astype(np.float64) * vs[blk, slot][..., None].astype(np.float64)
    return k, v


def paged_decode(q, key_cache, value_cache, k_scale, v_scale, block_table, seq_lens, query_start_loc,
                 num_seqs: int, scale: float, window: int = -1, causal: bool = True, qmax: int | None = None):
    """float64 [T, Hq, 256] outputs and a bool [T] mask of the rows the operator writes.

    Rows of tokens that belong to no sequence, of sequences with seq_len <= 0, or past qmax
    query tokens of their sequence are left at 0 and marked unwritten.
    """
    qn = _np(q).astype(np.float64)
    T, Hq, D = qn.shape
    Hkv = _np(key_cache).shape[2]
    G = Hq // Hkv
    sl, qsl, bt = _np(seq_lens), _np(query_start_loc), _np(block_table)
    out = np.zeros((T, Hq, D), dtype=np.float64)
    written = np.zeros(T, dtype=bool)
    for b in range(num_seqs):
        q0, q1, seq = int(qsl[b]), int(qsl[b + 1]), int(sl[b])
        ql = q1 - q0
        if ql <= 0 or seq <= 0:
            continue
        nrows = ql if qmax is None else min(ql, qmax)
        lo = max(0, seq - ql - window + 1) if window > 0 else 0
        k, v = gather_dequant(key_cache, value_cache, k_scale, v_scale, bt[b], lo, seq)
        mask = visible_mask(seq, ql, lo, causal, window)[:nrows]
        for g in range(Hkv):
            qg = qn[q0:q0 + nrows, g * G:(g + 1) * G].reshape(nrows * G, D)          # [rows*G, D]
            s = (qg @ np.ascontiguousarray(k[:, g]).T).reshape(nrows, G, -1) * scale  # [rows, G, keys]
            s = np.where(mask[:, None, :], s, -np.inf)
            s = s - s.max(axis=-1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=-1, keepdims=True)
            o = p.reshape(nrows * G, -1) @ np.ascontiguousarray(v[:, g])
            out[q0:q0 + nrows, g * G:(g + 1) * G] = o.reshape(nrows, G, D)
        written[q0:q0 + nrows] = True
    return out, written


def paged_prefill(q, key_cache, value_cache, k_scale, v_scale, block_table, seq_lens, scale: float,
                  q_abs_offset, rows=None):
    """float64 [B, Sq, Hq, 256] outputs and a bool [B, Sq] mask of rows with a visible key.

    rows: optional iterable of query rows to compute (the others stay 0 and unmarked), so that a
    full-size chunk can be checked on a sample of rows. Rows that see no key (seq_len <= 0 or a
    position below 0) stay 0 and unmarked.
    """
    qn = _np(q)
    B, Hq, Sq, D = qn.shape
    Hkv = _np(key_cache).shape[2]
    G = Hq // Hkv
    sl, qa, bt = _np(seq_lens), _np(q_abs_offset), _np(block_table)
    sel = np.arange(Sq) if rows is None else np.asarray(sorted(set(int(r) for r in rows)), dtype=np.int64)
    out = np.zeros((B, Sq, Hq, D), dtype=np.float64)
    written = np.zeros((B, Sq), dtype=bool)
    for b in range(B):
        seq = int(sl[b])
        pos = int(qa[b]) + sel
        hi = min(seq, int(pos.max()) + 1) if sel.size else 0
        if hi <= 0:
            continue
        k, v = gather_dequant(key_cache, value_cache, k_scale, v_scale, bt[b], 0, hi)
        mask = np.arange(hi)[None, :] <= pos[:, None]            # [rows, keys]; keys < hi <= seq_len
        live = mask.any(axis=1)
        for h in range(Hq):
            g = h // G
            for r0 in range(0, sel.size, 256):                    # bounded score blocks
                rs = slice(r0, min(r0 + 256, sel.size))
                s = (qn[b, h, sel[rs]].astype(np.float64) @ np.ascontiguousarray(k[:, g]).T) * scale
                s = np.where(mask[rs], s, -np.inf)
                mx = s.max(axis=1, keepdims=True)
                mx = np.where(np.isfinite(mx), mx, 0.0)
                p = np.exp(s - mx)
                tot = p.sum(axis=1, keepdims=True)
                o = (p @ np.ascontiguousarray(v[:, g])) / np.where(tot > 0, tot, 1.0)
                out[b, sel[rs], h] = np.where(live[rs, None], o, 0.0)
        written[b, sel[live]] = True
    return out, written


def paged_prefill_loops(q, key_cache, value_cache, k_scale, v_scale, block_table, seq_lens, scale: float,
                        q_abs_offset):
    """Loop-form restatement of paged_prefill for tiny inputs: one key and one dim at a time."""
    qn = _np(q)
    kc, vc, ks, vs = _np(key_cache), _np(value_cache), _np(k_scale), _np(v_scale)
    bt, sl, qa = _np(block_table), _np(seq_lens), _np(q_abs_offset)
    B, Hq, Sq, D = qn.shape
    Hkv, bs = kc.shape[2], kc.shape[1]
    out = [[[[0.0] * D for _ in range(Hq)] for _ in range(Sq)] for _ in range(B)]
    for b in range(B):
        for i in range(Sq):
            p_i = int(qa[b]) + i
            for h in range(Hq):
                g = h // (Hq // Hkv)
                scores, vals = [], []
                for key in range(int(sl[b])):
                    if key > p_i:
                        break
                    blk, slot = int(bt[b][key // bs]), key % bs
                    dot = 0.0
                    for d in range(D):
                        dot += float(qn[b][h][i][d]) * (float(kc[blk][slot][g][d]) * float(ks[blk][slot][g]))
                    scores.append(dot * scale)
                    vals.append([float(vc[blk][slot][g][d]) * float(vs[blk][slot][g]) for d in range(D)])
                if not scores:
                    continue
                mx = max(scores)
                w = [math.exp(x - mx) for x in scores]
                tot = sum(w)
                for d in range(D):
                    out[b][i][h][d] = sum(wi * vi[d] for wi, vi in zip(w, vals)) / tot
    return np.array(out, dtype=np.float64)


def paged_decode_loops(q, key_cache, value_cache, k_scale, v_scale, block_table, seq_lens, query_start_loc,
                       num_seqs: int, scale: float, window: int = -1, causal: bool = True):
    """Loop-form restatement for tiny inputs: plain Python floats, one key at a time."""
    qn = _np(q)
    kc, vc, ks, vs = _np(key_cache), _np(value_cache), _np(k_scale), _np(v_scale)
    bt, sl, qsl = _np(block_table), _np(seq_lens), _np(query_start_loc)
    T, Hq, D = qn.shape
    Hkv = kc.shape[2]
    bs = kc.shape[1]
    out = [[[0.0] * D for _ in range(Hq)] for _ in range(T)]
    for b in range(num_seqs):
        q0, q1, seq = int(qsl[b]), int(qsl[b + 1]), int(sl[b])
        for j in range(q1 - q0):
            p_j = seq - (q1 - q0) + j
            for h in range(Hq):
                g = h // (Hq // Hkv)
                scores, vals = [], []
                for key in range(seq):
                    if causal and key > p_j:
                        continue
                    if window > 0 and p_j - key >= window:
                        continue
                    blk, slot = int(bt[b][key // bs]), key % bs
                    kscale = float(ks[blk][slot][g])
                    dot = 0.0
                    for d in range(D):
                        dot += float(qn[q0 + j][h][d]) * (float(kc[blk][slot][g][d]) * kscale)
                    scores.append(dot * scale)
                    vscale = float(vs[blk][slot][g])
                    vals.append([float(vc[blk][slot][g][d]) * vscale for d in range(D)])
                mx = max(scores)
                w = [math.exp(x - mx) for x in scores]
                tot = sum(w)
                for d in range(D):
                    out[q0 + j][h][d] = sum(wi * vi[d] for wi, vi in zip(w, vals)) / tot
    return np.array(out, dtype=np.float64)
