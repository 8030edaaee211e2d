#!/usr/bin/env python3
"""Writes tests/golden/decode_cases.npz: small frozen decode problems with expected outputs.

The reference ships no golden vectors for this path (its tests draw CUDA-generator data and
compare two implementations live, kernels/pth_dec/test_dec.py:34-140). These fixtures freeze a
few small problems instead, so that the oracle, the input generator and the HIP operator are
all checked against numbers that cannot drift with them:

  inputs   the raw cache bytes in physical order, q, block_table, seq_lens, query_start_loc,
           softmax scale, window, causal flag, and the cache layout name;
  expected float64 attention computed here, row by row, straight from the definition of the
           reference's float64 path (test_dec.py:70-88: gather the sequence's pages through the
           block table, dequantise K and V with their per-token-head scales, softmax(q k^T *
           scale + mask) v), with the causal / sliding-window / non-causal rule of
           patches/vllm/gfx906_fa_paged.patch:7-20 written out as a per-key Python test.

This code shares nothing with oracle/attention.py beyond the cache views. Re-running it must
reproduce the committed file bit for bit (the generators are seeded CPU generators).
"""
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))


def _kvcache():
    """The seeded workload generator of the tests (tests/workload.py)."""
    sys.path.insert(0, os.path.dirname(HERE))
    import workload

    return workload


CASES = {
    # name: make_case keyword arguments
    "mtp_gqa6_hnd": dict(ctxs=[36, 9], qlens=[4, 1], num_q_heads=12, num_kv_heads=2, block_size=16,
                         layout="HND", seed=501, spare_blocks=1),
    "window_noncausal_poison_nhd": dict(ctxs=[70, 21], qlens=[8, 8], num_q_heads=6, num_kv_heads=1, block_size=8,
                                        layout="NHD", seed=502, window=16, causal=False, poison=True,
                                        spare_blocks=1),
    "bs1_noncontig_q_outliers": dict(ctxs=[33], qlens=[3], num_q_heads=6, num_kv_heads=1, block_size=1,
                                     layout="HND", seed=503, q_noncontig=True, outlier_frac=0.05,
                                     spare_blocks=1),
    "uniform_padded_slot": dict(ctxs=[50, 0, 17], qlens=[2, 0, 4], num_q_heads=6, num_kv_heads=1,
                                block_size=16, layout="HND", seed=504, kv_mode="uniform", spare_blocks=1),
}


def expected(case):
    """float64 [T, Hq, 256] and the mask of rows the operator writes."""
    kv = case.cache.kv.to(torch.int64)             # logical [blocks, Hkv, bs, 520], any physical order
    raw = case.cache.kv                            # keep int8 bytes for the scale words
    T, Hq = case.q.shape[0], case.q.shape[1]
    hkv = case.cache.num_kv_heads
    bs = case.cache.block_size
    G = Hq // hkv
    out = np.zeros((T, Hq, 256))
    written = np.zeros((T, Hq), dtype=bool)
    for b, (seq, ql) in enumerate(zip(case.seqs, case.qlens)):
        q0 = int(case.query_start_loc[b])
        for j in range(ql):
            p = seq - ql + j
            keys = [k for k in range(seq)
                    if (not case.causal or k <= p) and (case.window <= 0 or p - k < case.window)]
            for h in range(Hq):
                g = h // G
                q = case.q[q0 + j, h].double()
                scores, vals = [], []
                for k in keys:
                    blk = int(case.block_table[b, k // bs])
                    row = raw[blk, g, k % bs]
                    kint = row[:256].double()
                    ks = float(row[256:260].contiguous().view(torch.float32)[0])
                    vint = row[260:516].double()
                    vs = float(row[516:520].contiguous().view(torch.float32)[0])
                    scores.append(float((q * kint).sum()) * ks * case.scale)
                    vals.append(vint * vs)
                mx = max(scores)
                w = [math.exp(s - mx) for s in scores]
                tot = sum(w)
                acc = torch.zeros(256, dtype=torch.float64)
                for wi, v in zip(w, vals):
                    acc += wi * v
                out[q0 + j, h] = (acc / tot).numpy()
                written[q0 + j, h] = True
    del kv
    return out, written


def build():
    kvc = _kvcache()
    arrays = {}
    for name, kw in CASES.items():
        case = kvc.make_case(**kw)
        exp, written = expected(case)
        phys = case.cache.kv if case.cache.layout == "HND" else case.cache.kv.transpose(1, 2)
        arrays[f"{name}.kv"] = phys.contiguous().numpy()
        q = case.q
        arrays[f"{name}.q"] = q.contiguous().view(torch.int16).numpy()
        arrays[f"{name}.block_table"] = case.block_table.numpy()
        arrays[f"{name}.seq_lens"] = case.seq_lens.numpy()
        arrays[f"{name}.query_start_loc"] = case.query_start_loc.numpy()
        arrays[f"{name}.params"] = np.array([case.scale, case.window, 1.0 if case.causal else 0.0,
                                             case.num_q_heads, case.qmax])
        arrays[f"{name}.layout"] = np.frombuffer(case.cache.layout.encode(), dtype=np.uint8)
        arrays[f"{name}.expected"] = exp.astype(np.float32)  # float64 rounded once
        arrays[f"{name}.written"] = written
    path = os.path.join(HERE, "decode_cases.npz")
    np.savez_compressed(path, **arrays)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    sys.exit(build())
