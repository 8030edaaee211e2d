"""Pins the prefill oracle (oracle/attention.py: paged_prefill) on the CPU.

kernels/fa_pth/test_pth.py:71-82 checks forward_pth against a float64 dequantise-then-attend
path; it ships no vectors (CUDA-generator seeds). The restatement is pinned by its loop-form
twin on tiny inputs (arbitrary q_abs_offset, rows that see every key, rows that see none), by the
decode oracle on the rows both define (q_abs_offset = seq_len - Sq), by torch's float64
scaled_dot_product_attention with an explicit mask, by the closed form of a row that sees one
key, and by row sampling returning the full computation's rows.
"""
import numpy as np
import pytest
import torch

import workload as kvc
from oracle import attention as orc


def prefill(c, q_abs, rows=None):
    return orc.paged_prefill(kvc.prefill_query(c), c.cache.key_cache, c.cache.value_cache, c.cache.k_scale,
                             c.cache.v_scale, c.block_table, c.seq_lens, c.scale, torch.tensor(q_abs), rows)


TINY = [
    # ctxs, Sq, Hq, Hkv, bs, layout, kv_mode, q_abs (None: seq_len - Sq)
    ([5], 3, 2, 1, 4, "HND", "uniform", None),
    ([9, 2], 4, 4, 2, 3, "NHD", "normal", None),
    ([12], 4, 6, 2, 16, "HND", "uniform", [3]),          # rows in the middle of the sequence
    ([6], 3, 2, 2, 4, "HND", "normal", [20]),            # every row past the end: sees every key
    ([4, 7], 3, 4, 1, 5, "NHD", "uniform", [-2, 1]),     # first rows of sequence 0 see no key
    ([0, 3], 2, 2, 1, 16, "HND", "normal", None),
]


@pytest.mark.parametrize("ctxs,sq,hq,hkv,bs,layout,mode,q_abs", TINY)
def test_vectorised_matches_loops(ctxs, sq, hq, hkv, bs, layout, mode, q_abs):
    c = kvc.make_case(ctxs, [sq] * len(ctxs), num_q_heads=hq, num_kv_heads=hkv, block_size=bs, layout=layout,
                      seed=sum(ctxs) + 17 * sq, kv_mode=mode)
    qa = q_abs if q_abs is not None else list(ctxs)
    out, written = prefill(c, qa)
    ref = orc.paged_prefill_loops(kvc.prefill_query(c), c.cache.key_cache, c.cache.value_cache, c.cache.k_scale,
                                  c.cache.v_scale, c.block_table, c.seq_lens, c.scale, torch.tensor(qa))
    np.testing.assert_allclose(out, ref, rtol=1e-11, atol=1e-13)
    for b, (ctx, a) in enumerate(zip(ctxs, qa)):
        seq = ctx + sq
        for i in range(sq):
            assert written[b, i] == (seq > 0 and a + i >= 0)
    assert not out[~written].any()


@pytest.mark.parametrize("ctxs,sq,bs", [([40, 17], 6, 16), ([100], 33, 8), ([0], 9, 4)])
def test_matches_decode_oracle_when_chunk_ends_the_sequence(ctxs, sq, bs):
    c = kvc.make_case(ctxs, [sq] * len(ctxs), num_q_heads=6, num_kv_heads=2, block_size=bs, seed=5 + sq)
    out, written = prefill(c, list(ctxs))
    dec, dw = orc.paged_decode(c.q, c.cache.key_cache, c.cache.value_cache, c.cache.k_scale, c.cache.v_scale,
                               c.block_table, c.seq_lens, c.query_start_loc, c.num_seqs, c.scale)
    assert written.all() and dw.all()
    np.testing.assert_allclose(out.reshape(-1, 6, 256), dec, rtol=1e-12, atol=1e-13)


def test_matches_torch_sdpa_in_float64():
    ctx, sq, qa = 50, 7, 30
    c = kvc.make_case([ctx], [sq], num_q_heads=4, num_kv_heads=2, block_size=16, seed=11)
    out, written = prefill(c, [qa])
    seq = ctx + sq
    k, v = orc.gather_dequant(c.cache.key_cache, c.cache.value_cache, c.cache.k_scale, c.cache.v_scale,
                              c.block_table[0], 0, seq)
    q = kvc.prefill_query(c)[0].double()                                    # [Hq, Sq, D]
    kk = torch.from_numpy(k).permute(1, 0, 2).repeat_interleave(2, dim=0)   # [Hq, seq, D]
    vv = torch.from_numpy(v).permute(1, 0, 2).repeat_interleave(2, dim=0)
    pos = qa + torch.arange(sq)
    mask = torch.arange(seq)[None, :] <= pos[:, None]
    ref = torch.nn.functional.scaled_dot_product_attention(q, kk, vv, attn_mask=mask, scale=c.scale)
    assert written.all()
    np.testing.assert_allclose(out[0], ref.permute(1, 0, 2).numpy(), rtol=1e-10, atol=1e-12)


def test_first_row_of_a_fresh_sequence_returns_its_value_row():
    c = kvc.make_case([0], [4], num_q_heads=3, num_kv_heads=1, block_size=16, seed=2, kv_mode="uniform")
    out, _ = prefill(c, [0])
    blk = int(c.block_table[0, 0])
    v = c.cache.value_cache[blk, 0, 0, :256].double() * float(c.cache.v_scale[blk, 0, 0])
    for h in range(3):
        np.testing.assert_allclose(out[0, 0, h], v.numpy(), rtol=1e-12)


def test_row_sample_equals_full_rows():
    c = kvc.make_case([300], [40], num_q_heads=6, num_kv_heads=2, block_size=16, seed=9)
    full, fw = prefill(c, [300])
    rows = [0, 7, 39, 21]
    part, pw = prefill(c, [300], rows)
    assert pw[0, rows].all() and pw.sum() == len(rows)
    np.testing.assert_array_equal(part[0, rows], full[0, rows])


def test_prefill_flops_matches_reference_count():
    # kernels/fa_pth/test_pth.py:128: 4 * D * NQ * (2048 * ctx + 2048 * 2049 / 2)
    for ctx in (0, 16384, 61440):
        assert kvc.prefill_flops([ctx + 2048], [ctx], 2048, 24) == 4 * 256 * 24 * (2048 * ctx + 2048 * 2049 // 2)
