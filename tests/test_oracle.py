"""Pins the CPU oracle (oracle/attention.py) on the CPU.

The reference ships no golden vectors for this path (its seeds are CUDA-generator seeds,
kernels/pth_dec/test_dec.py:36), so the oracle is pinned by checks a plausible mistake would
fail: an independent loop-form restatement on tiny inputs, closed forms (one visible key,
uniform attention), a library routine (torch scaled_dot_product_attention in float64), the
reference's own windowed-row formula (upstream/pr-dflash2/0002-...patch:109-118), invariance to
the physical page layout, and NaN-poisoned freed pages.
"""
import math

import numpy as np
import pytest
import torch

import workload as kvc
from oracle import attention as orc


def run_oracle(c, qmax=None):
    return orc.paged_decode(c.q, c.cache.key_cache, c.cache.value_cache, c.cache.k_scale, c.cache.v_scale,
                            c.block_table, c.seq_lens, c.query_start_loc, c.num_seqs, c.scale, c.window,
                            c.causal, qmax)


def run_loops(c):
    return orc.paged_decode_loops(c.q, c.cache.key_cache, c.cache.value_cache, c.cache.k_scale,
                                  c.cache.v_scale, c.block_table, c.seq_lens, c.query_start_loc, c.num_seqs,
                                  c.scale, c.window, c.causal)


TINY = [
    # ctxs, qlens, Hq, Hkv, bs, layout, causal, window, kv_mode
    ([5], [1], 2, 1, 4, "HND", True, -1, "uniform"),
    ([9], [3], 4, 2, 4, "NHD", True, -1, "normal"),
    ([7, 0, 12], [2, 0, 4], 6, 2, 3, "HND", True, -1, "uniform"),
    ([13], [4], 4, 1, 16, "HND", False, -1, "normal"),
    ([20], [3], 4, 2, 4, "NHD", False, 6, "normal"),
    ([18], [2], 2, 2, 5, "HND", True, 7, "uniform"),
    ([0], [1], 2, 1, 16, "HND", True, -1, "normal"),
]


@pytest.mark.parametrize("ctxs,qlens,hq,hkv,bs,layout,causal,window,mode", TINY)
def test_vectorised_matches_loops(ctxs, qlens, hq, hkv, bs, layout, causal, window, mode):
    c = kvc.make_case(ctxs, qlens, num_q_heads=hq, num_kv_heads=hkv, block_size=bs, layout=layout,
                      seed=len(ctxs) * 31 + sum(ctxs), kv_mode=mode, window=window, causal=causal)
    out, written = run_oracle(c)
    ref = run_loops(c)
    assert written.all()
    np.testing.assert_allclose(out, ref, rtol=1e-11, atol=1e-13)


def test_single_visible_key_returns_its_value_row():
    # ctx 0, one query token: the only visible key is the token itself, so out = v_int8 * v_scale
    c = kvc.make_case([0], [1], num_q_heads=6, num_kv_heads=1, block_size=16, seed=3, kv_mode="uniform")
    out, _ = run_oracle(c)
    blk = int(c.block_table[0, 0])
    v = c.cache.value_cache[blk, 0, 0, :256].double() * float(c.cache.v_scale[blk, 0, 0])
    for h in range(6):
        assert np.array_equal(out[0, h], v.numpy())


@pytest.mark.parametrize("causal,window", [(True, -1), (False, -1), (True, 5), (False, 9)])
def test_zero_query_attends_uniformly(causal, window):
    # q = 0: every visible key gets the same weight, so out is the mean of the visible V rows
    c = kvc.make_case([40], [4], num_q_heads=2, num_kv_heads=1, block_size=8, seed=5, kv_mode="normal",
                      causal=causal, window=window)
    c.q.zero_()
    out, _ = run_oracle(c)
    seq = 44
    _, v = orc.gather_dequant(c.cache.key_cache, c.cache.value_cache, c.cache.k_scale, c.cache.v_scale,
                              c.block_table[0], 0, seq)
    for j in range(4):
        p = seq - 4 + j
        keys = [k for k in range(seq) if (not causal or k <= p) and (window <= 0 or p - k < window)]
        mean = v[keys, 0].mean(axis=0)
        np.testing.assert_allclose(out[j, 0], mean, rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("causal,window", [(True, -1), (False, -1), (True, 33), (False, 50)])
def test_matches_torch_sdpa_in_float64(causal, window):
    # Build the cache from known logical K/V, then compare with the library attention routine.
    g = torch.Generator().manual_seed(11)
    hq, hkv, seq, ql, bs = 6, 2, 150, 4, 16
    k = torch.randn((seq, hkv, 256), generator=g)
    v = torch.randn((seq, hkv, 256), generator=g)
    kq, ks = kvc.quantize_per_token_head(k)
    vq, vs = kvc.quantize_per_token_head(v)
    nblk = (seq + bs - 1) // bs + 2
    cache = kvc.allocate_cache(nblk, bs, hkv, "NHD")
    bt = torch.randperm(nblk, generator=g)[: (seq + bs - 1) // bs].to(torch.int32)[None]
    kvc.write_tokens(cache, bt[0], torch.arange(seq), kq, ks, vq, vs)
    q = torch.randn((ql, hq, 256), generator=g).half()
    out, _ = orc.paged_decode(q, cache.key_cache, cache.value_cache, cache.k_scale, cache.v_scale, bt,
                              torch.tensor([seq], dtype=torch.int32), torch.tensor([0, ql], dtype=torch.int32),
                              1, 1 / 16, window, causal)
    kd = (kq.double() * ks.double()[..., None]).transpose(0, 1)  # [hkv, seq, 256]
    vd = (vq.double() * vs.double()[..., None]).transpose(0, 1)
    pos = seq - ql + torch.arange(ql)[:, None]
    key = torch.arange(seq)[None, :]
    mask = torch.ones((ql, seq), dtype=torch.bool)
    if causal:
        mask &= key <= pos
    if window > 0:
        mask &= pos - key < window
    G = hq // hkv
    qd = q.double().transpose(0, 1)  # [hq, ql, 256]
    ref = torch.nn.functional.scaled_dot_product_attention(
        qd, kd.repeat_interleave(G, 0), vd.repeat_interleave(G, 0), attn_mask=mask, scale=1 / 16)
    np.testing.assert_allclose(out, ref.transpose(0, 1).numpy(), rtol=1e-10, atol=1e-12)


def test_noncausal_window_matches_reference_row_formula():
    # upstream/pr-dflash2/0002-...patch:112-116: row j of an sq-row block at the end of an
    # L-token sequence sees keys [L - sq + j - window + 1, L), in both directions of p_j.
    L, sq, W = 300, 8, 64
    c = kvc.make_case([L - sq], [sq], num_q_heads=4, num_kv_heads=2, block_size=16, seed=9,
                      kv_mode="normal", causal=False, window=W)
    out, _ = run_oracle(c)
    k, v = orc.gather_dequant(c.cache.key_cache, c.cache.value_cache, c.cache.k_scale, c.cache.v_scale,
                              c.block_table[0], 0, L)
    qn = c.q.double().numpy()
    for j in range(sq):
        lo = L - sq + j - W + 1
        for h in range(4):
            s = k[lo:, h // 2] @ qn[j, h] / 16.0
            p = np.exp(s - s.max())
            p /= p.sum()
            np.testing.assert_allclose(out[j, h], p @ v[lo:, h // 2], rtol=1e-11, atol=1e-13)


@pytest.mark.parametrize("bs", [16, 1584])
def test_physical_layout_does_not_change_outputs(bs):
    args = dict(num_q_heads=12, num_kv_heads=2, block_size=bs, seed=21, kv_mode="normal")
    a = kvc.make_case([2000, 37], [4, 2], layout="HND", layout_seed=1, **args)
    b = kvc.make_case([2000, 37], [4, 2], layout="NHD", layout_seed=2, **args)
    assert not torch.equal(a.block_table, b.block_table)
    oa, _ = run_oracle(a)
    ob, _ = run_oracle(b)
    assert np.array_equal(oa, ob)


def test_poisoned_out_of_window_pages_are_never_read():
    args = dict(num_q_heads=6, num_kv_heads=1, block_size=16, seed=4, kv_mode="normal", causal=False,
                window=64)
    clean = kvc.make_case([500, 90], [8, 8], **args)
    poisoned = kvc.make_case([500, 90], [8, 8], poison=True, **args)
    assert poisoned.poisoned_pages > 0
    o1, _ = run_oracle(clean)
    o2, _ = run_oracle(poisoned)
    assert np.isfinite(o2).all()
    assert np.array_equal(o1, o2)


def test_qmax_leaves_extra_rows_unwritten():
    c = kvc.make_case([30, 10], [5, 2], num_q_heads=2, num_kv_heads=1, block_size=8, seed=2)
    _, written = run_oracle(c, qmax=4)
    assert written.tolist() == [True, True, True, True, False, True, True]


def test_quantiser_closed_form():
    g = torch.Generator().manual_seed(0)
    x = torch.randn((64, 4, 256), generator=g) * torch.rand((64, 4, 1), generator=g) * 10
    x[3, 1] = 0.0
    q, s = kvc.quantize_per_token_head(x)
    assert q.dtype == torch.int8 and s.dtype == torch.float32
    assert int(q.abs().max()) == 127 and int(q.min()) >= -127
    nz = s > 0
    assert bool((q.abs().amax(-1)[nz] == 127).all())          # the absmax element maps to +-127
    err = (x - q.float() * s[..., None]).abs()
    assert bool((err <= s[..., None] / 2 + 1e-6 * x.abs().amax(-1, keepdim=True)).all())
    assert float(s[3, 1]) == 0.0 and int(q[3, 1].abs().max()) == 0


@pytest.mark.parametrize("layout", ["HND", "NHD"])
def test_cache_views_alias_the_row_bytes(layout):
    c = kvc.allocate_cache(3, 5, 2, layout)
    c.kv.copy_(torch.randint(-128, 128, c.kv.shape, dtype=torch.int8))
    es = c.key_cache.element_size()
    assert c.value_cache.data_ptr() - c.key_cache.data_ptr() == 260 * es
    assert c.k_scale.data_ptr() - c.key_cache.data_ptr() == 256
    assert c.v_scale.data_ptr() - c.key_cache.data_ptr() == 516
    row = c.kv[2, 1, 3]  # block 2, head 1, slot 3
    assert torch.equal(c.key_cache[2, 3, 1], row[:260])
    assert torch.equal(c.value_cache[2, 3, 1], row[260:])
    assert float(c.k_scale[2, 3, 1]) == float(row[256:260].view(torch.float32)[0]) or math.isnan(
        float(c.k_scale[2, 3, 1]))


def test_int8_to_fp16_widening_is_exact_for_all_256_values():
    # The device widens int8 b to fp16 as bits(0x6400 | (b ^ 0x80)) - 1152; check every b.
    b = np.arange(-128, 128, dtype=np.int32)
    u = (b.astype(np.uint8) ^ 0x80).astype(np.uint16)
    h = (np.uint16(0x6400) | u).view(np.float16)
    assert np.array_equal((h - np.float16(1152)).astype(np.float64), b.astype(np.float64))
