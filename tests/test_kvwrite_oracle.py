"""Pins the KV-cache writer oracle (oracle/kvwrite.py) on the CPU.

vLLM's writer is not in the reference (un-vendored fork); the oracle is pinned by the closed form
on hand-built rows (zero rows, exact multiples, ties rounding half to even, clamping at +-127),
the round-trip bound |q * scale - x| <= scale / 2, agreement with the independent torch quantiser
used to build the synthetic caches (mi50-vllm-lab_amd/kvcache.py), and the slot semantics
(negative slots skipped, other rows untouched, HND and NHD layouts).
"""
import numpy as np
import pytest
import torch

import workload as kvc
from oracle import kvwrite as kvw


def test_zero_row_has_zero_scale_and_quants():
    q, s = kvw.quantize_rows(np.zeros((2, 256), np.float32))
    assert (s == 0).all() and (q == 0).all()


def test_closed_form_on_exact_multiples_and_ties():
    x = np.zeros(256, np.float32)
    x[0] = 127.0                      # absmax 127 -> scale exactly 1
    x[1:6] = [2.5, 3.5, -2.5, -0.5, 1.5]
    x[6] = -127.0
    q, s = kvw.quantize_rows(x[None])
    assert s[0] == np.float32(1.0)
    assert q[0, 0] == 127 and q[0, 6] == -127
    assert list(q[0, 1:6]) == [2, 4, -2, 0, 2]  # rint: half to even


def test_scale_is_absmax_over_127_and_extremes_map_to_127():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((50, 4, 256)).astype(np.float32) * rng.uniform(0.01, 50, (50, 4, 1)).astype(np.float32)
    q, s = kvw.quantize_rows(x)
    np.testing.assert_array_equal(s, (np.abs(x).max(-1) / np.float32(127)).astype(np.float32))
    am = np.abs(x).argmax(-1)
    assert (np.abs(np.take_along_axis(q.astype(np.int32), am[..., None], -1)) == 127).all()


def test_round_trip_bound():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((100, 256)) * 3).astype(np.float32)
    q, s = kvw.quantize_rows(x)
    err = np.abs(q.astype(np.float64) * s[:, None].astype(np.float64) - x)
    assert (err <= s[:, None].astype(np.float64) * 0.5 * (1 + 1e-6)).all()


def test_subnormal_scales_are_kept():
    """Rows of absmax ~1e-37 have subnormal scales (1 / scale overflows float32 for most of
    them): the scale is not flushed to zero, the extremes still map to +-127 and the round-trip
    bound holds (the scale keeps ~19 significant bits at this size)."""
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((40, 256)) * rng.uniform(0.3, 3.0, (40, 1)) * 1e-37).astype(np.float32)
    q, s = kvw.quantize_rows(x)
    tiny = np.finfo(np.float32).tiny
    assert ((s > 0) & (s < tiny)).all()
    with np.errstate(over="ignore"):
        assert np.isinf(np.float32(1) / s).any() and np.isfinite(np.float32(1) / s).any()
    am = np.abs(x).argmax(-1)
    assert (np.abs(np.take_along_axis(q.astype(np.int32), am[:, None], -1)) == 127).all()
    err = np.abs(q.astype(np.float64) * s[:, None].astype(np.float64) - x)
    assert (err <= s[:, None].astype(np.float64) * 0.5 * (1 + 1e-5)).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_agrees_with_the_torch_quantiser(dtype):
    g = torch.Generator().manual_seed(5)
    x = (torch.randn((64, 4, 256), generator=g) * 2).to(dtype)
    q1, s1 = kvw.quantize_rows(x.float())
    q2, s2 = kvc.quantize_per_token_head(x)
    np.testing.assert_array_equal(q1, q2.numpy())
    np.testing.assert_array_equal(s1, s2.numpy())


@pytest.mark.parametrize("layout", ["HND", "NHD"])
def test_write_rows_slot_semantics(layout):
    cache = kvc.allocate_cache(6, 16, 2, layout)
    cache.kv.copy_(torch.randint(-128, 128, cache.kv.shape, dtype=torch.int8, generator=torch.Generator().manual_seed(1)))
    before = cache.kv.clone()
    g = torch.Generator().manual_seed(2)
    k = torch.randn((5, 2, 256), generator=g)
    v = torch.randn((5, 2, 256), generator=g)
    slots = torch.tensor([3, -1, 40, 95, 96 * 5], dtype=torch.int64)  # padding and a slot past the cache
    kvw.write_rows(k, v, cache.key_cache, cache.value_cache, cache.k_scale, cache.v_scale, slots)
    kq, ks = kvw.quantize_rows(k)
    vq, vs = kvw.quantize_rows(v)
    for t, slot in [(0, 3), (2, 40), (3, 95)]:
        blk, off = slot // 16, slot % 16
        assert torch.equal(cache.key_cache[blk, off, :, :256], torch.from_numpy(kq[t]))
        assert torch.equal(cache.value_cache[blk, off, :, :256], torch.from_numpy(vq[t]))
        assert torch.equal(cache.k_scale[blk, off], torch.from_numpy(ks[t]))
        assert torch.equal(cache.v_scale[blk, off], torch.from_numpy(vs[t]))
    # every other row is untouched
    mask = torch.ones(cache.key_cache.shape[:3], dtype=torch.bool)
    for slot in (3, 40, 95):
        mask[slot // 16, slot % 16] = False
    assert torch.equal(cache.kv.transpose(1, 2)[mask], before.transpose(1, 2)[mask])

