"""The routing shim on the GPU with the real operators: a batch ordered decode-first (two
sequences of 1 and 4 query tokens) then two prefill sequences (100 and 70 tokens) is routed
through the decode operator and the prefill operator and checked against the float64 oracle
(max-abs <= 2e-3, mean-abs <= 2e-4 on fp16 outputs); a 40-sequence decode batch with host-side
lengths goes through the split model the same way.
"""
import numpy as np
import pytest
import torch

import workload as kvc
from mi50_vllm_lab_amd import vllm_shim as shim
from oracle import attention as orc

pytestmark = pytest.mark.gpu


def test_mixed_batch_through_the_shim():
    shim.reset_loaders()
    ctxs, qlens = [500, 37, 1000, 0], [1, 4, 100, 70]
    c = kvc.make_case(ctxs, qlens, num_q_heads=24, num_kv_heads=4, block_size=16, seed=61)
    ref, written = orc.paged_decode(c.q, c.cache.key_cache, c.cache.value_cache, c.cache.k_scale, c.cache.v_scale,
                                    c.block_table, c.seq_lens, c.query_start_loc, c.num_seqs, c.scale)
    d = c.to("cuda")
    T = d.num_tokens
    po, pm, pl = kvc.partial_buffers(T, 24, 64, "cuda")
    meta = shim.AttnMeta(query_start_loc=d.query_start_loc, query_start_loc_cpu=c.query_start_loc.tolist(),
                         seq_lens=d.seq_lens, block_table=d.block_table, max_seq_len=max(c.seqs),
                         softmax_segm_output=po, softmax_segm_max=pm, softmax_segm_expsum=pl)
    impl = shim.Gfx950Int8Attention(num_heads=24, num_kv_heads=4, head_size=256, scale=c.scale,
                                    kv_quant_int8_per_token_head=True, is_rocm=True, is_decoder=True)
    assert impl.pth_dec is not None and impl.pth_fa is not None
    out = torch.full((T, 24, 256), float("nan"), dtype=torch.float16, device="cuda")
    handled = impl.route(d.q, d.cache.key_cache, d.cache.value_cache, d.cache.k_scale, d.cache.v_scale, meta, out,
                         max(qlens), T, lambda *a: pytest.fail("fell back to Triton"))
    torch.cuda.synchronize()
    assert handled and written.all()
    e = np.abs(out.double().cpu().numpy() - ref)
    print(f"shim mixed batch: max-abs {e.max():.2e} mean-abs {e.mean():.2e}", flush=True)
    assert np.isfinite(e).all() and e.max() <= 2e-3 and e.mean() <= 2e-4


def test_decode_batch_with_host_lengths():
    """40 decode sequences with their host-side lengths: the shim's split model picks a small
    split count (a few workgroups per sequence) and the result matches the oracle."""
    shim.reset_loaders()
    g = np.random.default_rng(9)
    ctxs = [int(x) for x in g.integers(100, 6000, 40)]
    qlens = [int(x) for x in g.integers(1, 5, 40)]
    c = kvc.make_case(ctxs, qlens, num_q_heads=24, num_kv_heads=4, block_size=16, seed=62)
    ref, written = orc.paged_decode(c.q, c.cache.key_cache, c.cache.value_cache, c.cache.k_scale, c.cache.v_scale,
                                    c.block_table, c.seq_lens, c.query_start_loc, c.num_seqs, c.scale)
    d = c.to("cuda")
    T = d.num_tokens
    po, pm, pl = kvc.partial_buffers(T, 24, 64, "cuda")
    meta = shim.AttnMeta(query_start_loc=d.query_start_loc, query_start_loc_cpu=c.query_start_loc.tolist(),
                         seq_lens=d.seq_lens, block_table=d.block_table, max_seq_len=max(c.seqs),
                         softmax_segm_output=po, softmax_segm_max=pm, softmax_segm_expsum=pl,
                         seq_lens_cpu=c.seq_lens.tolist())
    nsplit = shim.decode_splits(64, -1, 4, c.num_seqs, "cuda", meta.seq_lens_cpu, 4)
    assert nsplit < 64
    impl = shim.Gfx950Int8Attention(num_heads=24, num_kv_heads=4, head_size=256, scale=c.scale,
                                    kv_quant_int8_per_token_head=True, is_rocm=True, is_decoder=True)
    out = torch.full((T, 24, 256), float("nan"), dtype=torch.float16, device="cuda")
    handled = impl.route(d.q, d.cache.key_cache, d.cache.value_cache, d.cache.k_scale, d.cache.v_scale, meta, out,
                         max(qlens), T, lambda *a: pytest.fail("fell back to Triton"))
    torch.cuda.synchronize()
    assert handled and written.all()
    e = np.abs(out.double().cpu().numpy() - ref)
    print(f"shim decode batch (nsplit {nsplit}): max-abs {e.max():.2e} mean-abs {e.mean():.2e}", flush=True)
    assert np.isfinite(e).all() and e.max() <= 2e-3 and e.mean() <= 2e-4
