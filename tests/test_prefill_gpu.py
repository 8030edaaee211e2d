"""GPU parity of the gfx950 chunked-prefill operator (forward_pth interface) against the float64
oracle.

Cases follow kernels/fa_pth/test_pth.py:104-106 (its seven (ctx, chunk, layout) cases at block
size 1584, tolerance max-abs < 2e-2) on the full model's heads (24 q / 4 kv), plus the 2048-token
chunk over a 61,440-token context at block size 16 checked to the decode tolerance (max-abs <=
2e-3, mean-abs <= 2e-4) on sampled rows against the oracle and on every row against an fp32
torch reference pinned to the oracle, batches with mixed contexts and chunk offsets,
the generic (block size not a multiple of 16) and global page-table paths, bit-exact invariance
to the physical page layout, and HIP-graph replay.
"""
import math
import sys

import numpy as np
import pytest
import torch

import workload as kvc
from mi50_vllm_lab_amd import pth_dec
from oracle import attention as orc

pytestmark = pytest.mark.gpu

HQ, HKV = 24, 4
BS_REF = 1584


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def oracle_of(c, q_abs, rows=None):
    return orc.paged_prefill(kvc.prefill_query(c), c.cache.key_cache, c.cache.value_cache, c.cache.k_scale,
                             c.cache.v_scale, c.block_table, c.seq_lens, c.scale, torch.tensor(q_abs), rows)


def gpu_prefill(d, q_abs, exact=False, nsplit=None):
    q = kvc.prefill_query(d)
    out = torch.full((q.shape[0], q.shape[2], q.shape[1], 256), float("nan"), dtype=torch.float32, device="cuda")
    pth_dec.forward_pth(q, d.cache.key_cache, d.cache.value_cache, d.block_table, d.seq_lens, d.scale,
                        torch.tensor(q_abs, dtype=torch.int32, device="cuda"), out=out, exact=exact, nsplit=nsplit)
    torch.cuda.synchronize()
    return out


def errors(out, ref, written):
    o = out.double().cpu().numpy()[written]
    e = np.abs(o - ref[written])
    return float(e.max()), float(e.mean())


# kernels/fa_pth/test_pth.py:104-105: (ctx, chunk, NHD)
REF_CASES = [(0, 64, False), (0, 1500, False), (1000, 777, False), (BS_REF * 3 - 5, 2048, False),
             (5000, 2048, True), (20000, 33, False), (12345, 5, False)]


@pytest.mark.parametrize("ctx,n,nhd", REF_CASES, ids=[f"ref{i}" for i in range(len(REF_CASES))])
def test_reference_cases(ctx, n, nhd):
    c = kvc.make_case([ctx], [n], num_q_heads=HQ, num_kv_heads=HKV, block_size=BS_REF,
                      layout="NHD" if nhd else "HND", seed=ctx + n, kv_mode="uniform")
    say(f"prefill ctx={ctx} chunk={n} nhd={nhd}")
    out = gpu_prefill(c.to("cuda"), [ctx])
    rows = None if n <= 800 else list(range(0, 32)) + list(range(n - 32, n)) + list(range(100, n, 97))
    ref, written = oracle_of(c, [ctx], rows)
    emax, emean = errors(out, ref, written)
    say(f"  max-abs {emax:.2e} mean-abs {emean:.2e} |ref| {np.abs(ref[written]).mean():.3f}")
    assert torch.isfinite(out).all()
    assert math.isfinite(emax) and emax < 2e-2, (ctx, n, emax)
    assert emax <= 2e-3 and emean <= 2e-4, (ctx, n, emax, emean)


def torch_prefill_fp32(d, q_abs):
    """fp32 reference of a whole chunk on the GPU: K and V dequantised through the block table, then
    causal softmax(Q K^T * scale) V per kv head with torch matmul in fp32 (no reduced-precision
    matmul). Float64 on every row would take minutes on the CPU; this reference is held to the
    float64 oracle on sampled rows by the test that uses it."""
    q = kvc.prefill_query(d)
    B, Hq, Sq, D = q.shape
    cache = d.cache
    bs, Hkv = cache.block_size, cache.num_kv_heads
    G = Hq // Hkv
    out = torch.empty((B, Sq, Hq, D), dtype=torch.float32, device="cuda")
    for b in range(B):
        seq = int(d.seq_lens[b])
        pos = torch.arange(seq, device="cuda")
        blk = d.block_table[b].long()[pos // bs]
        slot = pos % bs
        rowpos = int(q_abs[b]) + torch.arange(Sq, device="cuda")
        hidden = pos[None, :] > rowpos[:, None]  # [Sq, seq]: keys after the row's position
        for g in range(Hkv):
            k = cache.key_cache[blk, slot, g, :D].float() * cache.k_scale[blk, slot, g][:, None]
            v = cache.value_cache[blk, slot, g, :D].float() * cache.v_scale[blk, slot, g][:, None]
            s = torch.matmul(q[b, g * G:(g + 1) * G], k.t().contiguous()) * d.scale  # [G, Sq, seq]
            s.masked_fill_(hidden[None], float("-inf"))
            p = torch.softmax(s, dim=-1)
            out[b, :, g * G:(g + 1) * G] = torch.matmul(p, v).permute(1, 0, 2)
            del s, p
    return out


@pytest.mark.parametrize("exact", [False, True], ids=["default", "exact"])
def test_chunk_of_2048_over_61440_cached(exact):
    """A 2,048-token chunk over 61,440 cached keys at full size: 32 rows against the float64
    oracle, and every one of the 2,048 x 24 rows against the fp32 torch reference, which must
    itself agree with the oracle on those 32 rows to 1e-5."""
    c = kvc.make_case([61440], [2048], num_q_heads=HQ, num_kv_heads=HKV, block_size=16, seed=1005)
    say(f"prefill 2048 over 61440, bs 16, exact={exact}")
    d = c.to("cuda")
    out = gpu_prefill(d, [61440], exact)
    rng = np.random.default_rng(5)
    rows = sorted(set([0, 1, 31, 32, 2047] + rng.choice(2048, 27, replace=False).tolist()))
    ref, written = oracle_of(c, [61440], rows)
    emax, emean = errors(out, ref, written)
    say(f"  sampled rows vs oracle: max-abs {emax:.2e} mean-abs {emean:.2e}")
    assert torch.isfinite(out).all()
    assert emax <= 2e-3 and emean <= 2e-4, (emax, emean)

    allow_tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        tref = torch_prefill_fp32(d, [61440])
    finally:
        torch.backends.cuda.matmul.allow_tf32 = allow_tf32
    pin = float(np.abs(tref.double().cpu().numpy()[written] - ref[written]).max())
    say(f"  torch fp32 reference vs oracle on the sampled rows: max-abs {pin:.2e}")
    assert pin <= 1e-5, pin
    e = (out - tref).abs()
    emax_all, emean_all = float(e.max()), float(e.mean())
    say(f"  all rows vs torch fp32: max-abs {emax_all:.2e} mean-abs {emean_all:.2e}")
    assert emax_all <= 2e-3 and emean_all <= 2e-4, (emax_all, emean_all)


@pytest.mark.parametrize("bs,layout", [(16, "HND"), (16, "NHD"), (8, "HND"), (1, "NHD"), (48, "HND")])
def test_batches_with_chunk_offsets(bs, layout):
    ctxs, sq = [3000, 0, 517], 70
    c = kvc.make_case(ctxs, [sq] * 3, num_q_heads=HQ, num_kv_heads=HKV, block_size=bs, layout=layout,
                      seed=bs * 3 + len(layout))
    # sequence 0: the chunk ends the sequence; 1: rows before its first key and in the middle;
    # 2: the chunk starts past the end (every row sees every key)
    q_abs = [3000, -20, 700]
    say(f"prefill batch bs={bs} layout={layout}")
    out = gpu_prefill(c.to("cuda"), q_abs)
    ref, written = oracle_of(c, q_abs)
    assert not written[1, :20].any() and written[1, 20:].all()
    for b in range(3):
        emax, emean = errors(out[b:b + 1], ref[b:b + 1], written[b:b + 1])
        say(f"  seq {b}: max-abs {emax:.2e} mean-abs {emean:.2e}")
        assert emax <= 2e-3 and emean <= 2e-4, (b, emax, emean)
    assert (out.cpu().numpy()[~written] == 0).all()  # rows that see no key are written as 0


@pytest.mark.parametrize("hq,hkv", [(8, 8), (32, 4), (28, 4), (48, 2)])
def test_gqa_group_sizes(hq, hkv):
    """G = 1, 8, 7 (192 rows per workgroup is not a multiple of 7: 27 tokens) and 24."""
    c = kvc.make_case([900, 40], [77, 77], num_q_heads=hq, num_kv_heads=hkv, block_size=16, seed=hq + 5 * hkv)
    q_abs = [900, 10]
    say(f"prefill gqa hq={hq} hkv={hkv}")
    out = gpu_prefill(c.to("cuda"), q_abs)
    ref, written = oracle_of(c, q_abs)
    emax, emean = errors(out, ref, written)
    say(f"  max-abs {emax:.2e} mean-abs {emean:.2e}")
    assert emax <= 2e-3 and emean <= 2e-4, (emax, emean)


def abs_value_case(c):
    """The case with every V quant replaced by its absolute value. The quantised rows hold
    [-127, 127]; only unused slots (never read) can hold -128."""
    cache = kvc.clone_cache(c.cache)
    v = cache.value_cache[..., :256]
    v.copy_(v.abs())
    return kvc.DecodeCase(c.q, cache, c.block_table, c.seq_lens, c.query_start_loc, list(c.ctxs), list(c.qlens),
                          c.num_q_heads, c.scale)


def test_outlier_rows_within_fp16_weight_rounding():
    """P' = p * v_scale enters the MFMA as fp16: each weight carries at most half an fp16 ulp
    (2^-12) of relative error, so |err| <= 2^-12 * sum_k p_k |V_k| / l per element; the bound
    checked is 2e-3 + 2^-11 * that sum (exact, from the oracle on |V|). 1% of the K and V rows
    are 50x outliers, as in the decode operator's long-context workload."""
    ctxs, sq = [3000, 517], 70
    c = kvc.make_case(ctxs, [sq] * 2, num_q_heads=HQ, num_kv_heads=HKV, block_size=16, seed=41,
                      outlier_frac=0.01, outlier_mult=50.0)
    q_abs = [3000, 400]
    say("prefill outliers")
    out = gpu_prefill(c.to("cuda"), q_abs)
    ref, written = oracle_of(c, q_abs)
    mag, _ = oracle_of(abs_value_case(c), q_abs)
    err = np.abs(out.double().cpu().numpy() - ref)[written]
    bound = 2e-3 + 2.0 ** -11 * mag[written]
    say(f"  max-abs {err.max():.2e} max |ref| {np.abs(ref[written]).max():.1f} worst err/bound {(err / bound).max():.3f}")
    assert (err <= bound).all()


def test_exact_outlier_rows_within_decode_tolerance():
    """pth_fa_forward_exact on the outlier case above: K and V are widened without bias and P' is
    carried as fp16 hi + lo, so the P' rounding (2^-12 relative per weight, times |V| up to 50
    v_scale) drops to ~2^-23 and the plain bar holds: max-abs <= 2e-3, mean-abs <= 2e-4. A second
    case puts 2% of the rows at 100x, with a 640-key context and the chunk inside the cache."""
    for ctxs, q_abs, frac, mult, seed in [([3000, 517], [3000, 400], 0.01, 50.0, 41),
                                          ([640, 2900], [600, 2900], 0.02, 100.0, 43)]:
        c = kvc.make_case(ctxs, [70] * 2, num_q_heads=HQ, num_kv_heads=HKV, block_size=16, seed=seed,
                          outlier_frac=frac, outlier_mult=mult)
        say(f"exact prefill outliers {frac} x{mult}")
        d = c.to("cuda")
        out = gpu_prefill(d, q_abs, exact=True)
        ref, written = oracle_of(c, q_abs)
        emax, emean = errors(out, ref, written)
        dmax, dmean = errors(gpu_prefill(d, q_abs), ref, written)
        say(f"  exact: max-abs {emax:.2e} mean-abs {emean:.2e}; default: max-abs {dmax:.2e} mean-abs {dmean:.2e}; "
            f"max |ref| {np.abs(ref[written]).max():.1f}")
        assert torch.isfinite(out).all()
        assert emax <= 2e-3 and emean <= 2e-4, (ctxs, emax, emean)


def test_rows_that_see_one_or_two_keys():
    """A chunk starting 4 positions before a 5-key sequence (G = 4, block size 1, NHD, uniform
    K/V): its written rows see one or two keys, so each output is close to a single V row
    (|out| ~ 2) and P''s fp16 rounding (2^-12 relative) is not averaged over many keys.
    pth_fa_forward stays within the per-element bound of that rounding (and max-abs 2e-3), but
    its mean-abs, 2.5e-4, is above 2e-4; pth_fa_forward_exact meets 2e-3 / 2e-4 (a draw of the
    extended random sweep)."""
    c = kvc.make_case([5], [6], num_q_heads=4, num_kv_heads=1, block_size=1, layout="NHD", seed=9930,
                      kv_mode="uniform")
    q_abs = [-4]
    say("prefill rows seeing 1-2 keys")
    d = c.to("cuda")
    ref, written = oracle_of(c, q_abs)
    mag, _ = oracle_of(abs_value_case(c), q_abs)
    out = gpu_prefill(d, q_abs)
    err = np.abs(out.double().cpu().numpy() - ref)[written]
    bound = 2e-3 + 2.0 ** -11 * mag[written]
    say(f"  default: max-abs {err.max():.2e} mean-abs {err.mean():.2e} worst err/bound {(err / bound).max():.3f}")
    assert err.max() <= 2e-3 and (err <= bound).all()
    emax, emean = errors(gpu_prefill(d, q_abs, exact=True), ref, written)
    say(f"  exact: max-abs {emax:.2e} mean-abs {emean:.2e}")
    assert emax <= 2e-3 and emean <= 2e-4, (emax, emean)


@pytest.mark.parametrize("nsplit", [2, 7, 64])
def test_key_splits_match_the_unsplit_operator(nsplit):
    """pth_fa_forward_split: each query tile's keys split over nsplit workgroups, merged by a second
    kernel. The default numerics against the oracle (2e-3 / 2e-4; each split rounds P' to fp16
    against its own running max, so the split and unsplit results differ by up to that
    rounding), and the exact numerics against the unsplit exact operator, which leaves only the
    order of the fp32 sums: K and V are widened exactly, so those sums are of the result's own
    magnitude and their reordering moves it by at most 3.1e-5 here (1.6e-5 / 3.1e-5 / 2.6e-5 at
    2 / 7 / 64 splits; bound 5e-5). With V widened as v + 1152 the same sums were ~1152 / |v|
    times the result and moved it by up to 6.3e-4. A wrong merge moves it by O(1).
    Sequence 1 has fewer key tiles than 64 splits (empty splits) and rows before its first key
    (written as 0)."""
    ctxs, sq = [3000, 40, 517], 70
    c = kvc.make_case(ctxs, [sq] * 3, num_q_heads=HQ, num_kv_heads=HKV, block_size=16, seed=300 + nsplit)
    q_abs = [3000, -20, 700]
    say(f"prefill split {nsplit}")
    d = c.to("cuda")
    qd = kvc.prefill_query(d)
    qa = torch.tensor(q_abs, dtype=torch.int32, device="cuda")
    def run(n, exact):
        return pth_dec.forward_pth(qd, d.cache.key_cache, d.cache.value_cache, d.block_table, d.seq_lens, d.scale, qa,
                                   nsplit=n, exact=exact)

    split = run(nsplit, False)
    one_x, split_x = run(1, True), run(nsplit, True)
    torch.cuda.synchronize()
    ref, written = oracle_of(c, q_abs)
    emax, emean = errors(split, ref, written)
    diff = float((split_x - one_x).abs().max())
    xmax, xmean = errors(split_x, ref, written)
    say(f"  vs oracle: max-abs {emax:.2e} mean-abs {emean:.2e}; exact: {xmax:.2e} / {xmean:.2e}; "
        f"exact split vs exact unsplit: max {diff:.2e}")
    assert torch.isfinite(split).all() and torch.isfinite(split_x).all()
    assert emax <= 2e-3 and emean <= 2e-4, (emax, emean)
    assert xmax <= 2e-3 and xmean <= 2e-4, (xmax, xmean)
    assert diff <= 5e-5, diff
    assert (split.cpu().numpy()[~written] == 0).all() and (split_x.cpu().numpy()[~written] == 0).all()


def test_key_splits_exact_and_short_chunk_over_long_context():
    """The exact entry through the split path, and a 16-token chunk over 20,000 cached keys (the
    case the split exists for: 4 workgroups without it), against the oracle."""
    c = kvc.make_case([20000], [16], num_q_heads=HQ, num_kv_heads=HKV, block_size=16, seed=321, outlier_frac=0.01)
    q_abs = [20000]
    say("prefill 16 tokens over 20000 keys, split, default and exact")
    d = c.to("cuda")
    qd = kvc.prefill_query(d)
    qa = torch.tensor(q_abs, dtype=torch.int32, device="cuda")
    assert pth_dec.prefill_splits(1, 16, HQ, HKV, d.block_table.shape[1] * 16) > 1
    ref, written = oracle_of(c, q_abs)
    mag, _ = oracle_of(abs_value_case(c), q_abs)
    out = pth_dec.forward_pth(qd, d.cache.key_cache, d.cache.value_cache, d.block_table, d.seq_lens, d.scale, qa)
    ex = pth_dec.forward_pth(qd, d.cache.key_cache, d.cache.value_cache, d.block_table, d.seq_lens, d.scale, qa,
                             exact=True)
    torch.cuda.synchronize()
    err = np.abs(out.double().cpu().numpy() - ref)[written]
    assert (err <= 2e-3 + 2.0 ** -11 * mag[written]).all()
    emax, emean = errors(ex, ref, written)
    say(f"  default max-abs {err.max():.2e}; exact max-abs {emax:.2e} mean-abs {emean:.2e}")
    assert emax <= 2e-3 and emean <= 2e-4, (emax, emean)


EXACT_CASES = [REF_CASES[i] for i in (0, 2, 3, 4, 6)]


@pytest.mark.parametrize("ctx,n,nhd", EXACT_CASES, ids=[f"ref{i}" for i in (0, 2, 3, 4, 6)])
def test_exact_reference_cases(ctx, n, nhd):
    c = kvc.make_case([ctx], [n], num_q_heads=HQ, num_kv_heads=HKV, block_size=BS_REF,
                      layout="NHD" if nhd else "HND", seed=ctx + n, kv_mode="uniform")
    say(f"exact prefill ctx={ctx} chunk={n} nhd={nhd}")
    out = gpu_prefill(c.to("cuda"), [ctx], exact=True)
    rows = None if n <= 800 else list(range(0, 32)) + list(range(n - 32, n)) + list(range(100, n, 97))
    ref, written = oracle_of(c, [ctx], rows)
    emax, emean = errors(out, ref, written)
    say(f"  max-abs {emax:.2e} mean-abs {emean:.2e}")
    assert torch.isfinite(out).all()
    assert emax <= 2e-3 and emean <= 2e-4, (ctx, n, emax, emean)


@pytest.mark.parametrize("bs,layout,hq,hkv", [(16, "HND", 24, 4), (8, "NHD", 28, 4), (1, "HND", 8, 8),
                                              (48, "NHD", 48, 2)])
def test_exact_batches_and_group_sizes(bs, layout, hq, hkv):
    """The exact entry on the batch shapes of the default's tests: chunk offsets before the first
    key, inside and past the cache, rows that see no key (written as 0), and G = 6, 7, 1, 24."""
    ctxs, sq = [3000, 0, 517], 70
    c = kvc.make_case(ctxs, [sq] * 3, num_q_heads=hq, num_kv_heads=hkv, block_size=bs, layout=layout,
                      seed=200 + bs + hq)
    q_abs = [3000, -20, 700]
    say(f"exact prefill batch bs={bs} layout={layout} hq={hq} hkv={hkv}")
    out = gpu_prefill(c.to("cuda"), q_abs, exact=True)
    ref, written = oracle_of(c, q_abs)
    emax, emean = errors(out, ref, written)
    say(f"  max-abs {emax:.2e} mean-abs {emean:.2e}")
    assert emax <= 2e-3 and emean <= 2e-4, (emax, emean)
    assert (out.cpu().numpy()[~written] == 0).all()


@pytest.mark.parametrize("bs,nsplit", [(16, 1), (8, 1), (16, None), (8, None)])
def test_page_table_beyond_lds(bs, nsplit):
    """nsplit 1: a workgroup streams more 16-key blocks (bs 16: 6,252) or pages (bs 8: 12,500)
    than its LDS table holds (6,144 entries), so the tile addresses come from the global block
    table: the 16-key-block path at bs 16, the per-row path at bs 8. nsplit None (forward_pth's
    pick, 32 splits of ~98 tiles): each split's slice fits the LDS table again."""
    ctx = 100000
    c = kvc.make_case([ctx], [40], num_q_heads=HQ, num_kv_heads=HKV, block_size=bs, seed=21 + bs)
    if nsplit == 1:  # more entries than the LDS table's 6,144: 16-key blocks at bs 16, pages at bs 8
        assert -(-(ctx + 40) // 16) > 6144 and -(-(ctx + 40) // bs) > 6144
    say(f"prefill global page table bs={bs} nsplit={nsplit}")
    out = gpu_prefill(c.to("cuda"), [ctx], nsplit=nsplit)
    ref, written = oracle_of(c, [ctx], [0, 13, 39])
    emax, emean = errors(out, ref, written)
    say(f"  max-abs {emax:.2e} mean-abs {emean:.2e}")
    assert emax <= 2e-3 and emean <= 2e-4, (emax, emean)


@pytest.mark.parametrize("bs", [16, 1584, 8])
def test_physical_layout_bit_exact(bs):
    args = dict(num_q_heads=HQ, num_kv_heads=HKV, block_size=bs, seed=78)
    a = kvc.make_case([2500, 300], [100, 100], layout="HND", layout_seed=5, **args).to("cuda")
    b = kvc.make_case([2500, 300], [100, 100], layout="NHD", layout_seed=6, **args).to("cuda")
    say(f"prefill layout invariance bs {bs}")
    oa = gpu_prefill(a, [2500, 300])
    ob = gpu_prefill(b, [2500, 300])
    assert torch.equal(oa.view(torch.int32), ob.view(torch.int32))


@pytest.mark.parametrize("nsplit", [1, None])
def test_hip_graph_capture_and_replay(nsplit):
    """Captured once, replayed three times, each replay bit-equal to the eager call: the unsplit
    launch, and (nsplit None: forward_pth's pick, 8 splits here) the split launch with its merge
    and the workspace taken from the graph's pool."""
    c = kvc.make_case([5000], [256], num_q_heads=HQ, num_kv_heads=HKV, block_size=16, seed=31).to("cuda")
    if nsplit is None:
        assert pth_dec.prefill_splits(1, 256, HQ, HKV, c.block_table.shape[1] * 16) > 1
    q = kvc.prefill_query(c)
    qa = torch.tensor([5000], dtype=torch.int32, device="cuda")
    ref = gpu_prefill(c, [5000], nsplit=nsplit)
    out = torch.zeros_like(ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            pth_dec.forward_pth(q, c.cache.key_cache, c.cache.value_cache, c.block_table, c.seq_lens, c.scale, qa,
                                out=out, nsplit=nsplit)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        say(f"graph replay {i}")
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32))
