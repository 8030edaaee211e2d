"""CPU tests of the vLLM routing shim (mi50-vllm-lab_amd/vllm_shim.py) with recording stand-ins
for the operators: the gating of triton_attn.patch:91-114 (and where it is relaxed), the
thresholds and fallbacks of :116-174 and :272-308, the suffix detection of :192-198, the
prefix routing of :199-242 and the per-sequence prefill calls of :243-262, and the loaders'
switches and failure handling (:15-70).
"""
import logging

import pytest
import torch

from mi50_vllm_lab_amd import vllm_shim as shim


class FakeOps:
    def __init__(self, layout_ok=True):
        self.calls = []
        self.layout_ok = layout_ok

    def supported_layout(self, kc, vc, ks, vs):
        self.calls.append(("layout",))
        return self.layout_ok

    def decode(self, q, kc, vc, ks, vs, bt, sl, qsl, out, scale, po, pm, pl, num_seqs, qmax, nsplit, window=-1,
               causal=True):
        self.calls.append(("decode", q.shape[0], num_seqs, qmax, nsplit, window, bt.shape[0]))
        out.fill_(1.0)

    def forward_pth(self, q, kc, vc, bt, sl, scale, q_abs, exact=False, max_keys=None):
        self.calls.append(("prefill", tuple(q.shape), int(sl[0]), int(q_abs[0]), q.dtype))
        self.exact = getattr(self, "exact", []) + [exact]
        self.max_keys = getattr(self, "max_keys", []) + [max_keys]
        return torch.full((1, q.shape[2], q.shape[1], q.shape[3]), 2.0)


@pytest.fixture
def ops(monkeypatch):
    f = FakeOps()
    monkeypatch.setattr(shim, "load_pth_dec", lambda: f)
    monkeypatch.setattr(shim, "load_pth_fa", lambda: f)
    return f


def impl(**kw):
    args = dict(num_heads=24, num_kv_heads=4, head_size=256, scale=0.0625, kv_quant_int8_per_token_head=True,
                is_rocm=True, is_decoder=True)
    args.update(kw)
    return shim.Gfx950Int8Attention(**args)


def meta(qlens, seqs, nseg=64, hq=24, segm=True, causal=True):
    qsl = [0]
    for q in qlens:
        qsl.append(qsl[-1] + q)
    T = qsl[-1]
    return shim.AttnMeta(
        query_start_loc=torch.tensor(qsl, dtype=torch.int32), query_start_loc_cpu=qsl,
        seq_lens=torch.tensor(seqs, dtype=torch.int32), block_table=torch.zeros((len(seqs), 8), dtype=torch.int32),
        max_seq_len=max(seqs), causal=causal,
        softmax_segm_output=torch.empty((max(T, 1), hq, nseg, 256)) if segm else None,
        softmax_segm_max=torch.empty((max(T, 1), hq, nseg)) if segm else None,
        softmax_segm_expsum=torch.empty((max(T, 1), hq, nseg)) if segm else None)


def tensors(T, hq=24):
    q = torch.randn((T, hq, 256))
    out = torch.zeros((T, hq, 256))
    kc = torch.zeros((4, 16, 4, 260), dtype=torch.int8)
    return q, out, kc


@pytest.mark.parametrize("kw,fa,dec", [
    ({}, True, True),
    ({"kv_quant_int8_per_token_head": False}, False, False),
    ({"is_rocm": False}, False, False),
    ({"is_decoder": False}, False, False),
    ({"head_size": 128}, False, False),
    ({"sinks": torch.zeros(24)}, False, False),
    ({"alibi_slopes": torch.zeros(24)}, False, False),
    ({"logits_soft_cap": 30.0}, False, False),
    ({"chunk_lookback": 128}, False, False),
    ({"use_td": True}, False, False),
    ({"on_gfx950": False}, False, False),
    ({"sliding_window": (2047, -1)}, False, True),        # decode takes the window, prefill does not
    ({"num_heads": 32, "num_kv_heads": 4}, True, True),   # G 8: 4 x 8 = 32 rows
    ({"num_heads": 52, "num_kv_heads": 4}, True, False),  # G 13: 52 rows > 48
])
def test_gating(ops, kw, fa, dec):
    a = impl(**kw)
    assert (a.pth_fa is not None) == fa and (a.pth_dec is not None) == dec


def test_window_is_passed_as_left_width(ops):
    a = impl(sliding_window=(2047, -1))
    assert a.window == 2048
    q, out, kc = tensors(8)
    m = meta([4, 4], [5000, 300])
    assert a.route(q, kc, kc, None, None, m, out, 4, 8, lambda *x: None)
    assert ops.calls[-1][5] == 2048


def test_decode_rows_route_to_decode_with_nsplit_cap(ops):
    a = impl()
    q, out, kc = tensors(6)
    m = meta([4, 1, 1], [100, 50, 7], nseg=32)
    assert a.route(q, kc, kc, None, None, m, out, 4, 6, lambda *x: pytest.fail("fallback"))
    assert ops.calls == [("layout",), ("decode", 6, 3, 4, 32, -1, 3)]
    assert (out == 1).all()


@pytest.mark.parametrize("nseqs,nseg,want", [(4, 64, 8), (1, 64, 32), (2, 24, 16), (2, 12, 12), (80, 64, 1)])
def test_window_rows_fill_one_round_of_workgroups(ops, nseqs, nseg, want):
    """With a sliding window the split count fills one round of partial workgroups (256 CUs on a
    CPU device). These groups have 4 x 6 = 24 rows, which the operator runs as two 16-row
    slices: CUs / (kv heads x sequences x 2), while that is at least 2 (80 sequences: the
    unsliced rule, CUs / (kv heads x sequences), gives 1)."""
    a = impl(sliding_window=(2047, -1))
    q, out, kc = tensors(4 * nseqs)
    m = meta([4] * nseqs, [3000 + 7 * i for i in range(nseqs)], nseg=nseg)
    assert a.route(q, kc, kc, None, None, m, out, 4, 4 * nseqs, lambda *x: pytest.fail("fallback"))
    assert ops.calls[-1][0] == "decode" and ops.calls[-1][4] == want
    assert shim.decode_splits(nseg, -1, 4, nseqs, "cpu") == min(64, nseg)  # no window: no cap


# (seq_lens incl. query tokens, qmax, window) -> the split count that measured fastest on
# MI355X (µs per layer at 1 / 2 / 4 / 8 / 16 / 32 / 64 splits, 24 q / 4 kv heads, bs 16)
MEASURED_BEST = [
    ([8196] * 16, 4, -1, 4),                    # 171 / 98 / 72 / 83 / 103 / 141 / 202
    ([4097] * 64, 1, -1, 1),                    # 124 / 124 / 133 / 159 / 203 / 271 / 411
    ([120004] + [2052] * 7, 4, -1, 32),         # 1993 / 1011 / 519 / 273 / 151 / 91 / 119
    ([61444], 4, -1, 64),                       # MTP verify, 4 tokens over 61k
    ([4097], 1, -1, 64),                        # one token over 4k: 15.1 at 16, 13.4 at 32, 12.2 at 64
    ([2056, 9224, 33800, 122888], 8, 2048, 5),   # 4 x 8 windowed rows, sliced: 19.7 at 5; unsliced 25.7 at 8, 24.1 at 16
]


def test_limits_match_the_operator_source():
    """The shim mirrors two limits of the decode operator: the rows per kv head it accepts
    (16 x kMaxRowBlocks) and the sequences x window up to which it slices row groups
    (kSliceKeys). Both are read from the operator's source so the two cannot drift apart."""
    import os
    import re
    src = open(os.path.join(os.path.dirname(shim.__file__), "csrc", "pd_kernels.hpp")).read()
    blocks = int(re.search(r"constexpr int kMaxRowBlocks = (\d+);", src).group(1))
    keys = int(re.search(r"constexpr int64_t kSliceKeys = (\d+);", src).group(1))
    assert shim.MAX_ROWS_PER_KV_HEAD == 16 * blocks
    assert shim.SLICE_KEYS == keys


def test_sliced_splits_rule():
    """Windowed groups of more than 16 rows: the largest split count at which slices of 16 rows
    still fill one round of workgroups, if at least 2 (else 0: the makespan model decides)."""
    ss = shim.sliced_splits
    assert ss(2048, 8, 6, 4, 4, 256, 64) == 5        # 4 x 8 windowed rows: 48 per group, 3 slices
    assert ss(2048, 8, 6, 4, 1, 256, 64) == 21
    assert ss(2048, 4, 6, 4, 4, 256, 64) == 8        # 24 rows, 2 slices
    assert ss(2048, 8, 6, 4, 16, 256, 64) == 0       # only 1 split would fit
    assert ss(2048, 8, 6, 4, 1, 256, 16) == 16       # capped at nseg
    assert ss(4096, 8, 6, 4, 2, 256, 64) == 10
    assert ss(8192, 8, 6, 4, 2, 256, 64) == 10       # 2 x 8,192 = 16,384 keys: still sliced
    assert ss(8193, 8, 6, 4, 2, 256, 64) == 0        # past 16,384 keys of windows
    assert ss(16384, 8, 6, 4, 1, 256, 64) == 21
    assert ss(8192, 8, 6, 4, 4, 256, 64) == 0        # 4 x 8,192: measured slower sliced
    assert ss(-1, 8, 6, 4, 1, 256, 64) == 0          # no window
    assert ss(2048, 2, 6, 4, 1, 256, 64) == 0        # 12 rows: one row block, nothing to slice
    # the model is consulted only when slicing does not apply
    assert shim.decode_splits(64, 2048, 4, 16, "cpu", [4104] * 16, 8) == \
        shim.decode_splits(64, 2048, 4, 16, "cpu", [4104] * 16, 8, 24)


@pytest.mark.parametrize("lens,qmax,window,best", MEASURED_BEST)
def test_split_model_picks_the_measured_best(lens, qmax, window, best):
    assert shim.decode_splits(64, window, 4, len(lens), "cpu", lens, qmax) == best
    assert shim.decode_splits(16, window, 4, len(lens), "cpu", lens, qmax) <= 16  # never above nseg


def test_route_passes_host_lengths_to_the_split_model(ops):
    a = impl()
    nseq = 16
    q, out, kc = tensors(4 * nseq)
    m = meta([4] * nseq, [8196] * nseq)
    m.seq_lens_cpu = [8196] * nseq
    assert a.route(q, kc, kc, None, None, m, out, 4, 4 * nseq, lambda *x: pytest.fail("fallback"))
    assert ops.calls[-1][0] == "decode" and ops.calls[-1][4] == 4
    m2 = meta([4] * nseq, [8196] * nseq)  # no host lengths, no window: the reference's cap
    assert a.route(q, kc, kc, None, None, m2, out, 4, 4 * nseq, lambda *x: None)
    assert ops.calls[-1][4] == 64


def test_graph_capture_ignores_host_lengths(ops, monkeypatch):
    """vLLM captures decode graphs with short dummy lengths: a split count fitted to them would be
    frozen into the graph and replayed on long contexts. While capturing, the split is sized
    without host lengths (the cap; one round of workgroups for windowed rows)."""
    nseq = 8
    q, out, kc = tensors(nseq)
    m = meta([1] * nseq, [1] * nseq)
    m.seq_lens_cpu = [1] * nseq
    assert impl().route(q, kc, kc, None, None, m, out, 1, nseq, lambda *x: pytest.fail("fallback"))
    assert ops.calls[-1][4] == 1  # eager: the model fits the short lengths
    monkeypatch.setattr(shim, "_capturing", lambda device: True)
    assert impl().route(q, kc, kc, None, None, m, out, 1, nseq, lambda *x: pytest.fail("fallback"))
    assert ops.calls[-1][4] == 64  # captured: the cap, whatever the dummy lengths
    assert impl(sliding_window=(2047, -1)).route(q, kc, kc, None, None, m, out, 1, nseq, lambda *x: None)
    assert ops.calls[-1][4] == 256 // (4 * nseq)  # windowed: one round of workgroups


@pytest.mark.parametrize("why", ["no_segm", "too_many_tokens", "q_stride", "layout", "mid_q", "noncausal"])
def test_decode_fallbacks(monkeypatch, why):
    f = FakeOps(layout_ok=why != "layout")
    monkeypatch.setattr(shim, "load_pth_dec", lambda: f)
    monkeypatch.setattr(shim, "load_pth_fa", lambda: f)
    a = impl()
    q, out, kc = tensors(4)
    m = meta([4], [100], segm=why != "no_segm", causal=why != "noncausal")
    if why == "too_many_tokens":
        m.softmax_segm_output = torch.empty((2, 24, 64, 256))
    if why == "q_stride":
        q = torch.randn((4, 24, 512))[..., :256]
    maxq = 10 if why == "mid_q" else 4
    assert not a.route(q, kc, kc, None, None, m, out, maxq, 4, lambda *x: None)
    assert not any(c[0] == "decode" for c in f.calls)


def test_layout_checked_once(ops):
    a = impl()
    q, out, kc = tensors(4)
    m = meta([4], [100])
    for _ in range(3):
        a.route(q, kc, kc, None, None, m, out, 4, 4, lambda *x: None)
    assert sum(1 for c in ops.calls if c[0] == "layout") == 1


def test_prefill_suffix_with_decode_prefix(ops):
    a = impl()
    q, out, kc = tensors(2 + 100 + 70)
    m = meta([1, 1, 100, 70], [500, 40, 1100, 70])
    assert a.route(q, kc, kc, None, None, m, out, 100, 172, lambda *x: pytest.fail("fallback"))
    dec = [c for c in ops.calls if c[0] == "decode"]
    pre = [c for c in ops.calls if c[0] == "prefill"]
    assert dec == [("decode", 2, 2, 1, 64, -1, 2)]
    assert pre == [("prefill", (1, 24, 100, 256), 1100, 1000, torch.float32),
                   ("prefill", (1, 24, 70, 256), 70, 0, torch.float32)]
    assert (out[:2] == 1).all() and (out[2:] == 2).all()


@pytest.mark.parametrize("nq,ctx", [(64, 0), (700, 0), (2560, 0), (5824, 0), (2048, 61440)])
def test_prefill_split_planned_for_the_host_length(ops, monkeypatch, nq, ctx):
    """vLLM's block table is as wide as max_model_len. The shim passes each sequence's host length
    to forward_pth, so a short prompt under a 131,072-key table is planned for its own keys
    (a fresh prompt up to ~5.8k tokens fills the GPU unsplit), not for the table's width; the
    table width is used only while a graph is being captured or without host lengths."""
    from mi50_vllm_lab_amd import pth_dec as pdm
    a = impl()
    q, out, kc = tensors(nq)
    m = meta([nq], [ctx + nq])
    m.block_table = torch.zeros((1, 131072 // 16), dtype=torch.int32)
    m.seq_lens_cpu = [ctx + nq]
    assert a.route(q, kc, kc, None, None, m, out, nq, nq, lambda *x: pytest.fail("fallback"))
    assert ops.max_keys[-1] == ctx + nq
    planned = pdm.prefill_splits(1, nq, 24, 4, ops.max_keys[-1])
    if ctx == 0 and nq >= 700:
        assert planned == 1
    # what the table width alone would plan: every chunk as if over 131,072 keys
    wide = pdm.prefill_splits(1, nq, 24, 4, m.block_table.shape[1] * kc.shape[1])
    assert planned <= wide
    m.seq_lens_cpu = None  # no host lengths: the batch's max_seq_len
    assert a.route(q, kc, kc, None, None, m, out, nq, nq, lambda *x: pytest.fail("fallback"))
    assert ops.max_keys[-1] == ctx + nq
    monkeypatch.setattr(shim, "_capturing", lambda device: True)  # capture: the table width
    m.seq_lens_cpu = [ctx + nq]
    assert a.route(q, kc, kc, None, None, m, out, nq, nq, lambda *x: pytest.fail("fallback"))
    assert ops.max_keys[-1] is None


def test_prefill_split_plan_of_a_short_prompt_under_a_wide_table():
    """The planning numbers behind the test above: under a 131,072-key table a 700-token fresh
    prompt was planned with 11 splits (a 191 MB workspace) and a 64-token one with 32; planned
    for their own keys both run unsplit."""
    from mi50_vllm_lab_amd import pth_dec as pdm
    assert pdm.prefill_splits(1, 700, 24, 4, 131072) > 1
    assert pdm.prefill_splits(1, 700, 24, 4, 700) == 1
    assert pdm.prefill_splits(1, 64, 24, 4, 131072) > 1
    assert pdm.prefill_splits(1, 64, 24, 4, 64) == 1


@pytest.mark.parametrize("exact", [False, True])
def test_prefill_exact_switch(ops, monkeypatch, exact):
    """VLLM_GFX950_PTH_FA_EXACT=1 (read at import into PTH_FA_EXACT) sends every prefill call to
    the exact entry; by default the call carries no exact flag."""
    monkeypatch.setattr(shim, "PTH_FA_EXACT", exact)
    a = impl()
    q, out, kc = tensors(100 + 70)
    m = meta([100, 70], [1100, 70])
    assert a.route(q, kc, kc, None, None, m, out, 100, 170, lambda *x: pytest.fail("fallback"))
    assert ops.exact == [exact, exact]


def test_prefill_prefix_too_long_for_decode_goes_to_triton(ops):
    a = impl()
    q, out, kc = tensors(10 + 80)
    m = meta([10, 80], [200, 500])
    seen = []
    assert a.route(q, kc, kc, None, None, m, out, 80, 90, lambda *x: seen.append(x))
    assert seen == [(0, 10, 0, 1, 10)]
    assert not any(c[0] == "decode" for c in ops.calls)


def test_no_prefill_suffix_falls_through(ops):
    a = impl()
    q, out, kc = tensors(100 + 1)
    m = meta([100, 1], [300, 20])          # the long sequence is not a suffix
    assert not a.route(q, kc, kc, None, None, m, out, 100, 101, lambda *x: pytest.fail("fallback"))
    assert not ops.calls


def test_loader_switches_and_failures(monkeypatch, caplog):
    shim.reset_loaders()
    monkeypatch.setenv("VLLM_GFX950_PTH_DEC", "0")
    assert shim.load_pth_dec() is None
    shim.reset_loaders()
    monkeypatch.setenv("VLLM_GFX950_PTH_DEC", "1")
    monkeypatch.setenv("VLLM_GFX950_PTH_DEC_LIB", "/nonexistent/libpthdec.so")
    with caplog.at_level(logging.WARNING):
        assert shim.load_pth_dec() is None
    assert "stays on Triton" in caplog.text
    shim.reset_loaders()
    monkeypatch.delenv("VLLM_GFX950_PTH_DEC_LIB")
    monkeypatch.setenv("VLLM_GFX950_PTH_FA", "0")
    assert shim.load_pth_fa() is None
    shim.reset_loaders()
