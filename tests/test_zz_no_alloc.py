"""pth_dec_launch_noalloc: the decode entry point that allocates nothing (its split partials live
in the library's own per-GPU device array). Checked against pth_dec_launch_window, which takes
the partial buffers from the caller: the two share their kernels, so the outputs must be
bit-identical, on two calls in a row (the second smaller than the first, so it runs over the
first call's leftovers in the array), for causal MTP rows and for windowed non-causal rows.
Also: sizes beyond the array are refused before anything is launched.
"""
import ctypes

import pytest
import torch

import workload as kvc
from mi50_vllm_lab_amd import pth_dec

HQ, HKV = 24, 4
NSEG = 128
HIP_ERROR_OUT_OF_MEMORY = 2
SCRATCH_BYTES = 32 << 20


def say(msg):
    print(msg, flush=True)


def _ptr(t, ty):
    return ctypes.cast(ctypes.c_void_p(t.data_ptr()), ctypes.POINTER(ty))


def _common(c, qmax):
    kc = c.cache.key_cache
    return [ctypes.c_void_p(c.q.data_ptr()), c.q.stride(0), ctypes.c_void_p(kc.data_ptr()), kc.stride(0),
            kc.stride(1), kc.stride(2), _ptr(c.block_table, ctypes.c_int), c.block_table.stride(0),
            _ptr(c.seq_lens, ctypes.c_int), _ptr(c.query_start_loc, ctypes.c_int), c.num_seqs, c.num_tokens, HQ, HKV,
            c.cache.block_size, c.scale, qmax]


def run_window(lib, c, qmax, nsplit, out):
    po, pm, pl = kvc.partial_buffers(c.num_tokens, HQ, NSEG, "cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = _common(c, qmax) + [_ptr(po, ctypes.c_float), _ptr(pm, ctypes.c_float), _ptr(pl, ctypes.c_float), NSEG,
                               nsplit, ctypes.c_void_p(out.data_ptr()), out.stride(0), out.stride(1), stream,
                               c.window, int(c.causal)]
    return lib.pth_dec_launch_window(*args)


def run_noalloc(lib, c, qmax, nsplit, out):
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = _common(c, qmax) + [nsplit, ctypes.c_void_p(out.data_ptr()), out.stride(0), out.stride(1), stream,
                               c.window, int(c.causal)]
    return lib.pth_dec_launch_noalloc(*args)


CASES = [
    # (contexts, query tokens, window, causal, nsplit, seed): each pair runs big then small
    (([20000, 3000], [4, 4], -1, True, 64, 31), ([500], [2], -1, True, 16, 32)),
    (([9000, 2048], [8, 8], 2048, False, 16, 33), ([100], [8], 2048, False, 4, 34)),
]


@pytest.mark.gpu
@pytest.mark.parametrize("pair", CASES, ids=["mtp", "windowed"])
def test_noalloc_matches_window_entry_point(pair):
    lib = pth_dec.load_library()
    for ctxs, qlens, window, causal, nsplit, seed in pair:
        say(f"noalloc vs window: ctxs {ctxs} qlens {qlens} window {window} causal {causal} nsplit {nsplit}")
        c = kvc.make_case(ctxs, qlens, num_q_heads=HQ, num_kv_heads=HKV, block_size=16, seed=seed, window=window,
                          causal=causal).to("cuda")
        qmax = max(qlens)
        ref = torch.full((c.num_tokens, HQ, 256), float("nan"), dtype=torch.float16, device="cuda")
        got = torch.full_like(ref, float("nan"))
        assert run_window(lib, c, qmax, nsplit, ref) == 0
        assert run_noalloc(lib, c, qmax, nsplit, got) == 0
        torch.cuda.synchronize()
        assert torch.isfinite(ref.float()).all()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


@pytest.mark.gpu
def test_noalloc_refuses_sizes_beyond_its_array():
    lib = pth_dec.load_library()
    c = kvc.make_case([300], [4], num_q_heads=HQ, num_kv_heads=HKV, block_size=16, seed=35).to("cuda")
    out = torch.full((c.num_tokens, HQ, 256), float("nan"), dtype=torch.float16, device="cuda")
    # 4 tokens x 24 heads x nsplit x 1032 bytes: nsplit 339 is the first count beyond 32 MiB
    nsplit = SCRATCH_BYTES // (c.num_tokens * HQ * 1032) + 1
    assert run_noalloc(lib, c, 4, nsplit, out) == HIP_ERROR_OUT_OF_MEMORY
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()  # nothing was launched
    assert run_noalloc(lib, c, 4, nsplit - 1, out) == 0
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
