"""Frozen small decode problems (tests/golden/decode_cases.npz, written by make_golden.py).

The expected outputs were computed once, row by row, from the definition of the reference's
float64 path (kernels/pth_dec/test_dec.py:70-88) with the mask rule of
patches/vllm/gfx906_fa_paged.patch:7-20; they are stored as float32. The oracle must reproduce
them to float32 rounding; the HIP operator must match them to the fp16-output tolerance
(max-abs <= 2e-3, mean-abs <= 2e-4, beyond half an fp16 ulp of the expected value, which is the
rounding of the output itself) and write exactly the rows the oracle writes.
"""
import os

import numpy as np
import pytest
import torch

import workload as kvc
from mi50_vllm_lab_amd import pth_dec
from oracle import attention as orc

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "decode_cases.npz")
NAMES = ("mtp_gqa6_hnd", "window_noncausal_poison_nhd", "bs1_noncontig_q_outliers", "uniform_padded_slot")


def load(name, device="cpu"):
    z = np.load(FIXTURE)
    layout = bytes(z[f"{name}.layout"]).decode()
    phys = torch.from_numpy(z[f"{name}.kv"].copy()).to(device)
    kv = phys if layout == "HND" else phys.transpose(1, 2)
    cache = kvc.cache_views(kv, layout)
    q = torch.from_numpy(z[f"{name}.q"].copy()).view(torch.float16).to(device)
    scale, window, causal, hq, qmax = z[f"{name}.params"].tolist()
    return dict(cache=cache, q=q, block_table=torch.from_numpy(z[f"{name}.block_table"]).to(device),
                seq_lens=torch.from_numpy(z[f"{name}.seq_lens"]).to(device),
                qsl=torch.from_numpy(z[f"{name}.query_start_loc"]).to(device), scale=float(scale),
                window=int(window), causal=bool(causal), qmax=int(qmax), expected=z[f"{name}.expected"],
                written=z[f"{name}.written"])


@pytest.mark.parametrize("name", NAMES)
def test_oracle_matches_golden(name):
    c = load(name)
    ref, written = orc.paged_decode(c["q"], c["cache"].key_cache, c["cache"].value_cache, c["cache"].k_scale,
                                    c["cache"].v_scale, c["block_table"], c["seq_lens"], c["qsl"],
                                    c["seq_lens"].numel(), c["scale"], c["window"], c["causal"])
    w = c["written"]
    assert (w.all(axis=1) == w.any(axis=1)).all()  # a token is written for all heads or none
    assert np.array_equal(written, w[:, 0])
    exp = c["expected"].astype(np.float64)
    assert np.abs(ref[w] - exp[w]).max() <= 1e-6 * max(1.0, np.abs(exp[w]).max())


@pytest.mark.gpu
@pytest.mark.parametrize("nsplit", [1, 3, 16])
@pytest.mark.parametrize("name", NAMES)
def test_hip_matches_golden(name, nsplit):
    print(f"golden {name} nsplit {nsplit}", flush=True)
    c = load(name, "cuda")
    q = c["q"]
    if name.startswith("bs1_noncontig"):
        parent = torch.zeros((q.shape[0], q.shape[1] + 3, 256), dtype=torch.float16, device="cuda")
        parent[:, 1:1 + q.shape[1]] = q
        q = parent[:, 1:1 + q.shape[1]]
    T, hq = q.shape[0], q.shape[1]
    out = torch.full((T, hq, 256), float("nan"), dtype=torch.float16, device="cuda")
    po, pm, pl = kvc.partial_buffers(max(T, 1), hq, 128, "cuda")
    cache = c["cache"]
    pth_dec.decode(q, cache.key_cache, cache.value_cache, cache.k_scale, cache.v_scale, c["block_table"],
                   c["seq_lens"], c["qsl"], out, c["scale"], po, pm, pl, c["seq_lens"].numel(), c["qmax"], nsplit,
                   c["window"], c["causal"])
    torch.cuda.synchronize()
    o = out.double().cpu().numpy()
    w = c["written"]
    assert np.isfinite(o[w]).all()
    assert np.isnan(o[~w]).all(), "rows the operator must not write were written"
    exp = c["expected"][w].astype(np.float64)
    # the output is fp16: on top of 2e-3 / 2e-4 allow half an fp16 ulp of the expected value
    # (the outlier fixture has outputs up to ~28, where half an ulp is 7.8e-3)
    half_ulp = np.spacing(np.abs(exp).astype(np.float16)).astype(np.float64) / 2
    e = np.abs(o[w] - exp)
    excess = np.maximum(e - half_ulp, 0.0)
    assert excess.max() <= 2e-3 and excess.mean() <= 2e-4, (e.max(), excess.max(), excess.mean())
