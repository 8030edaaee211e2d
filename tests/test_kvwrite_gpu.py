"""GPU parity of the KV-cache writer (pth_cache_write) against the CPU oracle: bit-exact cache
bytes for fp16, bf16 and fp32 inputs (including values on exact rounding ties, all-zero rows and
rows that clamp, rows whose scale is subnormal), HND and NHD, block sizes 16, 1584 and 1, padding
slots untouched, through each of its three kernel forms (one row per wave below 4,096 rows, four
rows per wave from there, and from 16,384 rows four rows per wave quantising through the row's
inverse scale); and decode over a GPU-written cache equals decode over the oracle-written one bit
for bit.
"""
import sys

import numpy as np
import pytest
import torch

import workload as kvc
from mi50_vllm_lab_amd import pth_dec
from oracle import kvwrite as kvw

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_inputs(T, hkv, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((T, hkv, 256), generator=g) * torch.rand((T, hkv, 1), generator=g) * 40
    v = torch.randn((T, hkv, 256), generator=g)
    # ties: a row whose absmax is 127 * 2^-3 has scale 2^-3, so multiples of 2^-4 are exact ties
    k[0, 0] = torch.randint(-254, 255, (256,), generator=g).float() * 0.0625
    k[0, 0, 0] = 127 * 0.125
    v[1 % T, 0] = 0.0                       # all-zero row
    # near-ties (float32 inputs): within 4 ulps of (m + 0.5) * scale for every m, where only a
    # correctly rounded x / scale gives the oracle's byte
    if T > 2:
        sc = np.float32(np.float32(38.1) / np.float32(127))
        near = ((np.arange(-126, 126, dtype=np.float32) + np.float32(0.5)) * sc).astype(np.float32)
        bits = near.view(np.int32) + np.where(near < 0, -1, 1) * np.resize(np.array([-4, -1, 1, 3]), near.size)
        row = np.zeros(256, np.float32)
        row[:near.size] = bits.astype(np.int32).view(np.float32)
        row[255] = 38.1
        k[2, 1] = torch.from_numpy(row)
    # subnormal scales (float32 and bfloat16 inputs; in float16 these rows underflow to zero): absmax
    # 1e-37 gives a scale whose inverse overflows to infinity, 127 x 3e-39 one whose inverse is
    # finite, and a row of subnormal inputs a scale of a few subnormal ulps
    if T > 4:
        k[3, 2 % hkv] = torch.randn(256, generator=g) * 1e-37
        k[3, 2 % hkv, 7] = 1e-37
        v[3, 2 % hkv] = torch.rand(256, generator=g) * (127 * 3e-39)
        v[3, 2 % hkv, 9] = -127 * 3e-39
        k[4, 3 % hkv] = torch.randn(256, generator=g) * 1e-40
    return k.to(dtype), v.to(dtype)


def write_and_compare(T, hkv, dtype, bs, layout, seed):
    nblk = (T + bs - 1) // bs + 3
    k, v = make_inputs(T, hkv, dtype, seed=seed)
    g = torch.Generator().manual_seed(9)
    slots = torch.randperm(nblk * bs, generator=g)[:T].to(torch.int64)
    slots[::17] = -1                          # padding tokens
    ref = kvc.allocate_cache(nblk, bs, hkv, layout)
    ref.kv.copy_(torch.randint(-128, 128, ref.kv.shape, dtype=torch.int8, generator=g))
    dev = kvc.clone_cache(ref, "cuda")
    kvw.write_rows(k.float(), v.float(), ref.key_cache, ref.value_cache, ref.k_scale, ref.v_scale, slots)
    say(f"cache write T={T} hkv={hkv} dtype={dtype} bs={bs} layout={layout}")
    pth_dec.cache_write(k.cuda(), v.cuda(), dev.key_cache, dev.value_cache, dev.k_scale, dev.v_scale, slots.cuda())
    torch.cuda.synchronize()
    assert torch.equal(dev.kv.cpu(), ref.kv)


# 300 x 4 rows take the kernel with one row per wave, 1,100 x 4 the one with four rows per wave
# (calls of at least 4,096 rows), 4,100 x 4 the one through the inverse scale (at least 16,384)
@pytest.mark.parametrize("T", [300, 1100, 4100])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bs,layout", [(16, "HND"), (16, "NHD"), (1584, "HND"), (1, "NHD")])
def test_bit_exact_against_oracle(T, dtype, bs, layout):
    write_and_compare(T, 4, dtype, bs, layout, seed=bs + T)


@pytest.mark.parametrize("T,hkv", [(819, 5), (1024, 4)])
def test_rows_per_wave_switch(T, hkv):
    """819 x 5 = 4,095 rows take one row per wave, 1,024 x 4 = 4,096 four rows per wave."""
    write_and_compare(T, hkv, torch.float16, 16, "NHD", seed=T)


def test_decode_over_gpu_written_cache_is_bit_identical():
    T, hkv, bs = 2000, 4, 16
    k, v = make_inputs(T, hkv, torch.float16, seed=77)
    nblk = T // bs + 2
    slots = torch.arange(T, dtype=torch.int64)
    ref = kvc.allocate_cache(nblk, bs, hkv, "HND")
    kvw.write_rows(k.float(), v.float(), ref.key_cache, ref.value_cache, ref.k_scale, ref.v_scale, slots)
    dev = kvc.allocate_cache(nblk, bs, hkv, "HND", device="cuda")
    pth_dec.cache_write(k.cuda(), v.cuda(), dev.key_cache, dev.value_cache, dev.k_scale, dev.v_scale, slots.cuda())
    refd = kvc.clone_cache(ref, "cuda")
    q = torch.randn((4, 24, 256), generator=torch.Generator().manual_seed(3)).half().cuda()
    bt = torch.arange(nblk, dtype=torch.int32).view(1, -1).cuda()
    sl = torch.tensor([T], dtype=torch.int32).cuda()
    qsl = torch.tensor([0, 4], dtype=torch.int32).cuda()
    outs = []
    for c in (dev, refd):
        out = torch.empty((4, 24, 256), dtype=torch.float16, device="cuda")
        po, pm, pl = kvc.partial_buffers(4, 24, 64, "cuda")
        pth_dec.decode(q, c.key_cache, c.value_cache, c.k_scale, c.v_scale, bt, sl, qsl, out, 1 / 16, po, pm, pl,
                       1, 4, 16)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
