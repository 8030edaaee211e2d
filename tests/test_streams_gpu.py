"""Concurrent calls on separate streams: the entry points keep no state outside the caller's
buffers, so two decode workloads (24 rows over 20,000 keys, and 48 windowed non-causal rows:
different kernel variants) and a prefill chunk launched together on three streams, several
times over without host waits, must give outputs bit-identical to the same calls run one after
the other. vLLM may overlap attention work across streams; a hidden global (a counter, a static
buffer) would make these runs differ. The streams have the default priority.
"""
import sys

import pytest
import torch

import workload as kvc
from mi50_vllm_lab_amd import pth_dec

pytestmark = pytest.mark.gpu

NSEG = 64


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_three_streams_bit_identical_to_sequential():
    a = kvc.make_case([20000], [4], num_q_heads=24, num_kv_heads=4, block_size=16, seed=71).to("cuda")
    b = kvc.make_case([3000, 900, 12000], [8, 8, 8], num_q_heads=24, num_kv_heads=4, block_size=16, seed=72,
                      window=1024, causal=False, poison=True).to("cuda")
    c = kvc.make_case([5000], [200], num_q_heads=24, num_kv_heads=4, block_size=16, seed=73).to("cuda")
    qc = kvc.prefill_query(c)
    qabs = torch.tensor([5000], dtype=torch.int32, device="cuda")

    def buffers(d):
        out = torch.full((d.num_tokens, 24, 256), float("nan"), dtype=torch.float16, device="cuda")
        return (out,) + kvc.partial_buffers(d.num_tokens, 24, NSEG, "cuda")

    def run_decode(d, bufs, qmax, nsplit):
        out, po, pm, pl = bufs
        pth_dec.decode(d.q, d.cache.key_cache, d.cache.value_cache, d.cache.k_scale, d.cache.v_scale, d.block_table,
                       d.seq_lens, d.query_start_loc, out, d.scale, po, pm, pl, d.num_seqs, qmax, nsplit, d.window,
                       d.causal)

    def run_prefill(out):
        pth_dec.forward_pth(qc, c.cache.key_cache, c.cache.value_cache, c.block_table, c.seq_lens, c.scale, qabs,
                            out=out)

    # one after the other on the current stream
    ra, rb = buffers(a), buffers(b)
    rc = torch.full((1, 200, 24, 256), float("nan"), dtype=torch.float32, device="cuda")
    run_decode(a, ra, 4, 64)
    run_decode(b, rb, 8, 16)
    run_prefill(rc)
    torch.cuda.synchronize()

    streams = [torch.cuda.Stream() for _ in range(3)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for rep in range(4):
        say(f"three streams, round {rep}")
        xa, xb = buffers(a), buffers(b)
        xc = torch.full_like(rc, float("nan"))
        torch.cuda.synchronize()
        for s in streams:
            s.wait_stream(torch.cuda.current_stream())
        for _ in range(3):  # several launches each, interleaved across the streams
            with torch.cuda.stream(streams[0]):
                run_decode(a, xa, 4, 64)
            with torch.cuda.stream(streams[1]):
                run_decode(b, xb, 8, 16)
            with torch.cuda.stream(streams[2]):
                run_prefill(xc)
        torch.cuda.synchronize()
        assert torch.equal(xa[0].view(torch.int16), ra[0].view(torch.int16))
        assert torch.equal(xb[0].view(torch.int16), rb[0].view(torch.int16))
        assert torch.equal(xc.view(torch.int32), rc.view(torch.int32))
