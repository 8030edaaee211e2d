"""Python face of libpthdec.so: the `_gfx906_pth_dec` torch-op interface, re-targeted at gfx950.

`decode` and `supported_layout` keep the names, argument order, meaning and error behaviour of
the reference torch extension (kernels/pth_dec/pth_dec.cpp:27-28,49-53,93-95): every check of
the reference's TORCH_CHECKs raises RuntimeError with the same message, the op allocates
nothing and launches on torch's current stream, so it is safe inside HIP-graph capture.
`decode` additionally takes `window` (<= 0: none) and `causal` (the DFlash2 drafter's
non-causal sliding-window rows, patches/vllm/gfx906_fa_paged.patch:7-20).

Tensors cross the C ABI as `pd_tensor` descriptors (data pointer, dtype code, sizes, strides);
no torch type appears in the ABI. The library has no CPU fallback: if it is not built, every
entry point raises.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("PTH_DEC_LIB", os.path.join(_HERE, "lib", "libpthdec.so"))

PD_DTYPE_INT8 = 1
PD_DTYPE_FP16 = 2
PD_DTYPE_FP32 = 3
PD_DTYPE_INT32 = 4
PD_DTYPE_BF16 = 5
PD_DTYPE_INT64 = 6
PD_MAX_DIMS = 4

_DTYPES = {
    torch.int8: PD_DTYPE_INT8,
    torch.float16: PD_DTYPE_FP16,
    torch.float32: PD_DTYPE_FP32,
    torch.int32: PD_DTYPE_INT32,
    torch.bfloat16: PD_DTYPE_BF16,
    torch.int64: PD_DTYPE_INT64,
}

# Every symbol include/pth_dec.h declares.
EXPORTED_SYMBOLS = (
    "pth_dec_launch",
    "pth_dec_launch_window",
    "pth_dec_launch_noalloc",
    "pth_dec_launch_partial",
    "pth_dec_launch_combine",
    "pth_dec_supported_layout",
    "pth_dec_decode",
    "pth_dec_version",
    "pth_fa_forward",
    "pth_fa_forward_exact",
    "pth_fa_forward_split",
    "pth_cache_write",
)


class PdTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("sizes", ctypes.c_int64 * PD_MAX_DIMS),
        ("strides", ctypes.c_int64 * PD_MAX_DIMS),
    ]


_lib = None
_lib_path = None


def load_library(path: str | None = None) -> ctypes.CDLL:
    """Load libpthdec.so and declare the C signatures; raises if it is not built. The library
    loaded last is the one every operator call uses: load_library() returns it (loading LIB_PATH
    the first time), load_library(path) switches to `path`."""
    global _lib, _lib_path
    if _lib is not None and (path is None or os.path.realpath(path) == _lib_path):
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise RuntimeError(f"libpthdec.so not found at {p}; build it with mi50-vllm-lab_amd/build.py")
    lib = ctypes.CDLL(p)
    c_int, c_long, c_float, c_double, vp = ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_double, ctypes.c_void_p
    ip = ctypes.POINTER(ctypes.c_int)
    fp = ctypes.POINTER(ctypes.c_float)
    launch_args = [vp, c_int, vp, c_int, c_int, c_int, ip, c_int, ip, ip, c_int, c_int, c_int, c_int, c_int,
                   c_float, c_int, fp, fp, fp, c_int, c_int, vp, c_long, c_long, vp]
    lib.pth_dec_launch.argtypes = launch_args
    lib.pth_dec_launch.restype = c_int
    lib.pth_dec_launch_window.argtypes = launch_args + [c_int, c_int]
    lib.pth_dec_launch_window.restype = c_int
    lib.pth_dec_launch_noalloc.argtypes = [vp, c_int, vp, c_int, c_int, c_int, ip, c_int, ip, ip, c_int, c_int, c_int,
                                           c_int, c_int, c_float, c_int, c_int, vp, c_long, c_long, vp, c_int, c_int]
    lib.pth_dec_launch_noalloc.restype = c_int
    lib.pth_dec_launch_partial.argtypes = [vp, c_int, vp, c_int, c_int, c_int, ip, c_int, ip, ip, c_int, c_int,
                                           c_int, c_int, c_int, c_float, c_int, fp, fp, fp, c_int, c_int, vp,
                                           c_int, c_int]
    lib.pth_dec_launch_partial.restype = c_int
    lib.pth_dec_launch_combine.argtypes = [ip, ip, c_int, c_int, c_int, c_int, fp, fp, fp, c_int, c_int, vp,
                                           c_long, c_long, vp]
    lib.pth_dec_launch_combine.restype = c_int
    tp = ctypes.POINTER(PdTensor)
    lib.pth_dec_supported_layout.argtypes = [tp, tp, tp, tp]
    lib.pth_dec_supported_layout.restype = c_int
    lib.pth_dec_decode.argtypes = [tp] * 9 + [c_double, tp, tp, tp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                              ctypes.c_int64, ctypes.c_int64, vp, ctypes.c_char_p, c_int]
    lib.pth_dec_decode.restype = c_int
    lib.pth_fa_forward.argtypes = [tp] * 5 + [c_double, tp, tp, vp, ctypes.c_char_p, c_int]
    lib.pth_fa_forward.restype = c_int
    lib.pth_fa_forward_exact.argtypes = lib.pth_fa_forward.argtypes
    lib.pth_fa_forward_exact.restype = c_int
    lib.pth_fa_forward_split.argtypes = [tp] * 5 + [c_double, tp, tp, tp, ctypes.c_int64, ctypes.c_int64, vp,
                                                    ctypes.c_char_p, c_int]
    lib.pth_fa_forward_split.restype = c_int
    lib.pth_cache_write.argtypes = [tp] * 7 + [vp, ctypes.c_char_p, c_int]
    lib.pth_cache_write.restype = c_int
    lib.pth_dec_version.argtypes = []
    lib.pth_dec_version.restype = ctypes.c_char_p
    _lib, _lib_path = lib, os.path.realpath(p)
    return lib


def describe(t: torch.Tensor) -> PdTensor:
    """pd_tensor descriptor of a strided tensor (no copy)."""
    if t.dim() > PD_MAX_DIMS:
        raise RuntimeError(f"tensor rank {t.dim()} exceeds {PD_MAX_DIMS}")
    d = PdTensor()
    d.data = t.data_ptr()
    d.dtype = _DTYPES.get(t.dtype, 0)
    d.ndim = t.dim()
    for i in range(t.dim()):
        d.sizes[i] = t.size(i)
        d.strides[i] = t.stride(i)
    return d


def supported_layout(key_cache: torch.Tensor, value_cache: torch.Tensor, k_scale: torch.Tensor,
                     v_scale: torch.Tensor) -> bool:
    """True if the cache views have vLLM's int8 per-token-head row layout
    [K 256 | k_scale f32 | V 256 | v_scale f32] (kernels/pth_dec/pth_dec.cpp:25-41)."""
    lib = load_library()
    descs = [describe(t) for t in (key_cache, value_cache, k_scale, v_scale)]
    return bool(lib.pth_dec_supported_layout(*[ctypes.byref(x) for x in descs]))


def decode(q: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor, k_scale: torch.Tensor,
           v_scale: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor,
           query_start_loc: torch.Tensor, out: torch.Tensor, scale: float, part_o: torch.Tensor,
           part_m: torch.Tensor, part_l: torch.Tensor, num_seqs: int, qmax: int, nsplit: int,
           window: int = -1, causal: bool = True) -> None:
    """Split-K decode attention over the int8 per-token-head paged KV cache, written into `out`.

    q: fp16 [T, Hq, 256] with head stride 256; out: fp16 [T, Hq, 256] with unit dim stride;
    block_table int32 [>= num_seqs, max_blocks]; seq_lens int32 [>= num_seqs];
    query_start_loc int32 [>= num_seqs + 1]; every sequence has <= qmax query tokens;
    part_o fp32 [>= T, Hq, NSEG, 256], part_m / part_l fp32 [>= T, Hq, NSEG] (caller-owned
    scratch, vLLM's softmax segment buffers); 1 <= nsplit <= NSEG.
    Reference: kernels/pth_dec/pth_dec.cpp:43-91.
    """
    if not q.is_cuda:
        raise RuntimeError("q must be fp16 [T, Hq, 256] with contiguous heads")
    lib = load_library()
    tensors = (q, key_cache, value_cache, k_scale, v_scale, block_table, seq_lens, query_start_loc, out)
    descs = [describe(t) for t in tensors]
    pdescs = [describe(t) for t in (part_o, part_m, part_l)]
    err = ctypes.create_string_buffer(256)
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        rc = lib.pth_dec_decode(*[ctypes.byref(x) for x in descs], float(scale),
                                *[ctypes.byref(x) for x in pdescs], int(num_seqs), int(qmax), int(nsplit),
                                int(window), 1 if causal else 0, ctypes.c_void_p(stream), err, len(err))
    if rc != 0:
        raise RuntimeError(err.value.decode())


PREFILL_ROWS_PER_WORKGROUP = 192  # query rows (tokens x heads of one kv head) per prefill workgroup
PREFILL_CUS = 256                 # workgroups that run at once: one per CU (the LDS takes the CU)
PREFILL_MAX_SPLITS = 64
PREFILL_MIN_TILES_PER_SPLIT = 8   # 256 keys
# makespan model of a prefill launch on MI355X (fit to graph-replayed chunks of 16..6,144 tokens
# over 8k..61k cached tokens): a workgroup costs ~16 us plus ~1.62 us per 32-key tile; a split
# launch adds ~0.6 us per MB of partials (stored, then merged) and ~5 us for the merge launch
PREFILL_US_PER_TILE = 1.62
PREFILL_US_PER_WORKGROUP = 16.0
PREFILL_US_PER_PARTIAL_MB = 0.6
PREFILL_US_MERGE_LAUNCH = 5.0
PREFILL_MAX_WORKSPACE = 1 << 30   # bytes of partials a split launch may take
# A workgroup keeps its block-table slice in LDS when it has at most 6,144 entries (16-key blocks
# when the block size is a multiple of 16, else pages); past that its tile addresses come from
# scalar loads of the global table, ~15 % more per tile (2,048 tokens over 131k keys, 24 q / 4 kv
# heads, bs 16: 7.79 ms unsplit, 1.87 against 1.63 us per tile)
PREFILL_LDS_TABLE = 6144
PREFILL_GLOBAL_TABLE_FACTOR = 1.15


def prefill_cost_us(batch: int, sq: int, heads_q: int, heads_kv: int, max_keys: int, nsplit: int,
                    block_size: int = 16) -> float:
    """Modelled time of one prefill launch with nsplit key splits per query tile: the workgroups
    run in ceil(workgroups / 256) rounds, each as long as the longest split (every row taken to
    see max_keys keys), plus the partials' store and merge when nsplit > 1."""
    g = max(1, heads_q // max(1, heads_kv))
    qtiles = -(-sq // max(1, PREFILL_ROWS_PER_WORKGROUP // g))
    wgs = qtiles * heads_kv * batch * nsplit
    tiles = -(-max(0, max_keys) // 32)
    rounds = -(-wgs // PREFILL_CUS)
    per_split = -(-tiles // nsplit)
    if block_size % 16 == 0:
        in_lds = 2 * per_split <= PREFILL_LDS_TABLE
    else:  # the page table of [0, seq_len), whatever the split
        in_lds = -(-max(0, max_keys) // max(1, block_size)) <= PREFILL_LDS_TABLE
    tile_us = PREFILL_US_PER_TILE * (1.0 if in_lds else PREFILL_GLOBAL_TABLE_FACTOR)
    t = rounds * (per_split * tile_us + PREFILL_US_PER_WORKGROUP)
    if nsplit > 1:
        t += PREFILL_US_MERGE_LAUNCH + PREFILL_US_PER_PARTIAL_MB * batch * sq * heads_q * nsplit * 1032 / 1e6
    return t


def prefill_splits(batch: int, sq: int, heads_q: int, heads_kv: int, max_keys: int, block_size: int = 16) -> int:
    """Key splits per query tile for a prefill launch: the count in 1..64 that minimises
    prefill_cost_us, with at least 8 key tiles (256 keys) of max_keys per split and at most 1 GiB
    of partials. Splitting pays where the query tiles alone leave CUs idle: short chunks (a 64-token
    chunk over 61k keys: 32 splits) and chunks whose workgroups end in a part-filled round (2,560
    tokens, 320 workgroups: 4 splits run them in 5 full rounds of a quarter of the keys instead of
    2 rounds of all of them), and long contexts whose key tiles overflow a workgroup's LDS block
    table (2,048 tokens over 131k keys at bs 16: 2 splits). max_keys is a host-side upper bound on
    the keys a row can see; the device splits each row's actual keys evenly."""
    if batch <= 0 or sq <= 0 or heads_q <= 0 or heads_kv <= 0:
        return 1
    tiles = -(-max(0, max_keys) // 32)
    top = max(1, min(PREFILL_MAX_SPLITS, tiles // PREFILL_MIN_TILES_PER_SPLIT))
    best, best_t = 1, prefill_cost_us(batch, sq, heads_q, heads_kv, max_keys, 1, block_size)
    for ns in range(2, top + 1):
        if batch * sq * heads_q * ns * 1032 > PREFILL_MAX_WORKSPACE:
            break
        t = prefill_cost_us(batch, sq, heads_q, heads_kv, max_keys, ns, block_size)
        if t < best_t:
            best, best_t = ns, t
    return best


def forward_pth(q: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor, block_table: torch.Tensor,
                seq_lens: torch.Tensor, scale: float, q_abs_offset: torch.Tensor,
                out: torch.Tensor | None = None, exact: bool = False, nsplit: int | None = None,
                max_keys: int | None = None) -> torch.Tensor:
    """Causal chunked prefill over the int8 per-token-head cache; returns fp32 [B, Sq, Hq, 256].

    q: fp32 [B, Hq, Sq, 256] contiguous; query token i of sequence b is at absolute position
    q_abs_offset[b] + i and attends to keys k <= that position, k < seq_lens[b].
    Reference: kernels/fa_pth/pth_fa.cpp:41-85 (same arguments; `out` may be passed in).
    exact=True runs pth_fa_forward_exact, which has no counterpart in the reference: K without
    the widening bias and P' as fp16 hi + lo, for caches with very large scales (outlier
    tokens), at about twice the P.V matrix work.
    nsplit: key splits per query tile (pth_fa_forward_split, no counterpart in the reference);
    None picks them with prefill_splits (1 for chunks that fill the GPU), and a workspace for the
    partials is taken from torch's allocator.
    max_keys: a host-side bound on the keys any row of the batch sees (the longest seq_len), used
    only to pick nsplit; None takes the block table's width in keys, which for a table sized to
    the model's maximum length plans every chunk for the longest context.
    """
    if not q.is_cuda:
        raise RuntimeError("q must be contiguous fp32 [B, Hq, Sq, D]")
    lib = load_library()
    if out is None:
        out = torch.empty((q.shape[0], q.shape[2], q.shape[1], q.shape[3]), dtype=torch.float32, device=q.device)
    descs = [describe(t) for t in (q, key_cache, value_cache, block_table, seq_lens)]
    qa, od = describe(q_abs_offset), describe(out)
    err = ctypes.create_string_buffer(256)
    if nsplit is None:
        if max_keys is None:
            max_keys = block_table.shape[1] * key_cache.shape[1] if block_table.dim() == 2 else 0
        nsplit = prefill_splits(q.shape[0], q.shape[2], q.shape[1], key_cache.shape[2], int(max_keys),
                                key_cache.shape[1] if key_cache.dim() == 4 else 16)
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        if nsplit > 1:
            ws = torch.empty((q.shape[0] * q.shape[2] * q.shape[1] * nsplit * (q.shape[3] + 2),), dtype=torch.float32,
                             device=q.device)
            wd = describe(ws)
            rc = lib.pth_fa_forward_split(*[ctypes.byref(x) for x in descs], float(scale), ctypes.byref(qa),
                                          ctypes.byref(od), ctypes.byref(wd), nsplit, 1 if exact else 0,
                                          ctypes.c_void_p(stream), err, len(err))
        else:
            fn = lib.pth_fa_forward_exact if exact else lib.pth_fa_forward
            rc = fn(*[ctypes.byref(x) for x in descs], float(scale), ctypes.byref(qa), ctypes.byref(od),
                    ctypes.c_void_p(stream), err, len(err))
    if rc != 0:
        raise RuntimeError(err.value.decode())
    return out


def cache_write(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                k_scale: torch.Tensor, v_scale: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Quantise key/value [T, Hkv, 256] per (token, kv head) into the int8 rows at slot_mapping.

    scale = absmax / 127, q = clamp(rint(x / scale), -127, 127); negative slots are skipped.
    Replaces vLLM's int8 per-token-head cache update (do_kv_cache_update,
    upstream/pr-dflash2/0002-fix-gfx906-keep-the-drafter-s-sliding-window-in-the-.patch:81-87).
    """
    if not key.is_cuda:
        raise RuntimeError("key and value must be fp16, bf16 or fp32 of the same dtype")
    lib = load_library()
    descs = [describe(t) for t in (key, value, key_cache, value_cache, k_scale, v_scale, slot_mapping)]
    err = ctypes.create_string_buffer(256)
    with torch.cuda.device(key.device):
        stream = torch.cuda.current_stream(key.device).cuda_stream
        rc = lib.pth_cache_write(*[ctypes.byref(x) for x in descs], ctypes.c_void_p(stream), err, len(err))
    if rc != 0:
        raise RuntimeError(err.value.decode())


def _ptr(t: torch.Tensor, ctype):
    return ctypes.cast(ctypes.c_void_p(t.data_ptr()), ctypes.POINTER(ctype))


def launch_partial(q, key_cache, block_table, seq_lens, query_start_loc, part_o, part_m, part_l, *,
                   num_seqs: int, heads_q: int, heads_kv: int, block_size: int, scale: float, qmax: int,
                   nsplit: int, window: int = -1, causal: bool = True, stream=None) -> int:
    """Raw C-ABI call of the split-K partial pass (pth_dec_launch_partial); returns the hipError_t."""
    lib = load_library()
    s = stream if stream is not None else torch.cuda.current_stream(q.device).cuda_stream
    return lib.pth_dec_launch_partial(
        ctypes.c_void_p(q.data_ptr()), q.stride(0), ctypes.c_void_p(key_cache.data_ptr()),
        key_cache.stride(0), key_cache.stride(1), key_cache.stride(2), _ptr(block_table, ctypes.c_int),
        block_table.stride(0), _ptr(seq_lens, ctypes.c_int), _ptr(query_start_loc, ctypes.c_int), num_seqs,
        q.size(0), heads_q, heads_kv, block_size, scale, qmax, _ptr(part_o, ctypes.c_float),
        _ptr(part_m, ctypes.c_float), _ptr(part_l, ctypes.c_float), part_o.size(2), nsplit,
        ctypes.c_void_p(s), window, 1 if causal else 0)


def launch_combine(seq_lens, query_start_loc, part_o, part_m, part_l, out, *, num_seqs: int, qmax: int,
                   nsplit: int, stream=None) -> int:
    """Raw C-ABI call of the log-sum-exp combine pass (pth_dec_launch_combine)."""
    lib = load_library()
    s = stream if stream is not None else torch.cuda.current_stream(out.device).cuda_stream
    return lib.pth_dec_launch_combine(
        _ptr(seq_lens, ctypes.c_int), _ptr(query_start_loc, ctypes.c_int), num_seqs, out.size(0), out.size(1),
        qmax, _ptr(part_o, ctypes.c_float), _ptr(part_m, ctypes.c_float), _ptr(part_l, ctypes.c_float),
        part_o.size(2), nsplit, ctypes.c_void_p(out.data_ptr()), out.stride(0), out.stride(1), ctypes.c_void_p(s))


def version() -> str:
    return load_library().pth_dec_version().decode()


def partial_kernel_name(rows_per_kv_head: int, block_size: int) -> str:
    """Name of the split-K partial kernel a decode launch with this many query rows per kv head
    (qmax * Hq / Hkv) and this block size runs (as rocprofv3 reports it, template arguments
    included)."""
    nrb = (rows_per_kv_head + 15) // 16
    fast = block_size % 16 == 0
    return f"pd_partial_kernel<{nrb}, {'true' if fast else 'false'}>"
