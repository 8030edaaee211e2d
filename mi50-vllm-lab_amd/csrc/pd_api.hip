// The C ABI of libpthdec.so (include/pth_dec.h): the reference's argument checks and error
// messages (kernels/pth_dec/pth_dec.cpp:16-91, kernels/fa_pth/pth_fa.cpp:41-85), the validation of
// the tensor descriptors, and the calls into the kernel files. The library is built with hidden
// visibility; only the entry points declared in pth_dec.h are exported.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#pragma GCC visibility push(default)
#include "pth_dec.h"
#pragma GCC visibility pop

#include "pd_kernels.hpp"

namespace pd {
namespace {

LaunchArgs make_args(const void* q, int64_t q_st, const void* kc, int64_t k_sb, int64_t k_ss, int64_t k_sh,
                     const int* block_table, int64_t bt_stride, const int* seq_lens, const int* qsl, int num_seqs,
                     int num_tokens, int heads_q, int heads_kv, int block_size, float scale, int qmax,
                     float* part_o, float* part_m, float* part_l, int nseg, int nsplit, void* out, int64_t o_st,
                     int64_t o_sh, int window, int causal) {
    LaunchArgs x;
    x.q = q;
    x.q_st = q_st;
    x.kc = kc;
    x.k_sb = k_sb;
    x.k_ss = k_ss;
    x.k_sh = k_sh;
    x.block_table = block_table;
    x.bt_stride = bt_stride;
    x.seq_lens = seq_lens;
    x.qsl = qsl;
    x.num_seqs = num_seqs;
    x.num_tokens = num_tokens;
    x.heads_q = heads_q;
    x.heads_kv = heads_kv;
    x.block_size = block_size;
    x.scale = scale;
    x.qmax = qmax;
    x.part_o = part_o;
    x.part_m = part_m;
    x.part_l = part_l;
    x.nseg = nseg;
    x.nsplit = nsplit;
    x.out = out;
    x.o_st = o_st;
    x.o_sh = o_sh;
    x.window = window;
    x.causal = causal;
    return x;
}

// ---- descriptor checks (pth_dec.cpp:16-80) ----

bool is_dtype(const pd_tensor* t, int dt) { return t && t->dtype == dt; }

bool same_rows(const pd_tensor* scale, const pd_tensor* cache, int64_t byte_off) {
    // f32 scale view [blocks, block_size, Hkv] sitting byte_off bytes into each cache row
    const uintptr_t base = reinterpret_cast<uintptr_t>(cache->data);
    return scale->ndim == 3 && scale->dtype == PD_DTYPE_FP32 &&
           reinterpret_cast<uintptr_t>(scale->data) == base + (uintptr_t)byte_off &&
           scale->strides[0] * 4 == cache->strides[0] && scale->strides[1] * 4 == cache->strides[1] &&
           scale->strides[2] * 4 == cache->strides[2];
}

bool layout_ok(const pd_tensor* kc, const pd_tensor* vc, const pd_tensor* ks, const pd_tensor* vs) {
    if (!kc || !vc || !ks || !vs) return false;
    if (kc->dtype != PD_DTYPE_INT8 || vc->dtype != PD_DTYPE_INT8 || kc->ndim != 4 || vc->ndim != 4 ||
        kc->sizes[3] != 260 || vc->sizes[3] != 260 || kc->strides[3] != 1 || vc->strides[3] != 1)
        return false;
    for (int i = 0; i < 3; ++i)
        if (kc->strides[i] != vc->strides[i] || kc->sizes[i] != vc->sizes[i]) return false;
    const uintptr_t kb = reinterpret_cast<uintptr_t>(kc->data);
    if (reinterpret_cast<uintptr_t>(vc->data) != kb + 260) return false;
    if (kb % 8 || kc->strides[0] % 8 || kc->strides[1] % 8 || kc->strides[2] % 8) return false;
    if (kc->strides[0] > INT32_MAX || kc->strides[1] > INT32_MAX || kc->strides[2] > INT32_MAX) return false;
    return same_rows(ks, kc, 256) && same_rows(vs, kc, 516);
}

bool is_contig(const pd_tensor* t) {
    for (int i = 0; i < t->ndim; ++i)
        if (t->sizes[i] == 0) return true;  // an empty tensor is contiguous whatever its strides
    int64_t expect = 1;
    for (int i = t->ndim - 1; i >= 0; --i) {
        if (t->sizes[i] != 1 && t->strides[i] != expect) return false;
        expect *= t->sizes[i];
    }
    return true;
}

int fail(char* err, int errlen, const char* msg) {
    if (err && errlen > 0) {
        strncpy(err, msg, (size_t)errlen - 1);
        err[errlen - 1] = '\0';
    }
    return 1;
}

}  // namespace
}  // namespace pd

using namespace pd;

#pragma GCC visibility push(default)

extern "C" {

hipError_t pth_dec_launch(const void* q, int q_st, const void* kc, int k_sb, int k_ss, int k_sh,
                          const int* block_table, int bt_stride, const int* seq_lens, const int* qsl,
                          int num_seqs, int num_tokens, int heads_q, int heads_kv, int block_size,
                          float scale, int qmax, float* part_o, float* part_m, float* part_l, int nseg,
                          int nsplit, void* out, long o_st, long o_sh, hipStream_t stream) {
    const LaunchArgs x = make_args(q, q_st, kc, k_sb, k_ss, k_sh, block_table, bt_stride, seq_lens, qsl, num_seqs,
                                   num_tokens, heads_q, heads_kv, block_size, scale, qmax, part_o, part_m, part_l,
                                   nseg, nsplit, out, o_st, o_sh, -1, 1);
    return launch_all(x, stream, true);
}

hipError_t pth_dec_launch_window(const void* q, int q_st, const void* kc, int k_sb, int k_ss, int k_sh,
                                 const int* block_table, int bt_stride, const int* seq_lens,
                                 const int* qsl, int num_seqs, int num_tokens, int heads_q, int heads_kv,
                                 int block_size, float scale, int qmax, float* part_o, float* part_m,
                                 float* part_l, int nseg, int nsplit, void* out, long o_st, long o_sh,
                                 hipStream_t stream, int window, int causal) {
    const LaunchArgs x = make_args(q, q_st, kc, k_sb, k_ss, k_sh, block_table, bt_stride, seq_lens, qsl, num_seqs,
                                   num_tokens, heads_q, heads_kv, block_size, scale, qmax, part_o, part_m, part_l,
                                   nseg, nsplit, out, o_st, o_sh, window, causal);
    return launch_all(x, stream, false);
}

hipError_t pth_dec_launch_noalloc(const void* q, int q_st, const void* kc, int k_sb, int k_ss, int k_sh,
                                  const int* block_table, int bt_stride, const int* seq_lens,
                                  const int* qsl, int num_seqs, int num_tokens, int heads_q,
                                  int heads_kv, int block_size, float scale, int qmax, int nsplit,
                                  void* out, long o_st, long o_sh, hipStream_t stream, int window,
                                  int causal) {
    LaunchArgs x = make_args(q, q_st, kc, k_sb, k_ss, k_sh, block_table, bt_stride, seq_lens, qsl, num_seqs,
                             num_tokens, heads_q, heads_kv, block_size, scale, qmax, nullptr, nullptr, nullptr,
                             nsplit, nsplit, out, o_st, o_sh, window, causal);
    hipError_t e = check_args(x, false);
    if (e != hipSuccess) return e;
    if (num_tokens == 0) return hipSuccess;
    // partial rows the array holds; the product is bounded in two steps so that it cannot wrap
    const uint64_t max_rows = kScratchBytes / ((kDim + 2) * sizeof(float));
    const uint64_t th = (uint64_t)num_tokens * (uint64_t)heads_q;  // both below 2^31
    if (th > max_rows || th * (uint64_t)nsplit > max_rows) return hipErrorOutOfMemory;
    const size_t rows = (size_t)(th * (uint64_t)nsplit);
    void* base = nullptr;
    e = scratch_address(&base);
    if (e != hipSuccess) return e;
    x.part_o = static_cast<float*>(base);
    x.part_m = x.part_o + rows * kDim;
    x.part_l = x.part_m + rows;
    e = launch_partial(x, stream);
    if (e != hipSuccess) return e;
    return launch_combine(x, stream);
}

hipError_t pth_dec_launch_partial(const void* q, int q_st, const void* kc, int k_sb, int k_ss, int k_sh,
                                  const int* block_table, int bt_stride, const int* seq_lens,
                                  const int* qsl, int num_seqs, int num_tokens, int heads_q,
                                  int heads_kv, int block_size, float scale, int qmax, float* part_o,
                                  float* part_m, float* part_l, int nseg, int nsplit,
                                  hipStream_t stream, int window, int causal) {
    const LaunchArgs x = make_args(q, q_st, kc, k_sb, k_ss, k_sh, block_table, bt_stride, seq_lens, qsl, num_seqs,
                                   num_tokens, heads_q, heads_kv, block_size, scale, qmax, part_o, part_m, part_l,
                                   nseg, nsplit, nullptr, 0, 0, window, causal);
    hipError_t e = check_args(x, false);
    if (e != hipSuccess) return e;
    if (num_tokens == 0) return hipSuccess;
    return launch_partial(x, stream);
}

hipError_t pth_dec_launch_combine(const int* seq_lens, const int* qsl, int num_seqs, int num_tokens,
                                  int heads_q, int qmax, const float* part_o, const float* part_m,
                                  const float* part_l, int nseg, int nsplit, void* out, long o_st,
                                  long o_sh, hipStream_t stream) {
    if (num_seqs < 1 || heads_q < 1 || qmax < 1 || nsplit < 1 || nsplit > nseg || num_tokens < 0)
        return hipErrorInvalidValue;
    if (num_tokens == 0) return hipSuccess;
    const LaunchArgs x = make_args(nullptr, 0, nullptr, 0, 0, 0, nullptr, 0, seq_lens, qsl, num_seqs, num_tokens,
                                   heads_q, 1, 1, 1.f, qmax, const_cast<float*>(part_o), const_cast<float*>(part_m),
                                   const_cast<float*>(part_l), nseg, nsplit, out, o_st, o_sh, -1, 1);
    return launch_combine(x, stream);
}

int pth_dec_supported_layout(const pd_tensor* key_cache, const pd_tensor* value_cache, const pd_tensor* k_scale,
                             const pd_tensor* v_scale) {
    return layout_ok(key_cache, value_cache, k_scale, v_scale) ? 1 : 0;
}

int pth_dec_decode(const pd_tensor* q, const pd_tensor* key_cache, const pd_tensor* value_cache,
                   const pd_tensor* k_scale, const pd_tensor* v_scale, const pd_tensor* block_table,
                   const pd_tensor* seq_lens, const pd_tensor* query_start_loc, const pd_tensor* out, double scale,
                   const pd_tensor* part_o, const pd_tensor* part_m, const pd_tensor* part_l, int64_t num_seqs,
                   int64_t qmax, int64_t nsplit, int64_t window, int64_t causal, hipStream_t stream, char* err,
                   int errlen) {
    if (!q || !key_cache || !value_cache || !k_scale || !v_scale || !block_table || !seq_lens ||
        !query_start_loc || !out || !part_o || !part_m || !part_l)
        return fail(err, errlen, "null tensor descriptor");
    if (!(q->dtype == PD_DTYPE_FP16 && q->ndim == 3 && q->sizes[2] == 256 && q->strides[2] == 1 &&
          q->strides[1] == 256 && q->strides[0] % 2 == 0 && q->strides[0] <= INT32_MAX &&
          (reinterpret_cast<uintptr_t>(q->data) % 4) == 0))
        return fail(err, errlen, "q must be fp16 [T, Hq, 256] with contiguous heads");
    if (!(out->dtype == PD_DTYPE_FP16 && out->ndim == 3 && out->sizes[0] == q->sizes[0] &&
          out->sizes[1] == q->sizes[1] && out->sizes[2] == 256 && out->strides[2] == 1))
        return fail(err, errlen, "out must be fp16 [T, Hq, 256] with unit dim stride");
    if (!(q->sizes[0] <= INT32_MAX && q->sizes[1] <= INT32_MAX && num_seqs <= INT32_MAX && qmax <= INT32_MAX &&
          nsplit <= INT32_MAX && window >= INT32_MIN && window <= INT32_MAX))
        return fail(err, errlen, "sizes, num_seqs, qmax, nsplit and window must fit in 32 bits");
    if (!layout_ok(key_cache, value_cache, k_scale, v_scale))
        return fail(err, errlen, "KV cache views do not have the int8 per-token-head row layout");
    if (!(block_table->dtype == PD_DTYPE_INT32 && seq_lens->dtype == PD_DTYPE_INT32 &&
          query_start_loc->dtype == PD_DTYPE_INT32 && block_table->ndim == 2 && block_table->strides[1] == 1 &&
          block_table->strides[0] <= INT32_MAX && is_contig(seq_lens) && is_contig(query_start_loc)))
        return fail(err, errlen, "block_table / seq_lens / query_start_loc must be int32");
    if (!(part_o->dtype == PD_DTYPE_FP32 && is_contig(part_o) && part_o->ndim == 4 && part_o->sizes[3] == 256 &&
          part_m->dtype == PD_DTYPE_FP32 && part_l->dtype == PD_DTYPE_FP32 && is_contig(part_m) &&
          is_contig(part_l) && part_m->ndim == 3 && part_l->ndim == 3))
        return fail(err, errlen, "partial buffers must be contiguous fp32");
    const int64_t T = q->sizes[0], Hq = q->sizes[1], Hkv = key_cache->sizes[2];
    const int64_t nseg = part_o->sizes[2];
    if (!(part_o->sizes[0] >= T && part_o->sizes[1] == Hq && part_m->sizes[0] >= T && part_m->sizes[1] == Hq &&
          part_m->sizes[2] == nseg && part_l->sizes[0] >= T && part_l->sizes[1] == Hq && part_l->sizes[2] == nseg &&
          nseg <= INT32_MAX))
        return fail(err, errlen, "partial buffers too small");
    if (!(Hkv > 0 && Hq % Hkv == 0)) return fail(err, errlen, "heads_q must be a multiple of heads_kv");
    if (!(qmax >= 1 && qmax * (Hq / Hkv) <= 16 * kMaxRowBlocks))
        return fail(err, errlen, "qmax * (Hq / Hkv) must be in [1, 48]");
    if (!(nsplit >= 1 && nsplit <= nseg)) return fail(err, errlen, "nsplit must be in [1, NSEG]");
    if (!(num_seqs >= 1 && seq_lens->sizes[0] >= num_seqs && query_start_loc->sizes[0] >= num_seqs + 1 &&
          block_table->sizes[0] >= num_seqs))
        return fail(err, errlen, "per-sequence tensors too small");
    if (T == 0) return 0;
    const LaunchArgs x = make_args(
        q->data, q->strides[0], key_cache->data, key_cache->strides[0], key_cache->strides[1],
        key_cache->strides[2], static_cast<const int*>(block_table->data), block_table->strides[0],
        static_cast<const int*>(seq_lens->data), static_cast<const int*>(query_start_loc->data), (int)num_seqs,
        (int)T, (int)Hq, (int)Hkv, (int)key_cache->sizes[1], (float)scale, (int)qmax,
        static_cast<float*>(const_cast<void*>(part_o->data)), static_cast<float*>(const_cast<void*>(part_m->data)),
        static_cast<float*>(const_cast<void*>(part_l->data)), (int)nseg, (int)nsplit, const_cast<void*>(out->data),
        out->strides[0], out->strides[1], (int)window, (int)causal);
    const hipError_t e = launch_all(x, stream, false);
    if (e != hipSuccess) {
        char msg[256];
        snprintf(msg, sizeof msg, "pth_dec launch failed: %s", hipGetErrorString(e));
        fail(err, errlen, msg);
        return 2;
    }
    return 0;
}

static int fa_forward(const pd_tensor* q, const pd_tensor* key_cache, const pd_tensor* value_cache,
                      const pd_tensor* block_table, const pd_tensor* seq_lens, double scale,
                      const pd_tensor* q_abs_offset, const pd_tensor* out, hipStream_t stream, char* err, int errlen,
                      bool exact, int64_t nsplit = 1, const pd_tensor* workspace = nullptr) {
    if (!q || !key_cache || !value_cache || !block_table || !seq_lens || !q_abs_offset || !out)
        return fail(err, errlen, "null tensor descriptor");
    if (!(q->dtype == PD_DTYPE_FP32 && q->ndim == 4 && is_contig(q)))
        return fail(err, errlen, "q must be contiguous fp32 [B, Hq, Sq, D]");
    if (!(key_cache->dtype == PD_DTYPE_INT8 && value_cache->dtype == PD_DTYPE_INT8))
        return fail(err, errlen, "key/value cache views must be int8");
    if (!(key_cache->ndim == 4 && value_cache->ndim == 4)) return fail(err, errlen, "cache views must be 4D");
    if (!(key_cache->strides[3] == 1 && value_cache->strides[3] == 1))
        return fail(err, errlen, "cache rows must be contiguous");
    if (!(block_table->dtype == PD_DTYPE_INT32 && seq_lens->dtype == PD_DTYPE_INT32 &&
          q_abs_offset->dtype == PD_DTYPE_INT32))
        return fail(err, errlen, "block_table/seq_lens/q_abs_offset must be int32");
    const int64_t B = q->sizes[0], Hq = q->sizes[1], Sq = q->sizes[2], D = q->sizes[3];
    const int64_t bs = key_cache->sizes[1], Hkv = key_cache->sizes[2];
    if (!(B <= INT32_MAX && Hq <= INT32_MAX && Sq <= INT32_MAX))
        return fail(err, errlen, "B, Hq and Sq must be below 2^31");
    if (D != 256) return fail(err, errlen, "head_dim must be 256 (only instantiation built)");
    if (!(key_cache->sizes[3] >= D + 4 && value_cache->sizes[3] >= D + 4))
        return fail(err, errlen, "cache rows must hold D int8 values and a fp32 scale");
    if (!(Hkv > 0 && Hq % Hkv == 0)) return fail(err, errlen, "heads_q must be a multiple of heads_kv");
    if (!(block_table->ndim == 2 && block_table->sizes[0] == B && block_table->strides[1] == 1 &&
          seq_lens->sizes[0] == B && q_abs_offset->sizes[0] == B && is_contig(seq_lens) && is_contig(q_abs_offset)))
        return fail(err, errlen, "per-sequence tensors must have B rows");
    const uintptr_t kb = reinterpret_cast<uintptr_t>(key_cache->data);
    if (!(kb % 8 == 0 && (reinterpret_cast<uintptr_t>(value_cache->data) % 4) == 0 && key_cache->strides[1] % 8 == 0 &&
          key_cache->strides[2] % 8 == 0 && key_cache->strides[0] % 8 == 0))
        return fail(err, errlen, "K rows must be 8-byte aligned and V rows 4-byte aligned");
    // the kernel reads K and V from one 520-byte row: V must be the same rows, 260 bytes in
    bool same = reinterpret_cast<uintptr_t>(value_cache->data) == kb + 260;
    for (int i = 0; i < 3; ++i)
        same = same && value_cache->strides[i] == key_cache->strides[i] && value_cache->sizes[i] == key_cache->sizes[i];
    if (!same) return fail(err, errlen, "value_cache must view the same cache rows as key_cache, 260 bytes in");
    if (!(key_cache->strides[0] <= INT32_MAX && key_cache->strides[1] <= INT32_MAX && key_cache->strides[2] <= INT32_MAX))
        return fail(err, errlen, "cache strides must be below 2^31");
    const int64_t G = Hq / Hkv;
    if (G > kFaRows) return fail(err, errlen, "heads_q / heads_kv must be at most 192");
    if (!(out->dtype == PD_DTYPE_FP32 && out->ndim == 4 && out->sizes[0] == B && out->sizes[1] == Sq &&
          out->sizes[2] == Hq && out->sizes[3] == D && out->strides[3] == 1))
        return fail(err, errlen, "out must be fp32 [B, Sq, Hq, D] with unit dim stride");
    // q rows are read and out rows written as 16-byte vectors
    if (!((reinterpret_cast<uintptr_t>(q->data) % 16) == 0 && (reinterpret_cast<uintptr_t>(out->data) % 16) == 0 &&
          out->strides[0] % 4 == 0 && out->strides[1] % 4 == 0 && out->strides[2] % 4 == 0))
        return fail(err, errlen, "q and out rows must be 16-byte aligned");
    if (!(nsplit >= 1 && nsplit <= 64)) return fail(err, errlen, "nsplit must be in [1, 64]");
    // the merge numbers rows (b, token, head) in 32 bits; B, Sq < 2^31 keep B * Sq within int64
    if (nsplit > 1 && Hq > 0 && B * Sq > INT32_MAX / Hq)
        return fail(err, errlen, "a split prefill takes at most 2^31 - 1 (token, head) rows");
    if (nsplit > 1) {
        if (!(workspace && workspace->dtype == PD_DTYPE_FP32 && workspace->ndim == 1 && is_contig(workspace) &&
              workspace->sizes[0] >= prefill_workspace_floats(B, Sq, Hq, nsplit) &&
              (reinterpret_cast<uintptr_t>(workspace->data) % 16) == 0))
            return fail(err, errlen, "workspace must be contiguous 16-byte aligned fp32 of B * Sq * Hq * nsplit * 258");
    }
    if (B == 0 || Sq == 0) return 0;
    FaParams p;
    p.q = static_cast<const float*>(q->data);
    p.q_sb = q->strides[0];
    p.q_sh = q->strides[1];
    p.q_st = q->strides[2];
    p.kc = static_cast<const int8_t*>(key_cache->data);
    p.k_sb = key_cache->strides[0];
    p.k_ss = key_cache->strides[1];
    p.k_sh = key_cache->strides[2];
    p.block_table = static_cast<const int*>(block_table->data);
    p.bt_stride = block_table->strides[0];
    p.seq_lens = static_cast<const int*>(seq_lens->data);
    p.q_abs = static_cast<const int*>(q_abs_offset->data);
    p.out = static_cast<float*>(const_cast<void*>(out->data));
    p.o_sb = out->strides[0];
    p.o_st = out->strides[1];
    p.o_sh = out->strides[2];
    p.Sq = (int)Sq;
    p.Hq = (int)Hq;
    p.G = (int)G;
    p.tok_per_wg = (int)(kFaRows / G);
    p.block_size = (int)bs;
    p.bs_shift = (bs & (bs - 1)) == 0 ? __builtin_ctz((unsigned)bs) : -1;
    p.scale_log2 = (float)scale * 1.4426950408889634f;
    // 16-key block offsets fit the LDS table's 32 bits (in 8-byte units) when the cache spans
    // less than 2^35 bytes
    const int64_t span = (key_cache->sizes[0] - 1) * key_cache->strides[0] + (bs - 1) * key_cache->strides[1] +
                         (Hkv - 1) * key_cache->strides[2] + 8;
    p.bt32 = span < ((int64_t)1 << 35);
    p.nsplit = (int)nsplit;
    p.part_o = nullptr;
    p.part_m = nullptr;
    p.part_l = nullptr;
    if (nsplit > 1) {
        float* ws = static_cast<float*>(const_cast<void*>(workspace->data));
        const int64_t prow = B * Sq * Hq * nsplit;
        p.part_o = ws;
        p.part_m = ws + prow * kDim;
        p.part_l = p.part_m + prow;
    }
    const hipError_t e = launch_prefill(p, (int)B, (int)Hkv, stream, exact);
    if (e != hipSuccess) {
        char msg[256];
        snprintf(msg, sizeof msg, "pth_fa launch failed: %s", hipGetErrorString(e));
        fail(err, errlen, msg);
        return 2;
    }
    return 0;
}

int pth_fa_forward(const pd_tensor* q, const pd_tensor* key_cache, const pd_tensor* value_cache,
                   const pd_tensor* block_table, const pd_tensor* seq_lens, double scale, const pd_tensor* q_abs_offset,
                   const pd_tensor* out, hipStream_t stream, char* err, int errlen) {
    return fa_forward(q, key_cache, value_cache, block_table, seq_lens, scale, q_abs_offset, out, stream, err, errlen,
                      false);
}

int pth_fa_forward_exact(const pd_tensor* q, const pd_tensor* key_cache, const pd_tensor* value_cache,
                         const pd_tensor* block_table, const pd_tensor* seq_lens, double scale,
                         const pd_tensor* q_abs_offset, const pd_tensor* out, hipStream_t stream, char* err,
                         int errlen) {
    return fa_forward(q, key_cache, value_cache, block_table, seq_lens, scale, q_abs_offset, out, stream, err, errlen,
                      true);
}

int pth_fa_forward_split(const pd_tensor* q, const pd_tensor* key_cache, const pd_tensor* value_cache,
                         const pd_tensor* block_table, const pd_tensor* seq_lens, double scale,
                         const pd_tensor* q_abs_offset, const pd_tensor* out, const pd_tensor* workspace,
                         int64_t nsplit, int64_t exact, hipStream_t stream, char* err, int errlen) {
    return fa_forward(q, key_cache, value_cache, block_table, seq_lens, scale, q_abs_offset, out, stream, err, errlen,
                      exact != 0, nsplit, workspace);
}

int pth_cache_write(const pd_tensor* key, const pd_tensor* value, const pd_tensor* key_cache,
                    const pd_tensor* value_cache, const pd_tensor* k_scale, const pd_tensor* v_scale,
                    const pd_tensor* slot_mapping, hipStream_t stream, char* err, int errlen) {
    if (!key || !value || !key_cache || !value_cache || !k_scale || !v_scale || !slot_mapping)
        return fail(err, errlen, "null tensor descriptor");
    if (!layout_ok(key_cache, value_cache, k_scale, v_scale))
        return fail(err, errlen, "KV cache views do not have the int8 per-token-head row layout");
    const int dt = key->dtype;
    if (!((dt == PD_DTYPE_FP16 || dt == PD_DTYPE_BF16 || dt == PD_DTYPE_FP32) && value->dtype == dt))
        return fail(err, errlen, "key and value must be fp16, bf16 or fp32 of the same dtype");
    const int64_t T = key->sizes[0], Hkv = key_cache->sizes[2];
    if (!(key->ndim == 3 && value->ndim == 3 && key->sizes[1] == Hkv && value->sizes[1] == Hkv &&
          key->sizes[2] == 256 && value->sizes[2] == 256 && value->sizes[0] == T && key->strides[2] == 1 &&
          value->strides[2] == 1))
        return fail(err, errlen, "key and value must be [T, Hkv, 256] with unit dim stride");
    if (T * Hkv > ((int64_t)1 << 30)) return fail(err, errlen, "at most 2^30 (token, kv head) rows per call");
    const int64_t esz = dt == PD_DTYPE_FP32 ? 4 : 2;
    const int64_t vec = 4 * esz;  // each lane loads 4 elements
    if (!((reinterpret_cast<uintptr_t>(key->data) % vec) == 0 && (reinterpret_cast<uintptr_t>(value->data) % vec) == 0 &&
          key->strides[0] % 4 == 0 && key->strides[1] % 4 == 0 && value->strides[0] % 4 == 0 &&
          value->strides[1] % 4 == 0))
        return fail(err, errlen, "key and value rows must be aligned to 4 elements");
    if (!(slot_mapping->dtype == PD_DTYPE_INT64 && slot_mapping->ndim == 1 && slot_mapping->sizes[0] >= T &&
          (slot_mapping->strides[0] == 1 || slot_mapping->sizes[0] <= 1)))
        return fail(err, errlen, "slot_mapping must be a contiguous int64 [T]");
    if (T == 0) return 0;
    CacheWriteParams p;
    p.key = key->data;
    p.value = value->data;
    p.k_st = key->strides[0];
    p.k_sh = key->strides[1];
    p.v_st = value->strides[0];
    p.v_sh = value->strides[1];
    p.kc = static_cast<int8_t*>(const_cast<void*>(key_cache->data));
    p.k_sb = key_cache->strides[0];
    p.k_ss = key_cache->strides[1];
    p.k_sh_c = key_cache->strides[2];
    p.slots = static_cast<const int64_t*>(slot_mapping->data);
    p.block_size = (int)key_cache->sizes[1];
    p.num_slots = key_cache->sizes[0] * key_cache->sizes[1];
    p.T = (int)T;
    p.Hkv = (int)Hkv;
    const hipError_t e = pd::launch_cache_write(p, dt, stream);
    if (e != hipSuccess) {
        char msg[256];
        snprintf(msg, sizeof msg, "cache write launch failed: %s", hipGetErrorString(e));
        fail(err, errlen, msg);
        return 2;
    }
    return 0;
}

const char* pth_dec_version(void) { return "pth_dec-gfx950 0.2"; }

}  // extern "C"

#pragma GCC visibility pop
