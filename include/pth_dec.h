/*
 * MI355X (gfx950) split-K decode attention over vLLM's int8 per-token-head paged KV cache.
 *
 * C ABI of libpthdec.so. Plain pointers, strides and sizes only; every device pointer is
 * owned by the caller and no entry point allocates, frees or synchronises the host, so a
 * launch may be captured in a HIP graph.
 *
 * Cache row layout (one row per (block, slot, kv head), 520 bytes):
 *     [ K int8 x 256 | k_scale f32 | V int8 x 256 | v_scale f32 ]
 * key_cache is the int8 view [blocks, block_size, Hkv, 260] whose last dim is contiguous;
 * value_cache is the same storage shifted by 260 bytes; k_scale / v_scale are f32 views
 * [blocks, block_size, Hkv] at +256 / +516 bytes of each row.
 *
 * Range of the attention entry points (decode and prefill): each key's value weight is formed in
 * fp16 as p * v_scale * 16 with p <= 16 (the running max lags a row's true max by at most 4 in
 * log2 units), so v_scale must stay below 255.9, i.e. V rows with absmax below ~32,500. Larger
 * scales can overflow that weight to infinity. pth_cache_write produces such scales only from
 * V inputs above ~32,500 in magnitude.
 *
 * Reference interfaces replaced (paths relative to the 0c33/mi50-vllm-lab tree):
 *   pth_dec_launch             <- kernels/pth_dec/pth_dec.cu:285-314 (same signature)
 *   pth_dec_launch_window      <- same, plus the window / non-causal rule of
 *                                 patches/vllm/gfx906_fa_paged.patch:7-20 and
 *                                 kernels/fa_pth/kernel/fattn-q8-paged.cuh:219-229
 *   pth_dec_supported_layout   <- supported_layout, kernels/pth_dec/pth_dec.cpp:25-41
 *   pth_dec_decode             <- decode, kernels/pth_dec/pth_dec.cpp:43-91 (the torch op body,
 *                                 with tensors passed as pd_tensor descriptors)
 *   pth_fa_forward             <- forward_pth, kernels/fa_pth/pth_fa.cpp:41-85 (chunked prefill)
 *   pth_cache_write            <- vLLM's int8 per-token-head cache update (do_kv_cache_update)
 */
#ifndef PTH_DEC_H
#define PTH_DEC_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes used in pd_tensor.dtype */
#define PD_DTYPE_INT8 1
#define PD_DTYPE_FP16 2
#define PD_DTYPE_FP32 3
#define PD_DTYPE_INT32 4
#define PD_DTYPE_BF16 5
#define PD_DTYPE_INT64 6

#define PD_MAX_DIMS 4

/* A strided tensor view: data pointer, dtype code, rank, sizes and strides in elements. */
typedef struct pd_tensor {
    const void* data;
    int32_t dtype;
    int32_t ndim;
    int64_t sizes[PD_MAX_DIMS];
    int64_t strides[PD_MAX_DIMS];
} pd_tensor;

/*
 * Split-K decode attention, causal, no window. Same arguments, meaning and error codes as
 * kernels/pth_dec/pth_dec.cu:285-290:
 *   q            fp16 [num_tokens, heads_q, 256], token stride q_st elements, head stride 256
 *   kc           int8 cache base (key_cache.data_ptr()); k_sb / k_ss / k_sh are the byte strides
 *                of blocks, slots and kv heads; V sits at +260 bytes of each K row
 *   block_table  int32, row stride bt_stride; seq_lens int32 [num_seqs];
 *   qsl          int32 query_start_loc [num_seqs + 1]
 *   part_o       fp32 [>= num_tokens, heads_q, nseg, 256]; part_m / part_l fp32 [.., heads_q, nseg]
 *   out          fp16, element (t, h, d) at out + t * o_st + h * o_sh + d
 * Returns hipErrorInvalidValue unless heads_q == 6 * heads_kv, 1 <= qmax <= 4,
 * 1 <= nsplit <= nseg and num_seqs >= 1.
 */
hipError_t pth_dec_launch(const void* q, int q_st, const void* kc, int k_sb, int k_ss, int k_sh,
                          const int* block_table, int bt_stride, const int* seq_lens, const int* qsl,
                          int num_seqs, int num_tokens, int heads_q, int heads_kv, int block_size,
                          float scale, int qmax, float* part_o, float* part_m, float* part_l, int nseg,
                          int nsplit, void* out, long o_st, long o_sh, hipStream_t stream);

/*
 * pth_dec_launch with the arguments the DFlash2 drafter needs appended:
 *   window  > 0: row j of a sequence (absolute position p_j = seq_len - q_len + j) sees key k
 *                only if p_j - k < window; <= 0 (e.g. -1): no window
 *   causal  != 0: key k > p_j is masked; 0: every key < seq_len is visible (non-causal block)
 * Any GQA ratio heads_q / heads_kv with qmax * (heads_q / heads_kv) <= 48 is accepted
 * (MTP 4 x 6 = 24 rows, DFlash2 8 x 6 = 48 rows).
 */
hipError_t pth_dec_launch_window(const void* q, int q_st, const void* kc, int k_sb, int k_ss, int k_sh,
                                 const int* block_table, int bt_stride, const int* seq_lens,
                                 const int* qsl, int num_seqs, int num_tokens, int heads_q, int heads_kv,
                                 int block_size, float scale, int qmax, float* part_o, float* part_m,
                                 float* part_l, int nseg, int nsplit, void* out, long o_st, long o_sh,
                                 hipStream_t stream, int window, int causal);

/*
 * The two stages of pth_dec_launch_window launched separately (no counterpart in the
 * reference, which always launches both): the split-K partial pass writes part_o / part_m /
 * part_l, the combine pass merges them into out. Same argument checks.
 */
hipError_t pth_dec_launch_partial(const void* q, int q_st, const void* kc, int k_sb, int k_ss, int k_sh,
                                  const int* block_table, int bt_stride, const int* seq_lens,
                                  const int* qsl, int num_seqs, int num_tokens, int heads_q,
                                  int heads_kv, int block_size, float scale, int qmax, float* part_o,
                                  float* part_m, float* part_l, int nseg, int nsplit,
                                  hipStream_t stream, int window, int causal);
hipError_t pth_dec_launch_combine(const int* seq_lens, const int* qsl, int num_seqs, int num_tokens,
                                  int heads_q, int qmax, const float* part_o, const float* part_m,
                                  const float* part_l, int nseg, int nsplit, void* out, long o_st,
                                  long o_sh, hipStream_t stream);

/*
 * pth_dec_launch_window without the partial buffers, for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. The split partials go to a device array the library holds (32 MiB
 * per GPU, for the life of the process); this call allocates nothing. Limit:
 * num_tokens * heads_q * nsplit * 1032 bytes <= 32 MiB (e.g. 4 tokens x 24 heads x 64 splits);
 * beyond it the call returns hipErrorOutOfMemory and launches nothing. Other checks and errors
 * as pth_dec_launch_window. Every call on a GPU shares that GPU's array: calls that overlap on
 * one GPU (different streams) race; calls on one stream are ordered and safe.
 */
hipError_t pth_dec_launch_noalloc(const void* q, int q_st, const void* kc, int k_sb, int k_ss, int k_sh,
                                  const int* block_table, int bt_stride, const int* seq_lens,
                                  const int* qsl, int num_seqs, int num_tokens, int heads_q,
                                  int heads_kv, int block_size, float scale, int qmax, int nsplit,
                                  void* out, long o_st, long o_sh, hipStream_t stream, int window,
                                  int causal);

/* 1 if the four cache views have the row layout above, else 0 (pth_dec.cpp:25-41). */
int pth_dec_supported_layout(const pd_tensor* key_cache, const pd_tensor* value_cache,
                             const pd_tensor* k_scale, const pd_tensor* v_scale);

/*
 * The torch op `decode` of kernels/pth_dec/pth_dec.cpp:49-91 over descriptors, with window
 * and causal appended. Validates every tensor like the reference's TORCH_CHECKs (and refuses
 * sizes, counts or a window that do not fit in 32 bits); on failure
 * returns 1 and writes the reference's message into err (errlen bytes, NUL-terminated);
 * returns 2 with the HIP error string if the launch fails; 0 on success.
 */
int pth_dec_decode(const pd_tensor* q, const pd_tensor* key_cache, const pd_tensor* value_cache,
                   const pd_tensor* k_scale, const pd_tensor* v_scale, const pd_tensor* block_table,
                   const pd_tensor* seq_lens, const pd_tensor* query_start_loc, const pd_tensor* out,
                   double scale, const pd_tensor* part_o, const pd_tensor* part_m, const pd_tensor* part_l,
                   int64_t num_seqs, int64_t qmax, int64_t nsplit, int64_t window, int64_t causal,
                   hipStream_t stream, char* err, int errlen);

/* Library version string. */
const char* pth_dec_version(void);

/*
 * Causal chunked prefill over the same int8 per-token-head cache. Replaces forward_pth,
 * kernels/fa_pth/pth_fa.cpp:41-85 (same arguments, meaning and error messages), with the output
 * passed in instead of allocated:
 *   q            fp32 [B, Hq, Sq, 256] contiguous; query token i of sequence b sits at absolute
 *                position q_abs_offset[b] + i and sees keys k <= that position, k < seq_lens[b]
 *   key_cache / value_cache  the cache views (value_cache = key_cache + 260 bytes)
 *   block_table  int32 [B, max_blocks]; seq_lens, q_abs_offset int32 [B]
 *   out          fp32 [B, Sq, Hq, 256], unit dim stride
 * Q is rounded to fp16 for the matrix cores; scores and P.V accumulate in fp32. B, Hq and Sq
 * must be below 2^31. Returns 0, 1 (validation failure, message in err) or 2 (launch failure).
 * Accuracy: each softmax weight enters P.V as one fp16 P' = p * v_scale * 16 (11 significant
 * bits), so an output element is within 2e-3 + 2^-11 * sum_k p_k |v_k| / l of the float64
 * result (v_k the dequantised value, l = sum_k p_k). On caches of N(0,1)-like rows that is
 * inside max-abs 2e-3 / mean-abs 2e-4; on caches with outlier rows (1 % of rows at 50x) the
 * second term dominates (max-abs 5.1e-2 at outputs near 148, 2^-11.5 relative). That is below
 * one fp16 spacing of the output, so a caller that stores fp16 (vLLM's attention output) loses
 * nothing to it; a caller that needs fp32-grade results on such caches uses
 * pth_fa_forward_exact.
 */
int pth_fa_forward(const pd_tensor* q, const pd_tensor* key_cache, const pd_tensor* value_cache,
                   const pd_tensor* block_table, const pd_tensor* seq_lens, double scale,
                   const pd_tensor* q_abs_offset, const pd_tensor* out, hipStream_t stream, char* err,
                   int errlen);

/*
 * No counterpart in the reference. pth_fa_forward with the decode's numerics: K and V converted
 * to fp16 without the widening bias, so the fp32 accumulators hold only the products' own sums,
 * and P' carried as fp16 hi + lo (~22 bits instead of 11). It is for callers whose caches hold rows
 * with very large scales (attention sinks, outlier tokens), where pth_fa_forward's single-fp16
 * P' can miss max-abs 2e-3. It is slower: the P.V products double. Arguments, checks, errors and
 * return codes are those of pth_fa_forward.
 */
int pth_fa_forward_exact(const pd_tensor* q, const pd_tensor* key_cache, const pd_tensor* value_cache,
                         const pd_tensor* block_table, const pd_tensor* seq_lens, double scale,
                         const pd_tensor* q_abs_offset, const pd_tensor* out, hipStream_t stream, char* err,
                         int errlen);

/*
 * No counterpart in the reference. pth_fa_forward (exact != 0: pth_fa_forward_exact) with each
 * query tile's keys split over nsplit workgroups, for chunks too short to fill the GPU (a
 * workgroup takes 192 query rows of one kv head, so a 64-token chunk of 24 q / 4 kv heads
 * launches 8 of them per split) or whose workgroups end in a part-filled round. Each split stores unnormalised partials in the caller's
 * workspace, and a second kernel merges them into out.
 *   workspace  fp32, contiguous, 16-byte aligned, at least B * Sq * Hq * nsplit * 258 floats
 *              (ignored when nsplit == 1)
 *   nsplit     1..64; when above 1, B * Sq * Hq must be below 2^31
 * Other arguments, checks, errors and return codes are those of pth_fa_forward. The results
 * equal pth_fa_forward's within rounding (the partial sums are merged in another order).
 */
int pth_fa_forward_split(const pd_tensor* q, const pd_tensor* key_cache, const pd_tensor* value_cache,
                         const pd_tensor* block_table, const pd_tensor* seq_lens, double scale,
                         const pd_tensor* q_abs_offset, const pd_tensor* out, const pd_tensor* workspace,
                         int64_t nsplit, int64_t exact, hipStream_t stream, char* err, int errlen);

/*
 * KV-cache writer and quantiser: the producer of the 520-byte rows the two operators read.
 * Replaces vLLM's cache update for int8 per-token-head KV, which the reference calls as
 * do_kv_cache_update(layer, key, value, kv_cache, slot_mapping)
 * (upstream/pr-dflash2/0002-fix-gfx906-keep-the-drafter-s-sliding-window-in-the-.patch:81-87;
 * the update itself lives in the un-vendored vLLM fork KIntegrated/vllm-gfx906-mobydick 0.30.0).
 *   key, value   fp16, bf16 or fp32 [T, Hkv, 256], unit dim stride
 *   key_cache, value_cache, k_scale, v_scale   the cache views (as for pth_dec_decode)
 *   slot_mapping int64 [T]: slot = block * block_size + offset; negative slots (padding) and
 *                slots past the cache are skipped
 * Per (token, kv head): scale = absmax / 127 (0 for an all-zero row), q = clamp(rint(x / scale),
 * -127, 127) with x / scale correctly rounded. At most 2^30 (token, kv head) rows per call.
 * Returns 0, 1 (validation failure, message in err) or 2 (launch failure).
 */
int pth_cache_write(const pd_tensor* key, const pd_tensor* value, const pd_tensor* key_cache,
                    const pd_tensor* value_cache, const pd_tensor* k_scale, const pd_tensor* v_scale,
                    const pd_tensor* slot_mapping, hipStream_t stream, char* err, int errlen);

#ifdef __cplusplus
}
#endif

#endif /* PTH_DEC_H */
