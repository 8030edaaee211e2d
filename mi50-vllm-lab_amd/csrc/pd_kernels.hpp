// Internal interface of libpthdec.so between the C ABI (pd_api.hip) and the kernel files
// (pd_decode.hip, pd_prefill.hip, pd_cache_write.hip): the parameter block each kernel takes and
// the host functions that launch them. The public interface is include/pth_dec.h; nothing here
// is exported from the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace pd {

constexpr int kDim = 256;             // head dim (the only one the cache row layout allows)
constexpr int kMaxRowBlocks = 3;      // decode: up to 48 query rows per kv head
constexpr int64_t kSliceKeys = 16384; // decode: largest sequences x window whose row groups are sliced

// Prefill workgroup shape: kFaWaves waves of kFaRB 16-row blocks, so a workgroup takes
// kFaRows / G query tokens of one sequence and all G heads of one kv head.
constexpr int kFaWaves = 4;
constexpr int kFaRB = 3;                        // row blocks per wave
constexpr int kFaRows = kFaWaves * kFaRB * 16;  // 192

// Split-K decode, partial pass (pd_partial_kernel).
struct PartialParams {
    const _Float16* q;
    int64_t q_st;            // elements between query tokens
    const int8_t* kc;        // cache base
    int64_t k_sb, k_ss, k_sh;  // bytes between blocks / slots / kv heads
    const int* block_table;
    int64_t bt_stride;
    const int* seq_lens;
    const int* qsl;
    int block_size;
    float scale_log2;        // softmax scale * log2(e)
    float* part_o;
    float* part_m;
    float* part_l;
    int nseg;
    int nsplit;
    int G;                   // query heads per kv head
    int qmax;
    int Hq;
    int window;              // > 0: sliding window, else none
    int causal;
    int bs_shift;            // log2(block_size) if it is a power of two, else -1
    int num_seqs;
    int rslices;             // workgroups per (sequence, kv head, split), each 16 NRB of the rows
};

// Split-K decode, log-sum-exp merge of the partials (pd_combine_kernel).
struct CombineParams {
    const float* part_o;
    const float* part_m;
    const float* part_l;
    const int* seq_lens;
    const int* qsl;
    _Float16* out;
    int64_t o_st, o_sh;
    int num_seqs;
    int nseg;
    int nsplit;
    int qmax;
};

// Chunked prefill (pd_prefill_kernel).
struct FaParams {
    const float* q;
    int64_t q_sb, q_sh, q_st;  // elements between batches / heads / tokens of q [B, Hq, Sq, 256]
    const int8_t* kc;
    int64_t k_sb, k_ss, k_sh;
    const int* block_table;
    int64_t bt_stride;
    const int* seq_lens;
    const int* q_abs;
    float* out;
    int64_t o_sb, o_st, o_sh;  // elements between batches / tokens / heads of out [B, Sq, Hq, 256]
    int Sq, Hq, G, tok_per_wg, block_size, bs_shift;
    int bt32;                  // every K row lies within 2^35 bytes of the cache base
    float scale_log2;
    // nsplit > 1: each query tile's visible key tiles are split into nsplit contiguous runs, one
    // workgroup each, which store unnormalised partials (O, m, l) for every row; row r = (b * Sq +
    // token) * Hq + head of split s at part_o[(r * nsplit + s) * 256], part_m / part_l[r * nsplit + s]
    int nsplit;
    float* part_o;
    float* part_m;
    float* part_l;
};

// KV-cache writer (pd_cache_write_kernel).
struct CacheWriteParams {
    const void* key;
    const void* value;
    int64_t k_st, k_sh, v_st, v_sh;  // elements between tokens / heads of key and value
    int8_t* kc;
    int64_t k_sb, k_ss, k_sh_c;      // cache bytes between blocks / slots / kv heads
    const int64_t* slots;
    int64_t num_slots;               // blocks * block_size
    int T, Hkv, block_size;
};

// The decode launch as the C ABI describes it (pointers, strides in bytes or elements as the
// entry points take them).
struct LaunchArgs {
    const void* q;
    int64_t q_st;
    const void* kc;
    int64_t k_sb, k_ss, k_sh;
    const int* block_table;
    int64_t bt_stride;
    const int* seq_lens;
    const int* qsl;
    int num_seqs, num_tokens, heads_q, heads_kv, block_size;
    float scale;
    int qmax;
    float* part_o;
    float* part_m;
    float* part_l;
    int nseg, nsplit;
    void* out;
    int64_t o_st, o_sh;
    int window, causal;
};

// Row blocks of 16 keys never straddle a page when block_size is a multiple of 16: then every
// row block of a tile has one scalar base address.
inline bool fast_block_table(int bs, int64_t k_ss) { return bs % 16 == 0 && k_ss < (int64_t(1) << 27); }

// decode (pd_decode.hip)
hipError_t check_args(const LaunchArgs& x, bool strict_reference);
hipError_t launch_partial(const LaunchArgs& x, hipStream_t stream);
hipError_t launch_combine(const LaunchArgs& x, hipStream_t stream);
hipError_t launch_all(const LaunchArgs& x, hipStream_t stream, bool strict);
// the device array behind pth_dec_launch_noalloc, and its address on the current device
constexpr size_t kScratchBytes = size_t(32) << 20;
hipError_t scratch_address(void** out);

// chunked prefill (pd_prefill.hip)
// exact: K converted to fp16 without the widening bias and P' as fp16 hi + lo (pth_fa_forward_exact)
hipError_t launch_prefill(const FaParams& p, int batch, int heads_kv, hipStream_t stream, bool exact);
// workspace floats a split prefill needs: B * Sq * Hq rows x nsplit x (256 + 2)
inline int64_t prefill_workspace_floats(int64_t B, int64_t Sq, int64_t Hq, int64_t nsplit) {
    return B * Sq * Hq * nsplit * (kDim + 2);
}

// cache writer (pd_cache_write.hip); dtype is a PD_DTYPE_* code of key and value
hipError_t launch_cache_write(const CacheWriteParams& p, int dtype, hipStream_t stream);

}  // namespace pd
