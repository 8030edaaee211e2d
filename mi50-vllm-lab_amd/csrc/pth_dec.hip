// Split-K decode attention over vLLM's int8 per-token-head paged KV cache, written for
// MI355X (gfx950, CDNA4). Behaviour follows kernels/pth_dec/pth_dec.cu:1-314 and
// kernels/pth_dec/pth_dec.cpp:1-96 of 0c33/mi50-vllm-lab (same C ABI, same partial-buffer
// semantics), extended with the sliding-window / non-causal rule of
// patches/vllm/gfx906_fa_paged.patch:7-20 and kernels/fa_pth/kernel/fattn-q8-paged.cuh:219-229.
//
// Work decomposition
//   grid (nsplit, Hkv, num_seqs), 256 threads = 4 waves of 64 lanes, one workgroup per CU.
//   The keys a sequence can see, [lo, seq_len), are cut into 32-key tiles aligned to
//   multiples of 32; split s owns a contiguous run of tiles and wave w of that split takes
//   every 4th tile. All R = q_len * G query rows of the GQA group (24 for MTP, 48 for
//   DFlash2) are held as 16-row blocks, so one read of a K/V tile serves every row.
//
// Memory path: HBM -> LDS by DMA (global_load_lds_dwordx4), double-buffered per wave, no VGPR
//   holding data in flight. A tile is 17 DMA instructions of 1 KiB: 8 for K (4 rows x 256
//   bytes each, at positions swizzled so the operand reads are bank-conflict free), 8 for
//   bytes [256, 512) of the rows (k_scale and V), one for bytes [504, 520) (the last V bytes and
//   v_scale). With block_size a multiple of 16 a 16-key row block sits in one page, so each
//   instruction is a scalar base (page, slot) plus a per-lane constant offset. Tile n + 1 is in
//   flight while tile n is computed; tile n + 2 is issued into tile n's slot in parts: its 8 K
//   copies as soon as tile n's operands are in registers (the queue space tile n has just freed
//   takes them without a stall), the other 9 once tile n is done (in the first two iterations
//   four of them already between the scores and the values). The block-table slice
//   of the split is staged in LDS once (as 64-bit row offsets), and with block sizes that are
//   multiples of 16 Q is copied into LDS the same way (48 rows: into the V images of the
//   second slots of waves 0-2), so the first tile (and the K copies of the second) is issued one
//   memory round trip after the kernel starts.
//
// Per 32-key tile, per wave
//   S^T = K Q^T on v_mfma_f32_16x16x32_f16: A = 16 keys x 32 dims of K (int8 widened to fp16
//     exactly: 0x6400|(b^0x80) encodes 1024+b+128), B = Q^T held in registers; the four
//     accumulation chains (2 key blocks x 2 row blocks) are interleaved.
//   softmax: base 2, fp32, online. A row's running max is raised only when a tile exceeds it
//     by > 2^4: each lane tests its own 8 scores and one ballot decides; only then is the row
//     max reduced across lanes and O rescaled (rare after the first tile). P' = p * v_scale * 16
//     in fp16 has the range of p * v_scale * 256 with p <= 1. Masked weights are chosen by
//     select, so a NaN scale on a masked row cannot leak in.
//   O^T += V^T P^T: ds_read_b64_tr_b8 hands each lane 8 keys of one V column (A operand,
//     16 dims x 32 keys); P^T never leaves registers: the S^T accumulator layout (lane = query
//     row, 4 keys per 16-key block) is the B-operand layout once the MFMA's key order is chosen
//     to match. Dim block j < 16 reads row bytes [256 + 16 j, 272 + 16 j) (dims 16 j - 4 ..),
//     block 16 the tail bytes (dims 244..255); lanes outside [0, 256) are discarded.
//   Keys outside [lo, seq_len) are never addressed through freed pages: rows of a tile that
//     fall outside are pointed at a page the split can see and masked.
//
// End of split: the 4 waves merge (m, l, O) through LDS and write one partial per row:
//   part_o [T, Hq, nseg, 256] unnormalised, part_m [T, Hq, nseg] running max in log2 units,
//   part_l the matching sum. Each wave stores its accumulators straight from the AGPRs and the
//   per-row factors are applied while summing. Splits with no
//   tiles write m = -inf. The combine kernel merges the partials of each (token, head) with a
//   log-sum-exp rescale.
//
// The file also holds the chunked-prefill kernel (same cache, same tile copies, 192 rows per
// workgroup) and the KV-cache writer; each has its own description below.
//
// Nothing is allocated, nothing waits for the host, and every split range is derived on
// the device from seq_lens / query_start_loc, so launches can be captured in a HIP graph.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <type_traits>

#include "pth_dec.h"

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef int int2_t __attribute__((ext_vector_type(2)));
typedef unsigned uint4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) unsigned char lds_u8;
typedef __attribute__((address_space(3))) int2_t lds_int2;
typedef __attribute__((address_space(3))) uint4_t lds_uint4;
typedef __attribute__((address_space(3))) float lds_float;
typedef __attribute__((address_space(3))) int lds_int;
typedef __attribute__((address_space(3))) uint64_t lds_u64;
typedef unsigned long long ull2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) ull2_t lds_ull2;
typedef __attribute__((address_space(3))) half8_t lds_half8;
typedef const __attribute__((address_space(4))) int* const_int_ptr;  // scalar-cache loads

constexpr int kDim = 256;             // head dim (the only one the cache row layout allows)
constexpr int kTile = 32;             // keys per tile
constexpr int kMaxRowBlocks = 3;      // up to 48 query rows per kv head
constexpr float kNegInf = -__builtin_inff();
// The running max m of a row is only raised when a tile's max exceeds it by more than
// kLazy (log2 units), so p = 2^(s - m) <= 2^kLazy and most tiles skip the O rescale.
// P' = p * v_scale * kPScale then spans the same fp16 range as p * v_scale * 256 with p <= 1.
constexpr float kLazy = 4.0f;
constexpr float kPScale = 16.0f;

// LDS slot of one tile (each wave double-buffers its tiles; 17664 bytes per slot).
//   K image, 8 DMA blocks of 1040 bytes (1024 + 16 of padding): block i holds the tile rows
//     16 (i >> 2) + 4 (i & 3) + q, q = 0..3, bytes [0, 256); row q of the block at 256 q, its
//     16-byte chunk c at position c ^ 4 q.
//   V image, 8 blocks of 1040 bytes at kImgV: block i holds rows 16 (i >> 2) + (i & 3) + 4 q,
//     bytes [256, 512) (k_scale, V[0..252)); row q at 256 q, chunk c at position c ^ 8 (q & 1).
//   Tail, 1024 bytes at kImgT: bytes [504, 520) of row r at 16 tpos(r), tpos(r) = r for r < 16
//     and 16 + ((r - 16) ^ 8) above (the DMA's lanes 32..63 land a copy at +512).
// With these placements the 16 rows one 16-lane group reads for the K operand, and the 8 rows a
// ds_read_b64_tr_b8 group reads, fall on distinct LDS banks. Each DMA block is 4 rows of 256
// contiguous bytes of one page, so its 64 lanes share a scalar base.
// Block sizes that are not a multiple of 16 use chunk-major images instead (chunk j of row r at
// 512 j + 16 r), filled from per-lane row addresses.
constexpr int kBlk = 1040;
constexpr int kImgK = 0;
constexpr int kImgV = 8 * kBlk;
constexpr int kImgT = 16 * kBlk;
constexpr int kSlot = kImgT + 1024;
constexpr int kWaveLds = 2 * kSlot;                // LDS bytes per wave
constexpr int kWaves = 4;                          // independent tile streams per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kBtCache = 1024;                     // block-table entries of a split kept in LDS
// With Q staged in LDS as well (block sizes that are multiples of 16) the block-table slice
// is smaller:
constexpr int kBtEarly = 384;                      // per-block row offsets (48 tiles per wave)
constexpr int kBtRaw = 384;                        // raw block-table entries (96 per wave)
constexpr int kBtWave = kBtEarly / 4;              // 16-key blocks staged per wave

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
};

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


// 8 signed bytes b (two dwords, byte 0 first) -> 8 fp16 holding b + 1152, exact: the bit
// pattern 0x6400 | (b ^ 0x80) encodes 1024 + (b + 128). The constant 1152 is not subtracted
// here; the kernel removes it once per row instead: S = sum_d q_d (k_d + 1152) - 1152 sum_d q_d
// and O = sum_k P'_k (v_k + 1152) - 1152 sum_k P'_k.
constexpr float kWidenBias = 1152.0f;
__device__ __forceinline__ half8_t widen_i8x8(unsigned w0, unsigned w1) {
    const unsigned u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;  // b + 128 as unsigned bytes
    // v_perm_b32 selector bytes 0..3 pick bytes of the 2nd operand, 4 picks byte 0 of the 1st.
    uint4_t h;
    h.x = __builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u);  // [u0.b0, 0x64, u0.b1, 0x64]
    h.y = __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u);  // [u0.b2, 0x64, u0.b3, 0x64]
    h.z = __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u);
    h.w = __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u);
    return __builtin_bit_cast(half8_t, h);
}

__device__ __forceinline__ float xor_max(float v, int mask) { return fmaxf(v, __shfl_xor(v, mask, 64)); }
__device__ __forceinline__ float xor_sum(float v, int mask) { return v + __shfl_xor(v, mask, 64); }

// Block-table access of one workgroup: the slice of pages its split can touch is staged in
// LDS when it fits (kBtCache entries), so the tile loop issues no loads of its own besides the
// K/V rows; otherwise entries are read with scalar loads through the constant address space.
struct PageTable {
    const lds_int* lds;      // slice [pfirst, pfirst + kBtCache)
    const lds_ull2* rows16;  // fast layout: per tile, the first-row offsets of its two 16-key blocks
    const_int_ptr glob;  // this sequence's block-table row
    int pfirst;
    int in_lds;
    template <bool kLds>
    __device__ __forceinline__ int64_t get(int lb) const {
        if constexpr (kLds)
            return (int64_t)lds[lb - pfirst];
        else
            return (int64_t)glob[lb];
    }
    // Same, for a wave-uniform lb: the result is made uniform (scalar register) explicitly.
    template <bool kLds>
    __device__ __forceinline__ int64_t get_uniform(int lb) const {
        if constexpr (kLds)
            return (int64_t)__builtin_amdgcn_readfirstlane(lds[lb - pfirst]);
        else
            return (int64_t)glob[lb];
    }
};

// Where a tile's rows live. kFast (block_size a multiple of 16, so a 16-key row block sits in
// one page): row 16 u + x of the tile at base[u] + x * k_ss, base[u] uniform. Other block sizes:
// base[0] is this lane's own tile row, lane & 31. Keys outside [lo, hi) are replaced by visible
// keys of the same tile (their scores are masked), so a freed page is never addressed.
struct TileSrc {
    const int8_t* base[2];
};

template <bool kFast, bool kLds, class P>
__device__ __forceinline__ TileSrc tile_src(const P& a, const PageTable& pt, const int8_t* gbase,
                                            int tile, int idx, int lo, int hi, int lane) {
    if constexpr (kFast && kLds) {
        // precomputed when the wave started (entry idx = the wave's tile number): one LDS read,
        // no address arithmetic. The halves are zero-extended (readfirstlane returns a signed int).
        const ull2_t r2 = pt.rows16[idx];
        const uint64_t o0 = ((uint64_t)(unsigned)__builtin_amdgcn_readfirstlane((unsigned)(r2.x >> 32)) << 32) |
                            (uint64_t)(unsigned)__builtin_amdgcn_readfirstlane((unsigned)r2.x);
        const uint64_t o1 = ((uint64_t)(unsigned)__builtin_amdgcn_readfirstlane((unsigned)(r2.y >> 32)) << 32) |
                            (uint64_t)(unsigned)__builtin_amdgcn_readfirstlane((unsigned)r2.y);
        TileSrc src;
        src.base[0] = gbase + (int64_t)o0;
        src.base[1] = gbase + (int64_t)o1;
        return src;
    }
    const int kb = tile * kTile;
    const int kfirst = max(kb, lo), klast = min(kb + kTile - 1, hi - 1);
    const int bs = a.block_size;
    TileSrc src;
    if constexpr (kFast) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int key0 = min(max(kb + 16 * u, kfirst), klast) & ~15;
            const int lb = a.bs_shift >= 0 ? key0 >> a.bs_shift : key0 / bs;
            src.base[u] = gbase + pt.get_uniform<kLds>(lb) * a.k_sb + (int64_t)(key0 - lb * bs) * a.k_ss;
        }
    } else {
        const int key = min(max(kb + (lane & 31), kfirst), klast);
        const int lb = a.bs_shift >= 0 ? key >> a.bs_shift : key / bs;
        src.base[0] = gbase + pt.get<kLds>(lb) * a.k_sb + (int64_t)(key - lb * bs) * a.k_ss;
        src.base[1] = src.base[0];
    }
    return src;
}

// 16-byte HBM -> LDS copies: LDS[dst + 16 * lane] = global[...]. Issued through asm so the
// compiler adds no vmcnt wait of its own before the LDS reads; completion is awaited with
// wait_vm. dma16_s: uniform base + per-lane 32-bit offset; dma16_v: per-lane address + imm.
__device__ __forceinline__ void dma16_s(const int8_t* sbase, unsigned voff, unsigned m0) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(m0)
                 : "memory", "m0");
}
// The immediate offset applies to the LDS destination too: the copy lands at m0 + kImm +
// 16 * lane, so m0 is passed already reduced by kImm.
template <int kImm>
__device__ __forceinline__ void dma16_v(const int8_t* vaddr, unsigned lds_dst) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off offset:%2" ::"v"(vaddr), "s"(lds_dst - kImm),
                 "i"(kImm)
                 : "memory", "m0");
}
// 4-byte copies: LDS[dst + 4 * lane] = *vaddr.
__device__ __forceinline__ void dma4_v(const int* vaddr, unsigned lds_dst) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(vaddr), "s"(lds_dst) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Per-lane constants of the DMA addressing (see the slot layout).
struct DmaLane {
    unsigned kvo, vvo;   // kFast: offsets of this lane's K / V source bytes from its block's base
    unsigned toff;       // kFast: offset of this lane's tail row from its key block's base
    int tsel;            // key block of this lane's tail row
    unsigned kb2[4];     // kFast: 4 q k_ss, q = 0..3 (K blocks: rows 4 (i & 3) + q)
};

// The 17 DMAs of one tile into the slot at LDS address `slot` (8 K blocks, 8 V blocks, tail).
template <bool kFast, class P>
__device__ __forceinline__ void issue_tile(const P& a, const TileSrc& src, const DmaLane& d,
                                           unsigned slot, int lane) {
    if constexpr (kFast) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int8_t* kb = src.base[i >> 2] + (int64_t)(4 * (i & 3)) * a.k_ss;
            dma16_s(kb, d.kvo, slot + kImgK + i * kBlk);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int8_t* vb = src.base[i >> 2] + (int64_t)(i & 3) * a.k_ss;
            dma16_s(vb, d.vvo, slot + kImgV + i * kBlk);
        }
        const int64_t delta = src.base[1] - src.base[0];
        dma16_v<0>(src.base[0] + (delta & -(int64_t)d.tsel) + d.toff, slot + kImgT);
    } else {
        // chunk-major images: lanes 0-31 copy chunk 2 i of rows 0..31, lanes 32-63 chunk 2 i + 1
        const int8_t* row = src.base[0];  // tile row lane & 31
        const int8_t* p = row + 16 * (lane >> 5);
        dma16_v<0>(p, slot + kImgK + 0 * 1024);
        dma16_v<32>(p, slot + kImgK + 1 * 1024);
        dma16_v<64>(p, slot + kImgK + 2 * 1024);
        dma16_v<96>(p, slot + kImgK + 3 * 1024);
        dma16_v<128>(p, slot + kImgK + 4 * 1024);
        dma16_v<160>(p, slot + kImgK + 5 * 1024);
        dma16_v<192>(p, slot + kImgK + 6 * 1024);
        dma16_v<224>(p, slot + kImgK + 7 * 1024);
        dma16_v<256>(p, slot + kImgV + 0 * 1024);
        dma16_v<288>(p, slot + kImgV + 1 * 1024);
        dma16_v<320>(p, slot + kImgV + 2 * 1024);
        dma16_v<352>(p, slot + kImgV + 3 * 1024);
        dma16_v<384>(p, slot + kImgV + 4 * 1024);
        dma16_v<416>(p, slot + kImgV + 5 * 1024);
        dma16_v<448>(p, slot + kImgV + 6 * 1024);
        dma16_v<480>(p, slot + kImgV + 7 * 1024);
        dma16_v<504>(row, slot + kImgT);
    }
}

// The operands of one tile, read from its LDS slot.
struct TileOps {
    uint4_t k[4][2];  // K operand: row 16 u + li, source chunk 4 c + lg
    int2_t v[17];     // transposed V reads, one per 16-dim block
    float ks[8];      // k_scale of this lane's keys 16 u + 4 lg + j
    float vs[8];      // v_scale of the same keys
};

// acc *= alpha for MFMA accumulators, through LDS (16 bytes per lane and accumulator, 1 KiB
// apart from `lds_addr`): the accumulators are read and written only by asm with AGPR operands.
// Four at a time: two LDS round trips per four accumulators.
__device__ __forceinline__ void agpr_scale4_via_lds(float4_t& a0, float4_t& a1, float4_t& a2, float4_t& a3,
                                                    float alpha, unsigned lds_addr) {
    float4_t t0, t1, t2, t3;
    asm volatile(
        "ds_write_b128 %4, %5\n\tds_write_b128 %4, %6 offset:1024\n\t"
        "ds_write_b128 %4, %7 offset:2048\n\tds_write_b128 %4, %8 offset:3072\n\t"
        "s_waitcnt lgkmcnt(0)\n\t"
        "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:1024\n\t"
        "ds_read_b128 %2, %4 offset:2048\n\tds_read_b128 %3, %4 offset:3072\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3)
        : "v"(lds_addr), "a"(a0), "a"(a1), "a"(a2), "a"(a3)
        : "memory");
    t0 *= alpha;
    t1 *= alpha;
    t2 *= alpha;
    t3 *= alpha;
    asm volatile(
        "ds_write_b128 %4, %5\n\tds_write_b128 %4, %6 offset:1024\n\t"
        "ds_write_b128 %4, %7 offset:2048\n\tds_write_b128 %4, %8 offset:3072\n\t"
        "s_waitcnt lgkmcnt(0)\n\t"
        "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:1024\n\t"
        "ds_read_b128 %2, %4 offset:2048\n\tds_read_b128 %3, %4 offset:3072\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&a"(a0), "=&a"(a1), "=&a"(a2), "=&a"(a3)
        : "v"(lds_addr), "v"(t0), "v"(t1), "v"(t2), "v"(t3)
        : "memory");
}

// The same for one accumulator.
__device__ __forceinline__ void agpr_scale_via_lds(float4_t& acc, float alpha, unsigned lds_addr) {
    float4_t t;
    asm volatile("ds_write_b128 %1, %2\n\ts_waitcnt lgkmcnt(0)\n\tds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                 : "=v"(t)
                 : "v"(lds_addr), "a"(acc)
                 : "memory");
    t *= alpha;
    asm volatile("ds_write_b128 %1, %2\n\ts_waitcnt lgkmcnt(0)\n\tds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                 : "=a"(acc)
                 : "v"(lds_addr), "v"(t)
                 : "memory");
}

// One workgroup = kWaves independent waves. Wave w of split s streams tiles tb + w, tb + w + 4,
// ... of the split and computes all R query rows of the kv head for each (NRB row blocks of
// 16), so every K/V byte is loaded and widened once. Each wave double-buffers its tiles in LDS:
// tile n + 1 is copied while tile n is computed, and tile n + 2 is issued as soon as tile n is
// done, so while the wave waits it has two tiles in flight.
template <int NRB, bool kFast>
__global__ void __launch_bounds__(kThreads, 1) pd_partial_kernel(const PartialParams a) {
    constexpr int kLdsWaves = kWaves * kWaveLds;
    constexpr int kLdsStats = kLdsWaves;                  // m, l: [wave][NRB][16]
    // kEarly (block sizes that are multiples of 16): Q and the block-table slice are copied into
    // LDS like the tiles, and each wave's
    // first tile is issued before anything is waited for (addressed with scalar block-table
    // loads), so the copies start one memory round trip after the kernel does; the second
    // tile's K copies follow at once, its other copies after the set-up (a copy issue stalls
    // while the memory queues are full).
    constexpr bool kEarly = kFast;
    constexpr int kLdsBt = kLdsStats + 2 * kWaves * NRB * 16 * 4;
    constexpr int kLdsRaw = kLdsBt + (kEarly ? kBtEarly : kBtCache) * 8;
    constexpr int kLdsQ = kLdsRaw + (kEarly ? kBtRaw * 4 : 0);
    // the merge's table of V widening biases reuses the Q region (or follows the block table)
    // (three row blocks: Q is staged in the V images of slot 1 of waves 0..2 instead, 16 rows
    // each; those slots receive their V copies only after Q is in registers)
    constexpr bool kQInSlots = NRB >= 3;
    constexpr int kQBytes = kEarly && !kQInSlots ? 16 * NRB * 2 * kDim : 0;
    constexpr int kMergeCBytes = kWaves * NRB * 16 * 4;
    constexpr int kLdsMergeC = kLdsQ;
    constexpr int kLdsBytes = kLdsQ + (kQBytes > kMergeCBytes ? kQBytes : kMergeCBytes);
    static_assert(2 * 17 * 1024 <= kWaveLds && kWaveLds % 16 == 0,
                  "two row blocks of accumulator blocks fit the slots of their wave");
    static_assert(kLdsBytes <= 160 * 1024, "gfx950 has 160 KiB of LDS per CU");
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];

    const int s = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, l = tid & 63, lg = l >> 4, li = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, uniform by construction

    // The set-up is a chain of dependent scalar loads (arguments, sequence, block table) before
    // the first copy: make each link one round trip. Every argument the set-up reads is
    // requested at once, then the three sequence words together.
    asm volatile("" ::"s"(a.qsl), "s"(a.seq_lens), "s"(a.block_table), "s"(a.bt_stride), "s"(a.kc), "s"(a.k_sb),
                 "s"(a.k_ss), "s"(a.k_sh), "s"(a.q), "s"(a.q_st), "s"(a.qmax), "s"(a.G), "s"(a.window),
                 "s"(a.nsplit), "s"(a.block_size), "s"(a.bs_shift));
    // (read-only for the kernel's lifetime: scalar loads through the constant address space)
    const int q0 = ((const_int_ptr)(uintptr_t)a.qsl)[b];
    const int q_end = ((const_int_ptr)(uintptr_t)a.qsl)[b + 1];
    const int seq_len = ((const_int_ptr)(uintptr_t)a.seq_lens)[b];
    asm volatile("" ::"s"(q0), "s"(q_end), "s"(seq_len));
    const int q_len = q_end - q0;
    if (q_len <= 0 || seq_len <= 0) return;
    const int ql = min(q_len, a.qmax);
    const int G = a.G;
    const int R = ql * G;
    const int ctx0 = seq_len - q_len;  // absolute position of query token 0
    const int lo = a.window > 0 ? max(0, ctx0 - a.window + 1) : 0;
    const int hi = seq_len;
    const int t_first = lo / kTile;
    const int ntiles = (hi - 1) / kTile - t_first + 1;
    // Tiles of each wave. Split s owns a contiguous run of tiles [tb, te) and its waves take every
    // kWaves-th tile of it, unless the block size is a multiple of 16 and there are at least as
    // many tiles as the W = kWaves * nsplit waves of a (sequence, kv head): then the waves
    // interleave over all the tiles, wave gw = kWaves * s + w taking tiles t_first + gw + W n, so
    // that every split has work and the waves' counts differ by at most one. (Fewer tiles than
    // waves: the contiguous runs measured faster, fewer workgroups with more waves busy.)
    const int per_split = (ntiles + a.nsplit - 1) / a.nsplit;
    const int tb = t_first + s * per_split;
    const int te = min(t_first + ntiles, tb + per_split);
    const int W = kWaves * a.nsplit, gw = kWaves * s + w;
    const bool interleave = kFast && ntiles >= W;
    const bool empty = interleave ? kWaves * s >= ntiles : tb >= te;

    auto prow = [&](int r) -> int64_t {  // partial row index of query row r
        const int i = r / G, hh = r - i * G;
        return ((int64_t)(q0 + i) * a.Hq + (g * G + hh)) * a.nseg + s;
    };

    if (empty) {  // no tiles: mark the split empty for the combine
        for (int r = tid; r < R; r += kThreads) {
            a.part_m[prow(r)] = kNegInf;
            a.part_l[prow(r)] = 0.f;
        }
        return;
    }

    const int nt = interleave ? (gw < ntiles ? (ntiles - 1 - gw) / W + 1 : 0)
                              : max(0, (te - tb - w + kWaves - 1) / kWaves);  // tiles of this wave
    auto tile_of = [&](int n) { return interleave ? t_first + gw + W * n : tb + w + kWaves * n; };

    lds_u8* L = (lds_u8*)lds;
    const unsigned lds_base = (unsigned)(uintptr_t)L;
    const unsigned wslots = lds_base + (unsigned)(w * kWaveLds);  // this wave's two slots
    const int8_t* gbase = a.kc + (int64_t)g * a.k_sh;

    DmaLane dl;
    {
        const int qq = l >> 4, c16 = l & 15, p = l & 31;
        dl.kvo = (unsigned)(qq * a.k_ss) + 16u * (unsigned)(c16 ^ (4 * qq));
        dl.vvo = (unsigned)(4 * qq * a.k_ss) + 256u + 16u * (unsigned)(c16 ^ (8 * (qq & 1)));
        const int rr = p < 16 ? p : ((p - 16) ^ 8);  // row inside its key block of tail position p
        dl.toff = kFast ? (unsigned)(rr * a.k_ss) + 504u : 0u;
        dl.tsel = p >> 4;
    }

    // The block table is read-only for the kernel's lifetime: read it through the constant
    // address space so uniform lookups become scalar loads.
    const_int_ptr bt_row = (const_int_ptr)(uintptr_t)(a.block_table + (int64_t)b * a.bt_stride);
    PageTable pt;
    pt.glob = bt_row;
    pt.lds = (const lds_int*)(L + kLdsBt);
    pt.rows16 = (const lds_ull2*)(L + kLdsBt + (kEarly ? w * kBtWave * 8 : 0));
    pt.pfirst = max(tb * kTile, lo) / a.block_size;

    // ---- Q^T operand (B of S^T = K Q^T) of every row block; lane (lg, li) holds row 16 rb + li,
    //      dims 64 (st / 2) + 16 lg + 8 (st % 2) + [0, 8) in qop[rb][st] ----
    half8_t qop[NRB][8];
    float4_t qneg[NRB];  // -1152 sum_d q_d of the row (every element): the widening bias of K
    bool rvalid[NRB];
    int rpos[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
        const int r = 16 * rb + li;
        rvalid[rb] = r < R;
        const int qi = r / G, qh = r - (r / G) * G;
        rpos[rb] = ctx0 + qi;
        if constexpr (kEarly) continue;
        const _Float16* qrow =
            a.q + (int64_t)(q0 + (rvalid[rb] ? qi : 0)) * a.q_st + (int64_t)(g * G + (rvalid[rb] ? qh : 0)) * kDim;
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            half8_t v;
            const int dim = 64 * (st >> 1) + 16 * lg + 8 * (st & 1);
            __builtin_memcpy(&v, __builtin_assume_aligned(qrow + dim, 4), 16);
            qop[rb][st] = rvalid[rb] ? v : (half8_t)(_Float16)0.0f;
        }
    }
    asm volatile("" ::: "memory");  // every Q load is issued before the block table is read

    // Running state per row block: max (log2 units), this lane's partial sum of p, and O^T in
    // 17 blocks of 16 "dims" (block m < 16: dims 16 m - 4 .. 16 m + 11; block 16: dims 244..255,
    // then 1152 * sum P' in lane group 3, the widening bias of V to remove at the end).
    float m_run[NRB], l_run[NRB];
    float4_t oacc[NRB][17];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
        m_run[rb] = kNegInf;
        l_run[rb] = 0.f;
#pragma unroll
        for (int m = 0; m < 17; ++m) oacc[rb][m] = (float4_t)0.f;
    }

    // ---- block-table slice of the split into LDS ----
    if constexpr (kEarly) {
        // the wave's own blocks (two per tile) are staged in its part of the table
        const int nblk = 2 * nt;
        pt.in_lds = nblk <= kBtWave;
        // block j of this wave: the first key of its 16-key block clamped into the tile's visible
        // keys (the tile_src rule), and that key's page
        auto wave_block = [&](int j, int& key0, int& lb) {
            const int kb = tile_of(j >> 1) * kTile;
            const int kfirst = max(kb, lo), klast = min(kb + kTile - 1, hi - 1);
            key0 = min(max(kb + 16 * (j & 1), kfirst), klast) & ~15;
            lb = a.bs_shift >= 0 ? key0 >> a.bs_shift : key0 / a.block_size;
        };
        // (0) the block-table entries of this wave's first two tiles (scalar loads), requested
        //     before any copy so that they do not queue behind the kernel's first copies
        //     (all four entries in one round trip; the tile_src rule, keys clamped into the tile's
        //     visible range, which also keeps the entries of a missing tile in bounds)
        int key0[4], lb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int kb = tile_of(i >> 1) * kTile;
            const int kfirst = max(kb, lo), klast = min(kb + kTile - 1, hi - 1);
            key0[i] = min(max(kb + 16 * (i & 1), kfirst), klast) & ~15;
            lb[i] = a.bs_shift >= 0 ? key0[i] >> a.bs_shift : key0[i] / a.block_size;
        }
        int ent[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) ent[i] = pt.glob[lb[i]];
        TileSrc src0, src1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int8_t* base = gbase + (int64_t)ent[i] * a.k_sb + (int64_t)(key0[i] - lb[i] * a.block_size) * a.k_ss;
            if (i < 2)
                src0.base[i] = base;
            else
                src1.base[i - 2] = base;
        }
        // (1) Q rows (two 512-byte rows per copy; rows past R repeat row R - 1), spread over the
        //     waves, and the raw block-table entries of each wave's blocks
        const int nq = (R + 1) / 2;
        for (int i = w; i < nq; i += kWaves) {
            const int r = min(2 * i + (l >> 5), R - 1);
            const int qi = r / G, qh = r - qi * G;
            const _Float16* qrow = a.q + (int64_t)(q0 + qi) * a.q_st + (int64_t)(g * G + qh) * kDim;
            const int qdst = kQInSlots ? (2 * i / 16) * kWaveLds + kSlot + kImgV + (2 * i % 16) * (2 * kDim)
                                       : kLdsQ + 1024 * i;
            dma16_v<0>(reinterpret_cast<const int8_t*>(qrow) + 16 * (l & 31), lds_base + (unsigned)qdst);
        }
        if (pt.in_lds) {
            const int* bt_glob = a.block_table + (int64_t)b * a.bt_stride;
            for (int j0 = 0; j0 < nblk; j0 += 64) {
                if (j0 + l < nblk) {  // lanes past the wave's blocks write nothing
                    int key0, lb;
                    wave_block(j0 + l, key0, lb);
                    dma4_v(bt_glob + lb, lds_base + (unsigned)(kLdsRaw + 4 * (w * kBtWave + j0)));
                }
            }
        }
        // (2) this wave's first tile
        if (nt > 0) issue_tile<kFast>(a, src0, dl, wslots, l);
        // the K blocks of the second tile follow at once, its other copies after the set-up
        if (nt > 1) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                dma16_s(src1.base[i >> 2] + (int64_t)(4 * (i & 3)) * a.k_ss, dl.kvo, wslots + kSlot + kImgK + i * kBlk);
        }
        // (3) wait for (1) only
        if (nt > 1)
            wait_vm<25>();
        else if (nt > 0)
            wait_vm<17>();
        else
            wait_vm<0>();
        __syncthreads();
        if (pt.in_lds) {  // the wave's own entries have landed (the wait above): row offsets
            const lds_int* raw = (const lds_int*)(L + kLdsRaw) + w * kBtWave;
            lds_u64* dst = (lds_u64*)(L + kLdsBt) + w * kBtWave;
            for (int j = l; j < nblk; j += 64) {
                int key0, lb;
                wave_block(j, key0, lb);
                dst[j] = (uint64_t)((int64_t)raw[j] * a.k_sb + (int64_t)(key0 - lb * a.block_size) * a.k_ss);
            }
        }
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            const lds_u8* qrow = kQInSlots ? L + rb * kWaveLds + kSlot + kImgV + li * (2 * kDim)
                                           : L + kLdsQ + (16 * rb + li) * (2 * kDim);
#pragma unroll
            for (int st = 0; st < 8; ++st) {
                const int dim = 64 * (st >> 1) + 16 * lg + 8 * (st & 1);
                const half8_t v = *(const lds_half8*)(qrow + 2 * dim);
                qop[rb][st] = rvalid[rb] ? v : (half8_t)(_Float16)0.0f;
            }
        }
        __syncthreads();  // the block offsets are visible
        if (nt > 1) {
            const unsigned slot = wslots + (unsigned)kSlot;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                dma16_s(src1.base[i >> 2] + (int64_t)(i & 3) * a.k_ss, dl.vvo, slot + kImgV + i * kBlk);
            const int64_t delta = src1.base[1] - src1.base[0];
            dma16_v<0>(src1.base[0] + (delta & -(int64_t)dl.tsel) + dl.toff, slot + kImgT);
        }
    } else {
        const int pk_first = max(tb * kTile, lo), pk_last = min(te * kTile, hi) - 1;
        const int* bt_glob = a.block_table + (int64_t)b * a.bt_stride;
        if constexpr (kFast) {
            // byte offset (from this kv head's base) of the first row of every 16-key block of
            // the split, two per tile; blocks outside [lo, hi) point at a visible block of the tile
            const int nblk = 2 * (te - tb);
            pt.in_lds = nblk <= kBtCache;
            if (pt.in_lds) {
                lds_u64* dst = (lds_u64*)(L + kLdsBt);
                for (int i = tid; i < nblk; i += kThreads) {
                    const int kb = (tb + (i >> 1)) * kTile;
                    const int kfirst = max(kb, lo), klast = min(kb + kTile - 1, hi - 1);
                    const int key0 = min(max(kb + 16 * (i & 1), kfirst), klast) & ~15;
                    const int lb = key0 / a.block_size;
                    dst[i] = (uint64_t)((int64_t)bt_glob[lb] * a.k_sb + (int64_t)(key0 - lb * a.block_size) * a.k_ss);
                }
            }
        } else {
            const int npages = pk_last / a.block_size - pt.pfirst + 1;
            pt.in_lds = npages <= kBtCache;
            if (pt.in_lds) {
                lds_int* dst = (lds_int*)(L + kLdsBt);
                for (int i = tid; i < npages; i += kThreads) dst[i] = bt_glob[pt.pfirst + i];
            }
        }
        __syncthreads();
    }
    {
        const half8_t nb = (half8_t)(_Float16)(-kWidenBias);
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            float4_t acc = (float4_t)0.f;
#pragma unroll
            for (int st = 0; st < 8; ++st) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(nb, qop[rb][st], acc, 0, 0, 0);
            qneg[rb] = acc;
        }
    }

    // ---- per-lane LDS read offsets inside a slot ----
    // K operand (u, c): row 16 u + li, source chunk 4 c + lg
    int kro[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
        kro[c] = kFast ? kImgK + (li >> 2) * kBlk + 256 * (li & 3) + 64 * (c ^ (li & 3)) + 16 * lg
                       : kImgK + (4 * c + lg) * 512 + 16 * li;
    constexpr int kKroU = kFast ? 4 * kBlk : 256;  // + for key block u = 1
    // transposed V reads: lane pair (2 i, 2 i + 1) of a 16-lane group names tile row tkey
    const int tslot = li >> 1;
    const int tkey = tslot < 4 ? 4 * lg + tslot : 16 + 4 * lg + (tslot - 4);
    const int th = 8 * (li & 1);
    // chunk m of row tkey: fast: block (tkey & 3) + 4 (tkey >> 4), slot lg, position m ^ 8 (lg & 1)
    const int vblk = kImgV + ((tkey & 3) + 4 * (tkey >> 4)) * kBlk + 256 * lg + th;
    const int vro_lo = kFast ? vblk + ((lg & 1) ? 128 : 0) : kImgV + 16 * tkey + th;   // chunks 0..7
    const int vro_hi = kFast ? vblk - ((lg & 1) ? 128 : 0) : kImgV + 16 * tkey + th;   // chunks 8..15
    constexpr int kVroStep = kFast ? 16 : 512;
    const int tpos = kFast ? (tkey < 16 ? tkey : 16 + ((tkey - 16) ^ 8)) : tkey;
    const int vro_t = kImgT + 16 * tpos + th;
    // scales of this lane's keys 16 u + 4 lg + j: k_scale = first word of V chunk 0, v_scale
    // the last word of the tail
    int kso[2], vso[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int t0 = 16 * u + 4 * lg;
        kso[u] = kFast ? kImgV + (4 * u) * kBlk + 256 * lg + ((lg & 1) ? 128 : 0) : kImgV + 16 * t0;
        const int tp0 = kFast ? (u == 0 ? t0 : 16 + ((t0 - 16) ^ 8)) : t0;
        vso[u] = kImgT + 16 * tp0 + 12;
    }
    constexpr int kKsoStep = kFast ? kBlk : 16;  // + per j

    int tile_cur = tb;  // the tile being computed

    // ---- S^T = K Q^T for every row block (the accumulator starts at -1152 sum q, the widening
    //      bias of K), times k_scale, relative to the running max: sv = s - m (log2 units; s itself
    //      while a row has no max yet); masked scores are -inf. Returns whether some row has to
    //      raise its max: its tile max exceeds the running max by more than kLazy, or it has none ----
    auto tile_scores = [&](const TileOps& o, float (&sv)[NRB][8], bool& interior) __attribute__((always_inline)) {
        float4_t sacc[NRB][2];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint4_t* kr = o.k[c];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const half8_t kf = hh == 0 ? widen_i8x8(kr[u].x, kr[u].y) : widen_i8x8(kr[u].z, kr[u].w);
#pragma unroll
                    for (int rb = 0; rb < NRB; ++rb)
                        sacc[rb][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            kf, qop[rb][2 * c + hh], (c | hh) ? sacc[rb][u] : qneg[rb], 0, 0, 0);
                }
            }
        }
        float ks[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) ks[e] = o.ks[e] * a.scale_log2;
        const int kb = tile_cur * kTile;
        // Interior tile: every key is visible to every row (padding rows have Q = 0 and are
        // never written out), so no per-element mask is needed.
        interior = kb >= lo && kb + kTile <= hi;
        if (a.causal) interior = interior && kb + kTile - 1 <= ctx0;
        if (a.window > 0) interior = interior && (ctx0 + ql - 1) - kb < a.window;
        bool need = false;
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            const bool fresh = m_run[rb] == kNegInf;
            const float nm = fresh ? 0.f : -m_run[rb];
            float mx = kNegInf;
            if (interior) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    sv[rb][e] = __builtin_fmaf(sacc[rb][e >> 2][e & 3], ks[e], nm);
                    mx = fmaxf(mx, sv[rb][e]);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int t = kb + 16 * (e >> 2) + 4 * lg + (e & 3);
                    const int rp = rpos[rb];
                    const bool vis = rvalid[rb] & (t >= lo) & (t < hi) & (!a.causal | (t <= rp)) &
                                     ((a.window <= 0) | ((rp - t) < a.window));
                    sv[rb][e] = vis ? __builtin_fmaf(sacc[rb][e >> 2][e & 3], ks[e], nm) : kNegInf;
                    mx = fmaxf(mx, sv[rb][e]);
                }
            }
            need |= fresh ? mx > kNegInf : mx > kLazy;
        }
        return need;
    };

    // rare path: raise the running max of the rows that need it, shift their relative scores and
    // rescale their state
    // With three row blocks the rescale goes through LDS (4 KiB of scratch in V blocks 4..7 of
    // the current tile's slot: its operands are all in registers by now, and only the K image and
    // V blocks 0..3 can already be refilling): the accumulators are then only ever
    // touched by MFMAs and by asm with AGPR operands, so the compiler keeps them in the AGPR
    // file (multiplying them in place made it spill ~250 registers, partly in the fast loop).
    // With fewer row blocks the registers suffice and the multiply in place is faster.
    auto raise_max = [&](float (&sv)[NRB][8], lds_u8* scr_slot) __attribute__((always_inline)) {
        const unsigned scr = (unsigned)(uintptr_t)(scr_slot + 16 * l);
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            float mloc = kNegInf;
#pragma unroll
            for (int e = 0; e < 8; ++e) mloc = fmaxf(mloc, sv[rb][e]);
            const float mrow = xor_max(xor_max(mloc, 16), 32);  // tile max, relative to m_run
            const bool fresh = m_run[rb] == kNegInf;
            const bool raise = fresh ? mrow > kNegInf : mrow > kLazy;
            const float shift = raise ? mrow : 0.f;
            const float alpha = fresh ? 0.f : __builtin_amdgcn_exp2f(-shift);
            if (raise) m_run[rb] = fresh ? mrow : m_run[rb] + mrow;
#pragma unroll
            for (int e = 0; e < 8; ++e) sv[rb][e] -= shift;
            l_run[rb] *= alpha;
            // O is still zero while every row of the block is fresh: skip the rescale then
            if (__builtin_amdgcn_ballot_w64(!fresh) != 0) {
                if constexpr (NRB >= 3) {
#pragma unroll
                    for (int m = 0; m < 16; m += 4)
                        agpr_scale4_via_lds(oacc[rb][m], oacc[rb][m + 1], oacc[rb][m + 2], oacc[rb][m + 3], alpha, scr);
                    agpr_scale_via_lds(oacc[rb][16], alpha, scr);
                } else {
#pragma unroll
                    for (int m = 0; m < 17; ++m) oacc[rb][m] *= alpha;
                }
            }
        }
    };

    // ---- p = 2^sv; P' = p * v_scale * 16 as two fp16 parts (hi + lo, ~22 significant bits: a
    //      single fp16 would put 2^-12 relative error on every term, too much next to outlier V
    //      rows); then O^T += V^T hi^T + V^T lo^T for every row block ----
    auto tile_values = [&](const TileOps& o, const float (&sv)[NRB][8], bool interior) __attribute__((always_inline)) {
        float vsc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) vsc[e] = o.vs[e] * kPScale;
        if (!interior) {  // outside [lo, hi) a scale may be garbage or NaN: use 0
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int t = tile_cur * kTile + 16 * (e >> 2) + 4 * lg + (e & 3);
                vsc[e] = (t >= lo) & (t < hi) ? vsc[e] : 0.f;
            }
        }
        half8_t phi[NRB], plo[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            float psum = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float p = __builtin_amdgcn_exp2f(sv[rb][e]);  // masked: 2^-inf = 0
                psum += p;
                const _Float16 h = (_Float16)(p * vsc[e]);
                phi[rb][e] = h;
                plo[rb][e] = (_Float16)__builtin_fmaf(p, vsc[e], -(float)h);
            }
            l_run[rb] += psum;
        }
#pragma unroll
        for (int m = 0; m < 17; ++m) {
            const half8_t vf = widen_i8x8((unsigned)o.v[m].x, (unsigned)o.v[m].y);
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb)
                oacc[rb][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, phi[rb], oacc[rb][m], 0, 0, 0);
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb)
                oacc[rb][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, plo[rb], oacc[rb][m], 0, 0, 0);
        }
    };

    // ---- every operand of a tile from its slot into registers, so the slot can be refilled
    //      before the tile is computed: v_scale of this lane's keys (then the v_scale words of the
    //      slot are cleared: that MFMA output row of the tail block becomes 1152 * sum P'), the K
    //      operand, k_scale, and the 17 transposed V reads ----
    auto read_ops = [&](lds_u8* T, TileOps& o) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) o.vs[4 * u + j] = *(const lds_float*)(T + vso[u] + 16 * j);
        if (l < 32) *(lds_float*)(T + kImgT + 16 * l + 12) = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u) o.k[c][u] = *(const lds_uint4*)(T + kro[c] + u * kKroU);
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) o.ks[4 * u + j] = *(const lds_float*)(T + kso[u] + j * kKsoStep);
#pragma unroll
        for (int m = 0; m < 17; ++m) {
            const int ofs = m < 8 ? vro_lo + kVroStep * m : (m < 16 ? vro_hi + kVroStep * m : vro_t);
            o.v[m] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_int2*)(T + ofs));
        }
    };

    // ---- the tile stream of this wave ----
    auto tile_loop = [&](auto lds_flag) __attribute__((always_inline)) {
        constexpr bool kLds = decltype(lds_flag)::value;
        auto issue = [&](int n) __attribute__((always_inline)) {
            wait_lds();  // every LDS access to the slot being refilled has completed
            issue_tile<kFast>(a, tile_src<kFast, kLds>(a, pt, gbase, tile_of(n), n, lo, hi, l), dl,
                              wslots + (unsigned)((n & 1) * kSlot), l);
        };
        // The same copies in two parts (16-key row blocks): the 8 K blocks, then the 8 V blocks
        // and the tail, from the addresses the first part looked up.
        TileSrc nsrc;
        auto issue_k = [&](int n) __attribute__((always_inline)) {
            wait_lds();  // every LDS access to the slot being refilled has completed
            nsrc = tile_src<kFast, kLds>(a, pt, gbase, tile_of(n), n, lo, hi, l);
            const unsigned slot = wslots + (unsigned)((n & 1) * kSlot);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                dma16_s(nsrc.base[i >> 2] + (int64_t)(4 * (i & 3)) * a.k_ss, dl.kvo, slot + kImgK + i * kBlk);
        };
        // While the stream ramps up (the refills of its first kRampTiles tiles) the first four V
        // blocks go between the scores and the values, the rest after the values.
        constexpr int kRampTiles = 2;
        auto ramp = [&](int n) { return n - 2 < kRampTiles; };  // refill n is issued by iteration n - 2
        auto issue_v0 = [&](int n) __attribute__((always_inline)) {
            const unsigned slot = wslots + (unsigned)((n & 1) * kSlot);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                dma16_s(nsrc.base[i >> 2] + (int64_t)(i & 3) * a.k_ss, dl.vvo, slot + kImgV + i * kBlk);
        };
        auto issue_v = [&](int n) __attribute__((always_inline)) {
            const unsigned slot = wslots + (unsigned)((n & 1) * kSlot);
            if (!ramp(n)) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    dma16_s(nsrc.base[i >> 2] + (int64_t)(i & 3) * a.k_ss, dl.vvo, slot + kImgV + i * kBlk);
            }
#pragma unroll
            for (int i = 4; i < 8; ++i)
                dma16_s(nsrc.base[i >> 2] + (int64_t)(i & 3) * a.k_ss, dl.vvo, slot + kImgV + i * kBlk);
            const int64_t delta = nsrc.base[1] - nsrc.base[0];
            dma16_v<0>(nsrc.base[0] + (delta & -(int64_t)dl.tsel) + dl.toff, slot + kImgT);
        };
        // The first two tiles (issued during the set-up when kEarly): all loads the compiler can
        // see (Q, block table) have been waited for by now, so no compiler-inserted wait will
        // include these copies.
        if constexpr (!kEarly) {
            if (nt > 0) issue(0);
            if (nt > 1) issue(1);
        }
        float sv[NRB][8];
        TileOps ops;
        bool interior = true;
        int n = 0;
        // The fast inner loop never rescales: O stays in the MFMA accumulators, untouched by
        // the vector ALU. When some row's max must be raised the loop is left, the rows are
        // rescaled, the tile is finished and the loop resumes with the next tile.
        while (n < nt) {
            bool rare = false;
            for (; n < nt; ++n) {
                if (n + 1 < nt)
                    wait_vm<17>();  // tile n has landed; tile n + 1 may still be in flight
                else
                    wait_vm<0>();
                lds_u8* T = L + w * kWaveLds + (n & 1) * kSlot;
                tile_cur = tile_of(n);
                read_ops(T, ops);
                if (kFast && n + 2 < nt) issue_k(n + 2);
                const bool need = tile_scores(ops, sv, interior);
                if (kFast && n + 2 < nt && ramp(n + 2)) issue_v0(n + 2);
                if (__builtin_amdgcn_ballot_w64(need) != 0) {
                    rare = true;
                    break;
                }
                tile_values(ops, sv, interior);
                if (n + 2 < nt) {
                    if constexpr (kFast)
                        issue_v(n + 2);
                    else
                        issue(n + 2);
                }
            }
            if (!rare) break;
            raise_max(sv, L + w * kWaveLds + (n & 1) * kSlot + kImgV + 4 * kBlk);
            tile_values(ops, sv, interior);
            if (n + 2 < nt) {
                if constexpr (kFast)
                    issue_v(n + 2);
                else
                    issue(n + 2);
            }
            ++n;
        }
    };
    if (pt.in_lds)
        tile_loop(std::true_type{});
    else
        tile_loop(std::false_type{});

    // ---- merge the waves through LDS and write one partial per row ----
    {
        // Each wave stores its accumulators as they are (a 1 KiB block per accumulator and row
        // block, straight from the AGPRs: no vector ALU work) into its own slots as soon as its
        // tiles are done, with its per-row max, sum and V widening bias; then thread (row, 32
        // dims) derives the wave factors of its row, sums the four waves' blocks with them and
        // writes the partial row. Row blocks go through the slots two at a time (kRawRounds
        // rounds).
        constexpr int kRawRounds = (NRB + 1) / 2;
        float* wm = reinterpret_cast<float*>(lds + kLdsStats);  // [wave][NRB][16] running max
        float* wl = wm + kWaves * NRB * 16;                     // [wave][NRB][16] row sum of p
        float* wc = reinterpret_cast<float*>(lds + kLdsMergeC);  // [wave][NRB][16] 1152 sum P'
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            const float l_row = xor_sum(xor_sum(l_run[rb], 16), 32);
            const float cr = __shfl(oacc[rb][16].x, 48 + li, 64);  // 1152 * sum of the row's P'
            if (lg == 0) {
                wm[(w * NRB + rb) * 16 + li] = m_run[rb];
                wl[(w * NRB + rb) * 16 + li] = l_row;
                wc[(w * NRB + rb) * 16 + li] = cr;
            }
        }
        const unsigned raw = lds_base + (unsigned)(w * kWaveLds + 16 * l);  // this wave's slots
        auto store_round = [&](int rd) __attribute__((always_inline)) {
#pragma unroll
            for (int rb = 2 * rd; rb < 2 * rd + 2 && rb < NRB; ++rb)
#pragma unroll
                for (int m = 0; m < 17; ++m)
                    asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(raw), "a"(oacc[rb][m]),
                                 "i"(((rb - 2 * rd) * 17 + m) * 1024)
                                 : "memory");
        };
        store_round(0);
        wait_lds();
        __syncthreads();  // every wave's stats and first accumulator blocks are in LDS
#pragma unroll
        for (int rd = 0; rd < kRawRounds; ++rd) {
            if (rd > 0) {
                store_round(rd);
                wait_lds();
                __syncthreads();
            }
            // thread: row 32 rd + (lane & 31), wave w's two 32-dim parts. Row factors: M =
            // max_w m_w, e_w = 2^(m_w - M), O = sum_w e_w O_w / 16 - sum_w e_w C_w / 16, L =
            // sum_w e_w l_w. Dims d of an accumulator block: block m < 16 holds 16 m - 4 + 4 lg
            // .. + 3 in lane group lg, block 16 holds 252..255 in lane group 2
            const int row = 32 * rd + (l & 31), part = 2 * w + (l >> 5);
            if (row < R) {
                float M = kNegInf;
#pragma unroll
                for (int v = 0; v < kWaves; ++v) M = fmaxf(M, wm[v * NRB * 16 + row]);
                float f[kWaves], C = 0.f, Lr = 0.f;
#pragma unroll
                for (int v = 0; v < kWaves; ++v) {
                    const float mw = wm[v * NRB * 16 + row];
                    const float e = mw == kNegInf ? 0.f : exp2f(mw - M);
                    f[v] = e * (1.0f / kPScale);
                    C += f[v] * wc[v * NRB * 16 + row];
                    Lr += e * wl[v * NRB * 16 + row];
                }
                const int64_t pr = prow(row);
                if (part == 0) {
                    a.part_m[pr] = M;
                    a.part_l[pr] = Lr;
                }
                const int rbl = (row >> 4) - 2 * rd;  // row block within the round
                float* dst = a.part_o + pr * kDim;
                const float4_t* rawp = reinterpret_cast<const float4_t*>(lds);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int d = 32 * part + 4 * j;
                    const int m = d < 252 ? (d + 4) >> 4 : 16;
                    const int glg = d < 252 ? ((d + 4) >> 2) & 3 : 2;
                    const int blk = (rbl * 17 + m) * 64 + 16 * glg + (row & 15);
                    float4_t acc = (float4_t)(-C);
#pragma unroll
                    for (int v = 0; v < kWaves; ++v) acc += rawp[v * (kWaveLds / 16) + blk] * f[v];
                    *reinterpret_cast<float4_t*>(dst + d) = acc;
                }
            }
            if (rd + 1 < kRawRounds) __syncthreads();  // the blocks are rewritten for the next round
        }
    }
}

__device__ __forceinline__ float wave_max64(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Log-sum-exp merge of the split partials (pth_dec.cu:245-283 semantics): M = max_p m_p,
// L = sum_p 2^(m_p - M) l_p, out = sum_p 2^(m_p - M) O_p / L, and 0 when L == 0. Grid
// (num_tokens, heads_q, 64 / kCols): each workgroup merges 4 kCols dims of one (token, head)
// row. Thread (sg = tid / kCols, c = tid % kCols) owns float4 column c of segments sg, sg +
// 256 / kCols, ...; all partial loads of the first 64 segments are issued before the one
// barrier that publishes M, so the merge costs one memory round trip.
template <int kCols>  // float4 columns per workgroup: 16 (a 64-dim quarter) or 32 (a half row)
__global__ void __launch_bounds__(256) pd_combine_kernel(const CombineParams a) {
    constexpr int kGroups = 256 / kCols;  // segment groups
    constexpr int kCombPer = 64 / kGroups;  // segments per thread in the first pass
    __shared__ float s_red[4];
    __shared__ float s_l[4];
    __shared__ float4_t s_acc[4][kCols];
    const int tok = blockIdx.x, head = blockIdx.y, quarter = blockIdx.z, Hq = gridDim.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = tid % kCols, sg = tid / kCols;

    // The partial loads go out first: they are in bounds for every (token, head) of the grid, and
    // the sequence lookup below (two dependent small loads) then overlaps their latency.
    const int64_t base = ((int64_t)tok * Hq + head) * a.nseg;
    const float* pm = a.part_m + base;
    const float* pl = a.part_l + base;
    const float4_t* po = reinterpret_cast<const float4_t*>(a.part_o + base * kDim + quarter * 4 * kCols) + c;

    float mv[kCombPer], lv[kCombPer];
    float4_t ov[kCombPer];
#pragma unroll
    for (int i = 0; i < kCombPer; ++i) {
        const int sgi = sg + kGroups * i;
        const bool ok = sgi < a.nsplit;
        mv[i] = ok ? pm[sgi] : kNegInf;
        lv[i] = ok ? pl[sgi] : 0.f;
        ov[i] = ok ? po[(int64_t)sgi * (kDim / 4)] : (float4_t)0.f;
    }

    // sequence of this token = number of sequences whose query rows end at or before it; the
    // lookup only gates the final store, so its loads overlap the merge (the merge of a padding
    // token reads allocated but unwritten partials and is discarded)
    int b = 0;
    for (int i0 = 0; i0 < a.num_seqs; i0 += 64) {
        const int i = i0 + lane + 1;
        const bool ended = i <= a.num_seqs && a.qsl[i] <= tok;
        b += __popcll(__ballot(ended));
    }
    const int bq = min(b, a.num_seqs - 1);
    const int q_b = a.qsl[bq], len_b = a.seq_lens[bq];
    const bool live = b < a.num_seqs && tok >= q_b && len_b > 0 && tok - q_b < a.qmax;
    float mx = kNegInf;
#pragma unroll
    for (int i = 0; i < kCombPer; ++i) mx = fmaxf(mx, mv[i]);
    for (int p = tid + kGroups * kCombPer; p < a.nsplit; p += 256) mx = fmaxf(mx, pm[p]);
    mx = wave_max64(mx);
    if (lane == 0) s_red[wave] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));

    float lsum = 0.f;
    float4_t acc = (float4_t)0.f;
    if (M != kNegInf) {
#pragma unroll
        for (int i = 0; i < kCombPer; ++i) {
            const float w = mv[i] != kNegInf ? exp2f(mv[i] - M) : 0.f;
            lsum += w * lv[i];
            acc += w != 0.f ? w * ov[i] : (float4_t)0.f;  // empty splits leave part_o unwritten
        }
        for (int p = sg + kGroups * kCombPer; p < a.nsplit; p += kGroups) {
            const float mp = pm[p];
            const float w = mp != kNegInf ? exp2f(mp - M) : 0.f;
            if (w != 0.f) {
                lsum += w * pl[p];
                acc += w * po[(int64_t)p * (kDim / 4)];
            }
        }
    }
    // reduce over the 16 segment slots: xor 16 / 32 inside the wave, then across the 4 waves
#pragma unroll
    for (int o = kCols; o <= 32; o <<= 1) {
        lsum += __shfl_xor(lsum, o, 64);
        acc.x += __shfl_xor(acc.x, o, 64);
        acc.y += __shfl_xor(acc.y, o, 64);
        acc.z += __shfl_xor(acc.z, o, 64);
        acc.w += __shfl_xor(acc.w, o, 64);
    }
    if (lane < kCols) s_acc[wave][lane] = acc;
    if (lane == 0) s_l[wave] = lsum;
    __syncthreads();
    if (live && tid < kCols) {
        const float4_t r = s_acc[0][tid] + s_acc[1][tid] + s_acc[2][tid] + s_acc[3][tid];
        const float L = s_l[0] + s_l[1] + s_l[2] + s_l[3];
        const float inv = L > 0.f ? 1.f / L : 0.f;
        typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
        const half4_t h = {(_Float16)(r.x * inv), (_Float16)(r.y * inv), (_Float16)(r.z * inv),
                           (_Float16)(r.w * inv)};
        _Float16* o = a.out + (int64_t)tok * a.o_st + (int64_t)head * a.o_sh + quarter * 4 * kCols + 4 * tid;
        __builtin_memcpy(o, &h, 8);
    }
}

// ---------------------------------------------------------------------------------------
// Chunked prefill over the same cache (kernels/fa_pth/pth_fa.cpp:41-85 interface): causal
// attention of Sq query tokens per sequence, query token i at absolute position q_abs + i,
// against keys [0, seq_len). One workgroup takes tok_per_wg query tokens of one sequence and all
// G heads of one kv head (kFaRows = 192 rows, 48 per wave as 3 row blocks of 16) and streams
// every visible 32-key tile once:
//   HBM -> LDS   each wave copies a quarter of every tile into a 4-slot ring, 4 tiles ahead;
//   int8 -> fp16 each wave widens a quarter of tile n + 1 (K operands, transposed V operands,
//                the tile's scales) into one of two fp16 buffers while it computes tile n;
//   MFMA         S^T = K Q^T and O^T += V^T P^T on fp16 MFMA with fp32 accumulation, Q held in
//                registers, K and V operands read from the fp16 buffer.
// One barrier per tile orders the three stages. There is no split: each row is normalised in
// registers and stored once. Q arrives as fp32 and is rounded to fp16 for the MFMA.
constexpr int kFaWaves = 4;
constexpr int kFaRB = 3;                        // row blocks per wave
constexpr int kFaRows = kFaWaves * kFaRB * 16;  // 192
constexpr int kFaRaw = 4;                       // raw (int8) tile slots
constexpr int kFaHK = 16 * 1024;                // fp16 K operands: (32-dim step, 16-key block) x 1 KiB
constexpr int kFaHV = 17 * 1024;                // fp16 V^T operands: 17 16-dim blocks x 1 KiB
constexpr int kFaHS = 256;                      // k_scale * scale * log2(e) [32], v_scale [32]
constexpr int kFaHBuf = kFaHK + kFaHV + kFaHS;
constexpr int kFaBt = 6144;                     // 16-key blocks (or pages) of the LDS block table

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
};

// The quarter `part` of a tile's 17 copies: K blocks 2 part, 2 part + 1, V blocks 2 part,
// 2 part + 1, and the tail for part 3.
template <bool kFast, int kPart, class P>
__device__ __forceinline__ void issue_quarter(const P& a, const TileSrc& src, const DmaLane& d, unsigned slot,
                                              int lane) {
    if constexpr (kFast) {
#pragma unroll
        for (int i = 2 * kPart; i < 2 * kPart + 2; ++i) {
            const int8_t* kb = src.base[i >> 2] + (int64_t)(4 * (i & 3)) * a.k_ss;
            dma16_s(kb, d.kvo, slot + kImgK + i * kBlk);
        }
#pragma unroll
        for (int i = 2 * kPart; i < 2 * kPart + 2; ++i) {
            const int8_t* vb = src.base[i >> 2] + (int64_t)(i & 3) * a.k_ss;
            dma16_s(vb, d.vvo, slot + kImgV + i * kBlk);
        }
        if constexpr (kPart == 3) {
            const int64_t delta = src.base[1] - src.base[0];
            dma16_v<0>(src.base[0] + (delta & -(int64_t)d.tsel) + d.toff, slot + kImgT);
        }
    } else {
        const int8_t* row = src.base[0];  // tile row lane & 31
        const int8_t* p = row + 16 * (lane >> 5);
        dma16_v<64 * kPart>(p, slot + kImgK + (2 * kPart) * 1024);
        dma16_v<64 * kPart + 32>(p, slot + kImgK + (2 * kPart + 1) * 1024);
        dma16_v<256 + 64 * kPart>(p, slot + kImgV + (2 * kPart) * 1024);
        dma16_v<256 + 64 * kPart + 32>(p, slot + kImgV + (2 * kPart + 1) * 1024);
        if constexpr (kPart == 3) dma16_v<504>(row, slot + kImgT);
    }
}

// Wait until at most `later` tiles' copies of this wave (4 per tile, 5 for wave 3) are in flight.
__device__ __forceinline__ void wait_quarters(int later, bool tail) {
    if (tail) {
        if (later >= 2)
            wait_vm<10>();
        else if (later == 1)
            wait_vm<5>();
        else
            wait_vm<0>();
    } else {
        if (later >= 2)
            wait_vm<8>();
        else if (later == 1)
            wait_vm<4>();
        else
            wait_vm<0>();
    }
}

template <bool kFast>
__global__ void __launch_bounds__(kFaWaves * 64, 1) pd_prefill_kernel(const FaParams a) {
    constexpr int kLdsRaw = 0;
    constexpr int kLdsH = kLdsRaw + kFaRaw * kSlot;
    constexpr int kLdsBt = kLdsH + 2 * kFaHBuf;
    constexpr int kLdsBytes = kLdsBt + kFaBt * 4;
    static_assert(kLdsBytes <= 160 * 1024, "gfx950 has 160 KiB of LDS per CU");
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];

    // Workgroups are dispatched to the 8 XCDs round robin (linear id L to XCD L % 8), and each XCD
    // has its own L2. Every query tile of a (sequence, kv head) streams the same keys, so the
    // logical workgroup index (query tile fastest) is laid out XCD by XCD: XCD x takes a
    // contiguous range of it, and the query tiles sharing a kv head mostly share an L2 (config 5:
    // each kv head's 64 query tiles on two XCDs).
    const unsigned nx = gridDim.x, ny = gridDim.y, nwg = nx * ny * gridDim.z;
    const unsigned lin = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
    const unsigned xcd = lin % 8u;
    const unsigned lidx = xcd * (nwg / 8u) + min(xcd, nwg % 8u) + lin / 8u;
    const int qt = (int)(lidx % nx), g = (int)((lidx / nx) % ny), b = (int)(lidx / (nx * ny));
    const int tid = threadIdx.x, l = tid & 63, lg = l >> 4, li = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = a.G;
    const int tq0 = qt * a.tok_per_wg;                 // first query token of the workgroup
    const int ntok = min(a.tok_per_wg, a.Sq - tq0);    // query tokens of the workgroup
    const int seq_len = a.seq_lens[b];
    const int qabs = a.q_abs[b];
    // keys any row can see: [0, min(seq_len, last row's position + 1))
    const int hi = min(seq_len, qabs + tq0 + ntok);
    const int ntiles = hi > 0 ? (hi - 1) / kTile + 1 : 0;
    const int pmin = qabs + tq0;                       // smallest row position

    // ---- rows of this wave: row r = 48 w + 16 rb + li -> (token r / G, head r % G) ----
    half8_t qop[kFaRB][8];
    float qneg[kFaRB];  // -1152 * sum_d q[row, d]: the K widening bias, the same for every key
    bool rvalid[kFaRB];
    int rpos[kFaRB];
#pragma unroll
    for (int rb = 0; rb < kFaRB; ++rb) {
        const int r = 48 * w + 16 * rb + li;
        const int tok = r / G, hh = r - (r / G) * G;
        rvalid[rb] = tok < ntok && r < a.tok_per_wg * G;
        rpos[rb] = qabs + tq0 + tok;
        const float* qrow = a.q + (int64_t)b * a.q_sb + (int64_t)(g * G + (rvalid[rb] ? hh : 0)) * a.q_sh +
                            (int64_t)(tq0 + (rvalid[rb] ? tok : 0)) * a.q_st;
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            const int dim = 64 * (st >> 1) + 16 * lg + 8 * (st & 1);
            const float4_t x0 = *reinterpret_cast<const float4_t*>(qrow + dim);
            const float4_t x1 = *reinterpret_cast<const float4_t*>(qrow + dim + 4);
            // Q is rounded to fp16 unscaled: fp16-valued queries enter the matrix cores exactly
            const half8_t v = {(_Float16)x0.x, (_Float16)x0.y, (_Float16)x0.z, (_Float16)x0.w,
                               (_Float16)x1.x, (_Float16)x1.y, (_Float16)x1.z, (_Float16)x1.w};
            qop[rb][st] = rvalid[rb] ? v : (half8_t)(_Float16)0.0f;
        }
    }
    asm volatile("" ::: "memory");  // every Q load is issued before the block table is read

    lds_u8* L = (lds_u8*)lds;
    const unsigned lds_base = (unsigned)(uintptr_t)L;
    const int8_t* gbase = a.kc + (int64_t)g * a.k_sh;
    DmaLane dl;
    {
        const int qq = l >> 4, c16 = l & 15, p = l & 31;
        dl.kvo = (unsigned)(qq * a.k_ss) + 16u * (unsigned)(c16 ^ (4 * qq));
        dl.vvo = (unsigned)(4 * qq * a.k_ss) + 256u + 16u * (unsigned)(c16 ^ (8 * (qq & 1)));
        const int rr = p < 16 ? p : ((p - 16) ^ 8);
        dl.toff = kFast ? (unsigned)(rr * a.k_ss) + 504u : 0u;
        dl.tsel = p >> 4;
    }

    // ---- block table of the workgroup's keys into LDS: for bs % 16 == 0 the byte offset / 8 of
    //      every 16-key block's first row, else the page numbers ----
    const_int_ptr bt_row = (const_int_ptr)(uintptr_t)(a.block_table + (int64_t)b * a.bt_stride);
    PageTable pt;
    pt.glob = bt_row;
    pt.lds = (const lds_int*)(L + kLdsBt);
    pt.rows16 = nullptr;
    pt.pfirst = 0;
    {
        const int* bt_glob = a.block_table + (int64_t)b * a.bt_stride;
        if constexpr (kFast) {
            const int nblk = 2 * ntiles;
            pt.in_lds = a.bt32 && nblk <= kFaBt;
            if (pt.in_lds) {
                lds_int* dst = (lds_int*)(L + kLdsBt);
                for (int i = tid; i < nblk; i += kFaWaves * 64) {
                    const int kb = (i >> 1) * kTile;
                    const int klast = min(kb + kTile - 1, hi - 1);
                    const int key0 = min(kb + 16 * (i & 1), klast) & ~15;
                    const int lb = key0 / a.block_size;
                    const int64_t off = (int64_t)bt_glob[lb] * a.k_sb + (int64_t)(key0 - lb * a.block_size) * a.k_ss;
                    dst[i] = (int)(unsigned)((uint64_t)off >> 3);
                }
            }
        } else {
            const int npages = hi > 0 ? (hi - 1) / a.block_size + 1 : 0;
            pt.in_lds = npages <= kFaBt;
            if (pt.in_lds) {
                lds_int* dst = (lds_int*)(L + kLdsBt);
                for (int i = tid; i < npages; i += kFaWaves * 64) dst[i] = bt_glob[i];
            }
        }
    }
    {
        const half8_t nb = (half8_t)(_Float16)(-kWidenBias);
#pragma unroll
        for (int rb = 0; rb < kFaRB; ++rb) {
            float4_t acc = (float4_t)0.f;
#pragma unroll
            for (int st = 0; st < 8; ++st) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(nb, qop[rb][st], acc, 0, 0, 0);
            qneg[rb] = acc.x;
        }
    }
    __syncthreads();  // the LDS block table is complete

    // ---- this lane's positions in a raw slot (the decode kernel's layout) ----
    // K operand (32-dim step pair c = this wave's quarter, 16-key block u): 16 source bytes
    const int kro = kFast ? kImgK + (li >> 2) * kBlk + 256 * (li & 3) + 64 * (w ^ (li & 3)) + 16 * lg
                          : kImgK + (4 * w + lg) * 512 + 16 * li;
    constexpr int kKroU = kFast ? 4 * kBlk : 256;
    // transposed V reads: 16-dim block m of this lane's 8 keys
    const int tslot = li >> 1;
    const int tkey = tslot < 4 ? 4 * lg + tslot : 16 + 4 * lg + (tslot - 4);
    const int th = 8 * (li & 1);
    const int vblk = kImgV + ((tkey & 3) + 4 * (tkey >> 4)) * kBlk + 256 * lg + th;
    const int vro_lo = kFast ? vblk + ((lg & 1) ? 128 : 0) : kImgV + 16 * tkey + th;
    const int vro_hi = kFast ? vblk - ((lg & 1) ? 128 : 0) : kImgV + 16 * tkey + th;
    constexpr int kVroStep = kFast ? 16 : 512;
    const int vro_t = kImgT + 16 * (kFast ? (tkey < 16 ? tkey : 16 + ((tkey - 16) ^ 8)) : tkey) + th;
    // scales: lane l < 32 reads k_scale of key l, lane l >= 32 v_scale of key l - 32
    const int sr = l & 31, sq = (sr >> 2) & 3;
    const int sco = l < 32 ? (kFast ? kImgV + (4 * (sr >> 4) + (sr & 3)) * kBlk + 256 * sq + 128 * (sq & 1)
                                    : kImgV + 16 * sr)
                           : kImgT + 16 * (kFast ? (sr < 16 ? sr : 16 + ((sr - 16) ^ 8)) : sr) + 12;
    const float sc_mul = l < 32 ? a.scale_log2 : 1.f;

    // Relative scores carry +kPLog2: p' = 2^(s - m + kPLog2) = 16 p, so P' = p' * v_scale spans the
    // same fp16 range as in the decode kernel; l accumulates p' and the final 1 / l removes it.
    constexpr float kPLog2 = 4.0f;
    float m_run[kFaRB], l_run[kFaRB];
    // per row: the score offset -m_run + kPLog2 (kPLog2 while the row has seen no key) and the
    // relative score above which m_run must be raised (any finite score while fresh)
    float nm_run[kFaRB], thr_run[kFaRB];
    float4_t oacc[kFaRB][17];
#pragma unroll
    for (int rb = 0; rb < kFaRB; ++rb) {
        m_run[rb] = kNegInf;
        l_run[rb] = 0.f;
        nm_run[rb] = kPLog2;
        thr_run[rb] = kNegInf;
#pragma unroll
        for (int m = 0; m < 17; ++m) oacc[rb][m] = (float4_t)0.f;
    }

    typedef __attribute__((address_space(3))) float4_t lds_float4;
    auto hbuf = [&](int n) __attribute__((always_inline)) { return L + kLdsH + (n & 1) * kFaHBuf; };
    auto raw = [&](int n) __attribute__((always_inline)) { return L + kLdsRaw + (n & (kFaRaw - 1)) * kSlot; };

    // ---- widen this wave's quarter of raw tile n into fp16 buffer n & 1: K operands of step
    //      pair c = w, V^T blocks w, w + 4, w + 8, w + 12 (and 16 for wave 0), the scales (wave 1) ----
    // ---- widen this wave's quarter of raw tile n into fp16 buffer n & 1: K operands of step
    //      pair c = w, V^T blocks w, w + 4, w + 8, w + 12 (and 16 for wave 0), the scales (wave 1).
    //      Staged so that the pieces can be spread between the P.V products of the previous tile ----
    struct WidenRegs {
        uint4_t kr[2];
        int2_t vr[5];
        float sc;
    };
    auto widen_load = [&](int n, WidenRegs& r) __attribute__((always_inline)) {
        const lds_u8* R = raw(n);
#pragma unroll
        for (int u = 0; u < 2; ++u) r.kr[u] = *(const lds_uint4*)(R + kro + u * kKroU);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = w + 4 * j;  // wave-uniform
            const int ofs = (m < 8 ? vro_lo : vro_hi) + kVroStep * m;
            r.vr[j] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_int2*)(R + ofs));
        }
        // every wave reads and writes the tail block and the scales: the copies are identical,
        // which costs less than branching on the wave
        r.vr[4] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_int2*)(R + vro_t));
        r.sc = *(const lds_float*)(R + sco);
    };
    // piece j of 0..9: K halves 0..3, V blocks 4..7, the tail block 8, the scales 9
    auto widen_store = [&](int n, const WidenRegs& r, int j) __attribute__((always_inline)) {
        lds_u8* H = hbuf(n);
        if (j < 4) {
            const int u = j >> 1, hh = j & 1;
            const half8_t kf = hh == 0 ? widen_i8x8(r.kr[u].x, r.kr[u].y) : widen_i8x8(r.kr[u].z, r.kr[u].w);
            *(lds_half8*)(H + ((2 * w + hh) * 2 + u) * 1024 + 16 * l) = kf;
        } else if (j < 8) {
            *(lds_half8*)(H + kFaHK + (w + 4 * (j - 4)) * 1024 + 16 * l) =
                widen_i8x8((unsigned)r.vr[j - 4].x, (unsigned)r.vr[j - 4].y);
        } else if (j == 8) {
            // rows 12..15 of the tail block are the v_scale bytes: widened from 0 they are
            // exactly 1152, so O^T rows 252..255 of that block accumulate 1152 * sum of P'
            const int2_t vt = li >= 12 ? int2_t{0, 0} : r.vr[4];
            *(lds_half8*)(H + kFaHK + 16 * 1024 + 16 * l) = widen_i8x8((unsigned)vt.x, (unsigned)vt.y);
        } else {
            // k_scale * scale * log2(e) [32] then v_scale [32]; keys past seq_len may hold garbage
            // scales (even NaN): v_scale 0 makes their P' 0
            const bool dead = l >= 32 && n * kTile + sr >= hi;
            *(lds_float*)(H + kFaHK + kFaHV + 4 * l) = dead ? 0.f : r.sc * sc_mul;
        }
    };
    auto widen = [&](int n) __attribute__((always_inline)) {
        WidenRegs r;
        widen_load(n, r);
#pragma unroll
        for (int j = 0; j < 10; ++j) widen_store(n, r, j);
    };


    // ---- front half of tile n: S^T = K Q^T from fp16 buffer n & 1 (widening tile n + 1 in
    //      between), relative scores; true when some row's running max must be raised.
    //      kMasked: the tile crosses the causal diagonal or seq_len ----
    auto tile_front = [&](auto masked_flag, int n, float (&sv)[kFaRB][8], float (&vs)[8])
        __attribute__((always_inline)) {
        constexpr bool kMasked = decltype(masked_flag)::value;
        const lds_u8* H = hbuf(n);
        float ks[8];
        {
            const float4_t k0 = *(const lds_float4*)(H + kFaHK + kFaHV + 16 * lg);
            const float4_t k1 = *(const lds_float4*)(H + kFaHK + kFaHV + 64 + 16 * lg);
            const float4_t v0 = *(const lds_float4*)(H + kFaHK + kFaHV + 128 + 16 * lg);
            const float4_t v1 = *(const lds_float4*)(H + kFaHK + kFaHV + 192 + 16 * lg);
            ks[0] = k0.x, ks[1] = k0.y, ks[2] = k0.z, ks[3] = k0.w;
            ks[4] = k1.x, ks[5] = k1.y, ks[6] = k1.z, ks[7] = k1.w;
            vs[0] = v0.x, vs[1] = v0.y, vs[2] = v0.z, vs[3] = v0.w;
            vs[4] = v1.x, vs[5] = v1.y, vs[6] = v1.z, vs[7] = v1.w;
        }
        float4_t sacc[kFaRB][2];
        half8_t kf[2][2];  // K operands of 32-dim step st: [st & 1][16-key block u]
        auto kread = [&](int st, half8_t (&dst)[2]) __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < 2; ++u) dst[u] = *(const lds_half8*)(H + (2 * st + u) * 1024 + 16 * l);
        };
        kread(0, kf[0]);
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            if (st < 7) kread(st + 1, kf[(st + 1) & 1]);
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int rb = 0; rb < kFaRB; ++rb)
                    sacc[rb][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[st & 1][u], qop[rb][st],
                                                                         st ? sacc[rb][u] : (float4_t)qneg[rb], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        const int kb = n * kTile;
        uint64_t need = 0;
#pragma unroll
        for (int rb = 0; rb < kFaRB; ++rb) {
            const float nm = nm_run[rb];
            float mx = kNegInf;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = __builtin_fmaf(sacc[rb][e >> 2][e & 3], ks[e], nm);
                if constexpr (kMasked) {
                    const int t = kb + 16 * (e >> 2) + 4 * lg + (e & 3);
                    const bool vis = rvalid[rb] & (t < hi) & (t <= rpos[rb]);
                    sv[rb][e] = vis ? x : kNegInf;
                } else {
                    sv[rb][e] = x;
                }
                mx = fmaxf(mx, sv[rb][e]);
            }
            need |= __builtin_amdgcn_ballot_w64(mx > thr_run[rb]);
        }
        return need != 0;
    };

    // ---- rare path: raise the running max of the rows that need it, shift their scores, rescale
    //      their state (O is still zero while every row of a block is fresh: no rescale then) ----
    auto raise_max = [&](float (&sv)[kFaRB][8], int n) __attribute__((always_inline)) {
        // scratch: this wave's own K blocks of fp16 buffer n + 1, idle until the wave widens
        // tile n + 1 into them later in this iteration
        lds_u8* scr = hbuf(n + 1) + 4096 * w + 16 * l;
        const unsigned scr_addr = (unsigned)(uintptr_t)scr;
#pragma unroll
        for (int rb = 0; rb < kFaRB; ++rb) {
            float mloc = kNegInf;
#pragma unroll
            for (int e = 0; e < 8; ++e) mloc = fmaxf(mloc, sv[rb][e]);
            const float mrow = xor_max(xor_max(mloc, 16), 32) - kPLog2;  // tile max relative to m_run
            const bool fresh = m_run[rb] == kNegInf;
            const bool raise = fresh ? mrow > kNegInf : mrow > kLazy;
            const float shift = raise ? mrow : 0.f;
            const float alpha = fresh ? 0.f : __builtin_amdgcn_exp2f(-shift);
            if (raise) m_run[rb] = fresh ? mrow : m_run[rb] + mrow;
            nm_run[rb] = m_run[rb] == kNegInf ? kPLog2 : kPLog2 - m_run[rb];
            thr_run[rb] = m_run[rb] == kNegInf ? kNegInf : kLazy + kPLog2;
#pragma unroll
            for (int e = 0; e < 8; ++e) sv[rb][e] -= shift;
            l_run[rb] *= alpha;
            if (__builtin_amdgcn_ballot_w64(!fresh) != 0) {
#pragma unroll
                for (int m = 0; m < 17; ++m) {
                    float4_t t;
                    asm volatile("ds_write_b128 %1, %2\n\ts_waitcnt lgkmcnt(0)\n\tds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                                 : "=v"(t) : "v"(scr_addr), "a"(oacc[rb][m]) : "memory");
                    t *= alpha;
                    asm volatile("ds_write_b128 %1, %2\n\ts_waitcnt lgkmcnt(0)\n\tds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                                 : "=a"(oacc[rb][m]) : "v"(scr_addr), "v"(t) : "memory");
                }
            }
        }
    };

    // ---- back half: p' = 2^sv, P' = p' * v_scale in fp16, O^T += V^T P'^T; tile n + 1 is
    //      widened in pieces between the products ----
    auto tile_back = [&](int n, const float (&sv)[kFaRB][8], const float (&vs)[8]) __attribute__((always_inline)) {
        const lds_u8* H = hbuf(n) + kFaHK + 16 * l;
        // tile n + 1 is widened even past the last tile: raw slots of tiles never copied hold stale
        // bytes, and the fp16 buffer they land in is never read
        WidenRegs wr;
        widen_load(n + 1, wr);
        constexpr int kVAhead = 4;  // V operand reads in flight ahead of their MFMAs
        half8_t vf[17];
#pragma unroll
        for (int m = 0; m < kVAhead; ++m) vf[m] = *(const lds_half8*)(H + m * 1024);
        half8_t pop[kFaRB];
#pragma unroll
        for (int rb = 0; rb < kFaRB; ++rb) {
            float psum = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float p = __builtin_amdgcn_exp2f(sv[rb][e]);
                psum += p;
                pop[rb][e] = (_Float16)(p * vs[e]);
            }
            l_run[rb] += psum;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = 0; m < 17; ++m) {
            if (m + kVAhead < 17) vf[m + kVAhead] = *(const lds_half8*)(H + (m + kVAhead) * 1024);
#pragma unroll
            for (int rb = 0; rb < kFaRB; ++rb)
                oacc[rb][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[m], pop[rb], oacc[rb][m], 0, 0, 0);
            if (m >= 2 && m < 12) widen_store(n + 1, wr, m - 2);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // tiles [0, n_int) are visible to every row of the workgroup: keys below its first row's
    // position and below hi
    const int n_int = min(pmin + 1 >= 0 ? (pmin + 1) / kTile : 0, hi / kTile);
    const bool tail_wave = w == 3;

    auto tile_loop = [&](auto lds_flag) __attribute__((always_inline)) {
        constexpr bool kLds = decltype(lds_flag)::value;
        auto issue = [&](int n) __attribute__((always_inline)) {
            TileSrc src;
            if constexpr (kFast && kLds) {
                const lds_int* e = pt.lds + 2 * n;
                const unsigned o0 = (unsigned)__builtin_amdgcn_readfirstlane(e[0]);
                const unsigned o1 = (unsigned)__builtin_amdgcn_readfirstlane(e[1]);
                src.base[0] = gbase + ((int64_t)o0 << 3);
                src.base[1] = gbase + ((int64_t)o1 << 3);
            } else {
                src = tile_src<kFast, kLds>(a, pt, gbase, n, n, 0, hi, l);
            }
            const unsigned slot = lds_base + kLdsRaw + (unsigned)((n & (kFaRaw - 1)) * kSlot);
            wait_lds();
            if constexpr (kFast) {
                // this wave's quarter: K blocks and V blocks 2 w, 2 w + 1 (rows of 16-key block w / 2),
                // and the tail for wave 3
                const int8_t* base = (w >> 1) ? src.base[1] : src.base[0];
                const int q2 = 2 * (w & 1);
                dma16_s(base + (int64_t)(4 * q2) * a.k_ss, dl.kvo, slot + kImgK + (2 * w) * kBlk);
                dma16_s(base + (int64_t)(4 * q2 + 4) * a.k_ss, dl.kvo, slot + kImgK + (2 * w + 1) * kBlk);
                dma16_s(base + (int64_t)q2 * a.k_ss, dl.vvo, slot + kImgV + (2 * w) * kBlk);
                dma16_s(base + (int64_t)(q2 + 1) * a.k_ss, dl.vvo, slot + kImgV + (2 * w + 1) * kBlk);
                if (w == 3) {
                    const int64_t delta = src.base[1] - src.base[0];
                    dma16_v<0>(src.base[0] + (delta & -(int64_t)dl.tsel) + dl.toff, slot + kImgT);
                }
                return;
            }
            switch (w) {
                case 0: issue_quarter<kFast, 0>(a, src, dl, slot, l); break;
                case 1: issue_quarter<kFast, 1>(a, src, dl, slot, l); break;
                case 2: issue_quarter<kFast, 2>(a, src, dl, slot, l); break;
                default: issue_quarter<kFast, 3>(a, src, dl, slot, l); break;
            }
        };
        for (int n = 0; n < min(ntiles, kFaRaw); ++n) issue(n);
        if (ntiles > 0) {
            // tile 0 has landed; of tiles 1..3 at most 2 are left in flight (conservative)
            wait_quarters(min(ntiles - 1, 2), tail_wave);
            __syncthreads();
            widen(0);
        }
        // Iteration n: tile n + 1 has landed and every wave is done with iteration n - 1, so
        // fp16 buffer n & 1 holds tile n and raw slot n & 3 (widened in iteration n - 1) is free
        // for tile n + 4.
        auto arrive = [&](int n) __attribute__((always_inline)) {
            if (n + 1 < ntiles) wait_quarters(min(2, ntiles - 2 - n), tail_wave);
            __syncthreads();
            if (n + kFaRaw < ntiles) issue(n + kFaRaw);
        };
        float sv[kFaRB][8], vs[8];
        // The fast inner loops never rescale: O stays in the MFMA accumulators. When some row's
        // max must be raised the loop is left, the rows are rescaled, the tile is finished and
        // the loop resumes with the next tile.
        auto run = [&](auto masked_flag, int n0, int n_end) __attribute__((always_inline)) {
            for (int n = n0; n < n_end; ++n) {
                arrive(n);
                if (__builtin_amdgcn_ballot_w64(tile_front(masked_flag, n, sv, vs)) != 0) raise_max(sv, n);
                tile_back(n, sv, vs);
            }
        };
        run(std::false_type{}, 0, n_int);
        run(std::true_type{}, n_int, ntiles);
    };
    if (pt.in_lds)
        tile_loop(std::true_type{});
    else
        tile_loop(std::false_type{});

    // ---- normalise and store: out[b, tq0 + tok, g G + hh, :] ----
#pragma unroll
    for (int rb = 0; rb < kFaRB; ++rb) {
        const float l_row = xor_sum(xor_sum(l_run[rb], 16), 32);
        const float inv = l_row > 0.f ? 1.f / l_row : 0.f;
        const float corr = __shfl(oacc[rb][16].x, 48 + li, 64);  // 1152 * sum of the row's P'

        if (rvalid[rb]) {
            const int r = 48 * w + 16 * rb + li;
            const int tok = r / G, hh = r - (r / G) * G;
            float* orow = a.out + (int64_t)b * a.o_sb + (int64_t)(tq0 + tok) * a.o_st + (int64_t)(g * G + hh) * a.o_sh;
#pragma unroll
            for (int m = 0; m < 17; ++m) {
                const int d0 = m < 16 ? 16 * m - 4 + 4 * lg : (lg == 2 ? 252 : -1);
                if (d0 >= 0 && d0 < kDim) *reinterpret_cast<float4_t*>(orow + d0) = (oacc[rb][m] - corr) * inv;
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// KV-cache writer: the producer of the 520-byte rows (vLLM's cache update for int8
// per-token-head KV, called as do_kv_cache_update(layer, key, value, kv_cache, slot_mapping),
// upstream/pr-dflash2/0002-fix-gfx906-keep-the-drafter-s-sliding-window-in-the-.patch:81-87).
// One wave per (token, kv head): 64 lanes x 4 elements of K and of V; absmax by a wave
// reduction, scale = absmax / 127 (0 for an all-zero row), q = clamp(rint(x / scale), -127, 127)
// with x / scale correctly rounded; the row's K bytes, k_scale, V bytes and v_scale are written
// with 4-byte stores. Tokens whose slot is negative (padding) or past the cache are skipped.
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

template <class In>
__device__ __forceinline__ float4_t load4(const In* p) {
    if constexpr (sizeof(In) == 4) {
        return *reinterpret_cast<const float4_t*>(p);
    } else {
        typedef In in4_t __attribute__((ext_vector_type(4)));
        const in4_t v = *reinterpret_cast<const in4_t*>(p);
        return float4_t{(float)v.x, (float)v.y, (float)v.z, (float)v.w};
    }
}

__device__ __forceinline__ unsigned quant4(float4_t x, float scale) {
    if (scale == 0.f) return 0u;
    auto q = [&](float v) -> unsigned {
        const float r = fminf(fmaxf(__builtin_rintf(v / scale), -127.f), 127.f);
        return (unsigned)((int)r & 0xff);
    };
    return q(x.x) | (q(x.y) << 8) | (q(x.z) << 16) | (q(x.w) << 24);
}

template <class In>
__global__ void __launch_bounds__(256) pd_cache_write_kernel(const CacheWriteParams a) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
    if (row >= a.T * a.Hkv) return;
    const int t = row / a.Hkv, h = row - t * a.Hkv;
    const int64_t slot = a.slots[t];
    if (slot < 0 || slot >= a.num_slots) return;
    const float4_t k = load4(static_cast<const In*>(a.key) + t * a.k_st + h * a.k_sh + 4 * l);
    const float4_t v = load4(static_cast<const In*>(a.value) + t * a.v_st + h * a.v_sh + 4 * l);
    float km = fmaxf(fmaxf(fabsf(k.x), fabsf(k.y)), fmaxf(fabsf(k.z), fabsf(k.w)));
    float vm = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        km = fmaxf(km, __shfl_xor(km, o, 64));
        vm = fmaxf(vm, __shfl_xor(vm, o, 64));
    }
    const float ks = km / 127.f, vs = vm / 127.f;
    const int64_t blk = slot / a.block_size, off = slot - blk * a.block_size;
    int8_t* r = a.kc + blk * a.k_sb + off * a.k_ss + h * a.k_sh_c;
    reinterpret_cast<unsigned*>(r)[l] = quant4(k, ks);
    reinterpret_cast<unsigned*>(r + 260)[l] = quant4(v, vs);
    if (l == 0) {
        *reinterpret_cast<float*>(r + 256) = ks;
        *reinterpret_cast<float*>(r + 516) = vs;
    }
}

// ---------------------------------------------------------------------------------------
// host side

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
bool fast_block_table(int bs, int64_t k_ss) { return bs % 16 == 0 && k_ss < (int64_t(1) << 27); }

hipError_t check_args(const LaunchArgs& x, bool strict_reference) {
    if (x.heads_kv < 1 || x.heads_q < 1 || x.heads_q % x.heads_kv != 0) return hipErrorInvalidValue;
    const int G = x.heads_q / x.heads_kv;
    if (x.nsplit < 1 || x.nsplit > x.nseg || x.num_seqs < 1) return hipErrorInvalidValue;
    if (x.qmax < 1 || x.block_size < 1) return hipErrorInvalidValue;
    if (strict_reference) {
        if (G != 6 || x.qmax > 4) return hipErrorInvalidValue;
    } else if ((int64_t)x.qmax * G > 16 * kMaxRowBlocks) {
        return hipErrorInvalidValue;
    }
    if (x.num_tokens < 0) return hipErrorInvalidValue;
    return hipSuccess;
}

template <int NRB>
hipError_t launch_partial_nrb(const PartialParams& p, dim3 grid, hipStream_t stream, bool fast) {
    const dim3 block(kThreads);
    if (fast)
        hipLaunchKernelGGL((pd_partial_kernel<NRB, true>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((pd_partial_kernel<NRB, false>), grid, block, 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_partial(const LaunchArgs& x, hipStream_t stream) {
    PartialParams p;
    p.q = static_cast<const _Float16*>(x.q);
    p.q_st = x.q_st;
    p.kc = static_cast<const int8_t*>(x.kc);
    p.k_sb = x.k_sb;
    p.k_ss = x.k_ss;
    p.k_sh = x.k_sh;
    p.block_table = x.block_table;
    p.bt_stride = x.bt_stride;
    p.seq_lens = x.seq_lens;
    p.qsl = x.qsl;
    p.block_size = x.block_size;
    p.scale_log2 = x.scale * 1.4426950408889634f;
    p.part_o = x.part_o;
    p.part_m = x.part_m;
    p.part_l = x.part_l;
    p.nseg = x.nseg;
    p.nsplit = x.nsplit;
    p.G = x.heads_q / x.heads_kv;
    p.qmax = x.qmax;
    p.Hq = x.heads_q;
    p.window = x.window > 0 ? x.window : 0;
    p.causal = x.causal ? 1 : 0;
    p.bs_shift = (x.block_size & (x.block_size - 1)) == 0 ? __builtin_ctz((unsigned)x.block_size) : -1;
    const int rows = x.qmax * p.G;
    const dim3 grid(x.nsplit, x.heads_kv, x.num_seqs);
    const bool fast = fast_block_table(x.block_size, x.k_ss);
    if (rows <= 16) return launch_partial_nrb<1>(p, grid, stream, fast);
    if (rows <= 32) return launch_partial_nrb<2>(p, grid, stream, fast);
    return launch_partial_nrb<3>(p, grid, stream, fast);
}

hipError_t launch_combine(const LaunchArgs& x, hipStream_t stream) {
    CombineParams c;
    c.part_o = x.part_o;
    c.part_m = x.part_m;
    c.part_l = x.part_l;
    c.seq_lens = x.seq_lens;
    c.qsl = x.qsl;
    c.out = static_cast<_Float16*>(x.out);
    c.o_st = x.o_st;
    c.o_sh = x.o_sh;
    c.num_seqs = x.num_seqs;
    c.nseg = x.nseg;
    c.nsplit = x.nsplit;
    c.qmax = x.qmax;
    // Few rows: a quarter row per workgroup for parallelism; many rows: half rows, fewer
    // workgroups (config 3, 768 rows: 31.3 -> 29.7 us per layer; 24 rows: 12.2 against 12.6).
    if ((int64_t)x.num_tokens * x.heads_q <= 256)
        hipLaunchKernelGGL((pd_combine_kernel<16>), dim3(x.num_tokens, x.heads_q, 4), dim3(256), 0, stream, c);
    else
        hipLaunchKernelGGL((pd_combine_kernel<32>), dim3(x.num_tokens, x.heads_q, 2), dim3(256), 0, stream, c);
    return hipGetLastError();
}

hipError_t launch_all(const LaunchArgs& x, hipStream_t stream, bool strict) {
    hipError_t e = check_args(x, strict);
    if (e != hipSuccess) return e;
    if (x.num_tokens == 0) return hipSuccess;
    e = launch_partial(x, stream);
    if (e != hipSuccess) return e;
    return launch_combine(x, stream);
}

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

hipError_t launch_prefill(const FaParams& p, int batch, int heads_kv, hipStream_t stream) {
    const dim3 grid((p.Sq + p.tok_per_wg - 1) / p.tok_per_wg, heads_kv, batch);
    if (fast_block_table(p.block_size, p.k_ss))
        hipLaunchKernelGGL((pd_prefill_kernel<true>), grid, dim3(kFaWaves * 64), 0, stream, p);
    else
        hipLaunchKernelGGL((pd_prefill_kernel<false>), grid, dim3(kFaWaves * 64), 0, stream, p);
    return hipGetLastError();
}

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

// Partials of pth_dec_launch_noalloc: part_o [T, Hq, nsplit, 256], then part_m and part_l
// [T, Hq, nsplit], in device memory the library holds (one copy per GPU, for the life of the
// process). Host code never passes `scratch` itself to a kernel (on the host it only names the
// symbol): each device's address comes from hipGetSymbolAddress, once per device.
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Address of the current device's scratch array (looked up on its first use on that device).
hipError_t scratch_address(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_acquire);
        if (p == nullptr) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return e;
            if (p == nullptr) return hipErrorInvalidSymbol;
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return hipSuccess;
}

}  // namespace

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
    const size_t rows = (size_t)num_tokens * (size_t)heads_q * (size_t)nsplit;
    if (rows * (kDim + 2) * sizeof(float) > kScratchBytes) return hipErrorOutOfMemory;
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
          part_m->sizes[2] == nseg && part_l->sizes[0] >= T && part_l->sizes[1] == Hq && part_l->sizes[2] == nseg))
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

int pth_fa_forward(const pd_tensor* q, const pd_tensor* key_cache, const pd_tensor* value_cache,
                   const pd_tensor* block_table, const pd_tensor* seq_lens, double scale, const pd_tensor* q_abs_offset,
                   const pd_tensor* out, hipStream_t stream, char* err, int errlen) {
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
    const hipError_t e = launch_prefill(p, (int)B, (int)Hkv, stream);
    if (e != hipSuccess) {
        char msg[256];
        snprintf(msg, sizeof msg, "pth_fa launch failed: %s", hipGetErrorString(e));
        fail(err, errlen, msg);
        return 2;
    }
    return 0;
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
    const dim3 grid((unsigned)((T * Hkv + 3) / 4));
    if (dt == PD_DTYPE_FP16)
        hipLaunchKernelGGL((pd_cache_write_kernel<_Float16>), grid, dim3(256), 0, stream, p);
    else if (dt == PD_DTYPE_BF16)
        hipLaunchKernelGGL((pd_cache_write_kernel<__bf16>), grid, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL((pd_cache_write_kernel<float>), grid, dim3(256), 0, stream, p);
    const hipError_t e = hipGetLastError();
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
