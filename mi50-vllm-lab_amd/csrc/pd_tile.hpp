// The tile copy path shared by the decode (pd_decode.hip) and prefill (pd_prefill.hip) kernels:
// the 32-key tile, its raw image in LDS, the DMA copies that fill it from the paged cache, the
// block-table access, and the exact int8 -> fp16 widening. Both kernels copy tiles into the
// image below and read their K operands, transposed V operands and scales at these positions,
// so the layout constants are one contract for both: a change here changes both kernels, and
// both kernels' GPU tests cover it.
#pragma once

#include <type_traits>

#include "pd_kernels.hpp"

namespace pd {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef int int2_t __attribute__((ext_vector_type(2)));
typedef unsigned uint4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) unsigned char lds_u8;
typedef __attribute__((address_space(3))) int2_t lds_int2;
typedef __attribute__((address_space(3))) uint4_t lds_uint4;
typedef __attribute__((address_space(3))) float lds_float;
typedef __attribute__((address_space(3))) float4_t lds_float4;
typedef __attribute__((address_space(3))) int lds_int;
typedef __attribute__((address_space(3))) uint64_t lds_u64;
typedef unsigned long long ull2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) ull2_t lds_ull2;
typedef __attribute__((address_space(3))) half8_t lds_half8;
typedef const __attribute__((address_space(4))) int* const_int_ptr;  // scalar-cache loads

constexpr int kTile = 32;             // keys per tile
constexpr float kNegInf = -__builtin_inff();
// The running max m of a row is only raised when a tile's max exceeds it by more than
// kLazy (log2 units), so p = 2^(s - m) <= 2^kLazy and most tiles skip the O rescale.
// P' = p * v_scale * kPScale then spans the same fp16 range as p * v_scale * 256 with p <= 1.
constexpr float kLazy = 4.0f;
constexpr float kPScale = 16.0f;

// LDS slot of one tile, 17,664 bytes (the decode double-buffers tiles per wave in two slots, the
// prefill keeps a ring of four slots per workgroup).
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

// 8 signed bytes b (two dwords, byte 0 first) -> 8 fp16 holding b + 1152, exact: the bit
// pattern 0x6400 | (b ^ 0x80) encodes 1024 + (b + 128). The constant 1152 is not subtracted
// here; the default prefill removes it once per row instead: O = sum_k P'_k (v_k + 1152) -
// 1152 sum_k P'_k and S = sum_d q_d (k_d + 1152) - 1152 sum_d q_d.
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

// 8 signed bytes b (as widen_i8x8) -> 8 fp16 holding b itself, exact: each byte is sign-extended
// and converted by an SDWA v_cvt_f16_i16 straight into its half of the destination. One
// instruction per value against 0.75 for widen_i8x8, with no bias left in the operand, so the
// products accumulate without the 1152 sum_d q_d (scores) or 1152 sum_k P'_k (values) that the
// fp32 accumulator would otherwise carry (and round) along with them. The decode widens K and V
// this way, and so does the exact prefill.
__device__ __forceinline__ half8_t widen_i8x8_exact(unsigned w0, unsigned w1) {
    uint4_t h;
    asm("v_cvt_f16_i16_sdwa %0, sext(%4) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%4) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%4) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%4) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3\n\t"
        "v_cvt_f16_i16_sdwa %2, sext(%5) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %2, sext(%5) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %3, sext(%5) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f16_i16_sdwa %3, sext(%5) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3"
        : "=&v"(h.x), "=&v"(h.y), "=&v"(h.z), "=&v"(h.w)
        : "v"(w0), "v"(w1));
    return __builtin_bit_cast(half8_t, h);
}

// x = p * s as two fp16 parts, hi + lo with ~22 significant bits: hi is the fp32 product rounded
// to fp16, lo = fp16(p * s - hi) with the product exact (fma). hi must be the same value in both
// places. The fp32 product is therefore pinned in a register: left to itself the compiler folds
// the product into the conversion for one use (v_fma_mix, a single rounding of p * s) and keeps a
// multiply and a convert (two roundings) for the other, and when the fp32 product is an fp16 tie
// the two roundings differ by an fp16 ulp, so hi + lo misses x by up to 2^-10 relative.
__device__ __forceinline__ void split_fp16(float p, float s, _Float16& hi, _Float16& lo) {
    float prod = p * s;
    asm("" : "+v"(prod));
    hi = (_Float16)prod;
    lo = (_Float16)__builtin_fmaf(p, s, -(float)hi);
}

// split_fp16 for two values at once: both hi are converted by one packed conversion, and each lo
// reads its hi from the packed pair.
__device__ __forceinline__ void split_fp16x2(float p0, float s0, float p1, float s1, half2_t& hi, half2_t& lo) {
    float a = p0 * s0, b = p1 * s1;
    asm("" : "+v"(a), "+v"(b));
    hi = __builtin_convertvector((float2_t){a, b}, half2_t);
    lo = (half2_t){(_Float16)__builtin_fmaf(p0, s0, -(float)hi.x), (_Float16)__builtin_fmaf(p1, s1, -(float)hi.y)};
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
// dma16_s into LDS slot + kOff: the destination is formed in m0 by the copy's own s_add (one
// scalar instruction per copy instead of an add into a register and a move).
template <int kOff>
__device__ __forceinline__ void dma16_so(const int8_t* sbase, unsigned voff, unsigned slot) {
    if constexpr (kOff == 0)
        asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(slot)
                     : "memory", "m0");
    else
        asm volatile("s_add_u32 m0, %2, %3\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(slot),
                     "i"(kOff)
                     : "memory", "m0", "scc");
}
// The same with a wave-uniform offset held in a scalar register.
__device__ __forceinline__ void dma16_ss(const int8_t* sbase, unsigned voff, unsigned slot, unsigned off) {
    asm volatile("s_add_u32 m0, %2, %3\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(slot),
                 "s"(off)
                 : "memory", "m0", "scc");
}
// Calls f(std::integral_constant<int, I>) for I = kBegin .. kEnd - 1 (copy offsets that the asm
// takes as immediates must be compile-time constants).
template <int kBegin, int kEnd, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (kBegin < kEnd) {
        f(std::integral_constant<int, kBegin>{});
        static_for<kBegin + 1, kEnd>(f);
    }
}
// The immediate offset applies to the LDS destination too: the copy lands at m0 + kImm +
// 16 * lane, so m0 is passed already reduced by kImm.
template <int kImm>
__device__ __forceinline__ void dma16_v(const int8_t* vaddr, unsigned lds_dst) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off offset:%2" ::"v"(vaddr), "s"(lds_dst - kImm),
                 "i"(kImm)
                 : "memory", "m0");
}
// dma16_v<0> into LDS slot + kOff, m0 formed by the copy's own s_add.
template <int kOff>
__device__ __forceinline__ void dma16_vo(const int8_t* vaddr, unsigned slot) {
    asm volatile("s_add_u32 m0, %1, %2\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(vaddr), "s"(slot), "i"(kOff)
                 : "memory", "m0", "scc");
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

}  // namespace pd
