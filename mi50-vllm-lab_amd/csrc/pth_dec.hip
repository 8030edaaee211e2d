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
// Memory path: HBM -> LDS by DMA (global_load_lds_dwordx4), double-buffered per wave.
//   Each lane owns one key row of the tile (rows are 520 bytes, 8-byte aligned) and issues
//   17 16-byte DMAs for it: 8 for the K bytes, 9 for row bytes [248, 520) (k_scale, V,
//   v_scale). The tile's image lands in LDS chunk-major ([chunk][row][16 B]) so every later
//   LDS read is bank-conflict free, and no VGPR ever holds data in flight. The next tile's
//   DMAs are issued before the current tile is computed; s_waitcnt vmcnt(17) waits for the
//   current one only. The block-table entries of a tile are read with scalar loads one tile
//   ahead.
//
// Per 32-key tile, per wave
//   S^T = K Q^T on v_mfma_f32_16x16x32_f16: A = 16 keys x 32 dims of K (int8 widened to fp16
//     exactly: 0x6400|(b^0x80) encodes 1024+b+128), B = Q^T held in registers.
//   softmax: base 2, fp32, online; per-row max = in-lane max + two cross-lane exchanges. The
//     running max of a row is raised only when a tile exceeds it by > 2^4 (rare after the
//     first tile), so O is rarely rescaled; P' = p * v_scale * 16 in fp16 has the same range as
//     p * v_scale * 256 with p <= 1. Masked weights are chosen by select, so a NaN scale on a
//     masked row cannot leak in.
//   O^T += V^T P^T: ds_read_b64_tr_b8 hands each lane 8 keys of one V column (the A operand,
//     16 dims x 32 keys); P^T never leaves registers: the S^T accumulator layout (lane = query
//     row, 4 keys per 16-key block) is the B-operand layout once the MFMA's key order is
//     chosen to match. The V image starts 12 bytes before V[0], so 17 16-dim blocks cover the
//     256 dims; the lanes that fall outside [0, 256) are discarded.
//   Keys outside [lo, seq_len) are never addressed: their row pointers are clamped onto the
//     first / last visible key, so block-table entries of freed pages are never read.
//
// End of split: the 4 waves merge (m, l, O) through LDS and write one partial per row:
//   part_o [T, Hq, nseg, 256] unnormalised, part_m [T, Hq, nseg] running max in log2 units,
//   part_l the matching sum. Splits with no tiles write m = -inf. The combine kernel
//   merges the partials of each (token, head) with a log-sum-exp rescale.
//
// Nothing is allocated, nothing waits for the host, and every split range is derived on
// the device from seq_lens / query_start_loc, so launches can be captured in a HIP graph.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

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
typedef const __attribute__((address_space(4))) int* const_int_ptr;  // scalar-cache loads

constexpr int kDim = 256;             // head dim (the only one the cache row layout allows)
constexpr int kTile = 32;             // keys per wave tile
constexpr int kWaves = 4;             // waves per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxRowBlocks = 3;      // up to 48 query rows per kv head
constexpr float kNegInf = -__builtin_inff();
// The running max m of a row is only raised when a tile's max exceeds it by more than
// kLazy (log2 units), so p = 2^(s - m) <= 2^kLazy and most tiles skip the O rescale.
// P' = p * v_scale * kPScale then spans the same fp16 range as p * v_scale * 256 with p <= 1.
constexpr float kLazy = 4.0f;
constexpr float kPScale = 16.0f;

// LDS image of one tile: K [16 chunks][32 rows][16 B], then V [18 pos][32 rows][16 B] where
// pos p holds row bytes [248 + 16 p, 264 + 16 p) (pos 17 repeats pos 16).
constexpr int kKBytes = 16 * kTile * 16;
constexpr int kVFirst = 248;
constexpr int kVBytes = 18 * kTile * 16;
constexpr int kTileBytes = kKBytes + kVBytes;
constexpr int kWaveBytes = 2 * kTileBytes;              // double buffer
constexpr int kLdsTiles = kWaves * kWaveBytes;
constexpr int kOPitch = kDim + 4;                       // floats per row of the merge buffer
constexpr int kLdsMerge = kWaves * 16 * kOPitch * 4;    // aliases the tile buffers
constexpr int kLdsStats = kLdsTiles;
constexpr int kLdsBytes = kLdsStats + 2 * kWaves * 16 * kMaxRowBlocks * 4;
constexpr int kDmaPerTile = 17;
static_assert(kLdsMerge <= kLdsTiles, "merge buffer must fit in the tile buffers");
static_assert(kLdsBytes <= 160 * 1024, "gfx950 has 160 KiB of LDS per CU");

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

// 8 signed bytes (two dwords, byte 0 first) -> 8 fp16, exact.
__device__ __forceinline__ half8_t widen_i8x8(unsigned w0, unsigned w1) {
    const unsigned u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;  // b + 128 as unsigned bytes
    // v_perm_b32 selector bytes 0..3 pick bytes of the 2nd operand, 4 picks byte 0 of the 1st.
    uint4_t h;
    h.x = __builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u);  // [u0.b0, 0x64, u0.b1, 0x64]
    h.y = __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u);  // [u0.b2, 0x64, u0.b3, 0x64]
    h.z = __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u);
    h.w = __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u);
    return __builtin_bit_cast(half8_t, h) - (_Float16)1152.0f;
}

__device__ __forceinline__ float xor_max(float v, int mask) { return fmaxf(v, __shfl_xor(v, mask, 64)); }
__device__ __forceinline__ float xor_sum(float v, int mask) { return v + __shfl_xor(v, mask, 64); }

// One 16-byte HBM -> LDS DMA per lane: LDS[m0 + IMM + 16 * lane] = global[g + IMM .. + 16).
// Issued through asm so the compiler does not add its conservative vmcnt(0) before every LDS
// read; completion is awaited explicitly with wait_vm.
template <int IMM>
__device__ __forceinline__ void dma16(const int8_t* g, unsigned m0) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off offset:%2" ::"v"(g), "s"(m0), "i"(IMM)
                 : "memory", "m0");
}
// If do_scale (wave-uniform, nonzero): acc *= alpha, for an MFMA accumulator kept in AGPRs.
// The test and the multiply are both inside the asm so that, to the compiler, this is an
// in-place update with no control flow: a C-level branch makes the register allocator copy
// every accumulator out of the AGPRs on each loop iteration although the rescale is rare.
__device__ __forceinline__ void scale_acc_if(float4_t& acc, float alpha, int do_scale) {
    float a0 = acc[0], a1 = acc[1], a2 = acc[2], a3 = acc[3];
    float t;
    asm volatile(
        "s_cmp_eq_u32 %6, 0\n\t"
        "s_cbranch_scc1 .Lpd_skip_%=\n\t"
        "v_accvgpr_read_b32 %4, %0\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %0, %4\n\t"
        "v_accvgpr_read_b32 %4, %1\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %1, %4\n\t"
        "v_accvgpr_read_b32 %4, %2\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %2, %4\n\t"
        "v_accvgpr_read_b32 %4, %3\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %3, %4\n\t"
        "s_nop 1\n"
        ".Lpd_skip_%=:"
        : "+a"(a0), "+a"(a1), "+a"(a2), "+a"(a3), "=&v"(t)
        : "v"(alpha), "s"(do_scale)
        : "scc");
    acc = float4_t{a0, a1, a2, a3};
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// The 17 DMAs of one tile for this lane's key row. kofs / vofs: LDS addresses of the tile's
// K and V images. Lanes h = 0 / 1 fetch alternate 16-byte chunks of the same row.
__device__ __forceinline__ void issue_tile(const int8_t* row, int h, unsigned kofs, unsigned vofs) {
    const int8_t* gh = row + 16 * h;
    // K: chunk 2i + h at LDS kofs + 512 (2i + h) + 16 row = m0 + imm + 16 lane
#define PD_K(i) dma16<32 * (i)>(gh, kofs + 1024u * (i) - 32u * (i))
    PD_K(0); PD_K(1); PD_K(2); PD_K(3); PD_K(4); PD_K(5); PD_K(6); PD_K(7);
#undef PD_K
    // V image pos 2i + h: row bytes [248 + 32 i + 16 h, +16)
#define PD_V(i) dma16<kVFirst + 32 * (i)>(gh, vofs + 1024u * (i) - (unsigned)(kVFirst + 32 * (i)))
    PD_V(0); PD_V(1); PD_V(2); PD_V(3); PD_V(4); PD_V(5); PD_V(6); PD_V(7);
#undef PD_V
    // pos 16 = row bytes [504, 520); the h = 1 half lands a copy in pos 17
    dma16<kVFirst + 256>(row, vofs + 8192u - (unsigned)(kVFirst + 256));
}

// Uniform page lookups of one tile: the (at most two) pages its visible keys live on.
struct TilePages {
    int kb, kfirst, klast, lbA, split;
    int64_t blkA, blkB;
};

template <bool kFastBT>
__device__ __forceinline__ TilePages tile_pages(const PartialParams& a, const_int_ptr bt_row, int tile, int lo,
                                                int hi) {
    TilePages p;
    p.kb = tile * kTile;
    p.kfirst = max(p.kb, lo);
    p.klast = min(p.kb + kTile - 1, hi - 1);
    if constexpr (kFastBT) {
        // block_size == 16 or >= 32: a 32-aligned tile touches at most two pages.
        const int bs = a.block_size;
        p.lbA = p.kfirst / bs;
        const int lbB = p.klast / bs;
        p.blkA = bt_row[p.lbA];
        p.blkB = bt_row[lbB];
        p.split = (p.lbA + 1) * bs;
    } else {
        p.lbA = 0;
        p.blkA = p.blkB = 0;
        p.split = 0;
    }
    return p;
}

// Address of this lane's key row (row rho of the tile), clamped into the visible keys.
template <bool kFastBT>
__device__ __forceinline__ const int8_t* tile_row(const PartialParams& a, const_int_ptr bt_row, const TilePages& p,
                                                  int rho, int g) {
    const int t = min(max(p.kb + rho, p.kfirst), p.klast);
    int64_t blk;
    int sl;
    if constexpr (kFastBT) {
        const bool inB = t >= p.split;
        blk = inB ? p.blkB : p.blkA;
        sl = t - (inB ? p.split : p.lbA * a.block_size);
    } else {
        const int lb = t / a.block_size;
        sl = t - lb * a.block_size;
        blk = bt_row[lb];
    }
    return a.kc + blk * a.k_sb + (int64_t)sl * a.k_ss + (int64_t)g * a.k_sh;
}

template <int NRB, bool kFastBT>
__global__ void __launch_bounds__(kThreads, 1) __attribute__((amdgpu_waves_per_eu(1, 1)))
pd_partial_kernel(const PartialParams a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];

    const int s = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, l = tid & 63, lg = l >> 4, li = l & 15, h = l >> 5;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, uniform by construction

    const int q0 = a.qsl[b];
    const int q_len = a.qsl[b + 1] - q0;
    const int seq_len = a.seq_lens[b];
    if (q_len <= 0 || seq_len <= 0) return;
    const int ql = min(q_len, a.qmax);
    const int G = a.G;
    const int R = ql * G;
    const int ctx0 = seq_len - q_len;  // absolute position of query token 0
    const int lo = a.window > 0 ? max(0, ctx0 - a.window + 1) : 0;
    const int hi = seq_len;
    const int t_first = lo / kTile;
    const int ntiles = (hi - 1) / kTile - t_first + 1;
    const int per_split = (ntiles + a.nsplit - 1) / a.nsplit;
    const int tb = t_first + s * per_split;
    const int te = min(t_first + ntiles, tb + per_split);

    auto prow = [&](int r) -> int64_t {  // partial row index of query row r
        const int i = r / G, hh = r - i * G;
        return ((int64_t)(q0 + i) * a.Hq + (g * G + hh)) * a.nseg + s;
    };

    if (tb >= te) {  // no tiles: mark the split empty for the combine
        for (int r = tid; r < R; r += kThreads) {
            a.part_m[prow(r)] = kNegInf;
            a.part_l[prow(r)] = 0.f;
        }
        return;
    }

    // ---- per-lane query rows and Q^T operand (B of S^T = K Q^T) ----
    bool rvalid[NRB];
    int rpos[NRB];
    half8_t qop[NRB][8];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
        const int r = 16 * rb + li;
        const int i = r / G, hh = r - (r / G) * G;
        rvalid[rb] = r < R;
        rpos[rb] = ctx0 + i;
        const _Float16* qrow = a.q + (int64_t)(q0 + (rvalid[rb] ? i : 0)) * a.q_st + (int64_t)(g * G + hh) * kDim;
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            half8_t v;
            const int dim = 64 * (st >> 1) + 16 * lg + 8 * (st & 1);
            __builtin_memcpy(&v, __builtin_assume_aligned(qrow + dim, 4), 16);
            qop[rb][st] = rvalid[rb] ? v : (half8_t)(_Float16)0.0f;
        }
    }

    float m_run[NRB], l_run[NRB];
    float4_t oacc[NRB][17];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
        m_run[rb] = kNegInf;
        l_run[rb] = 0.f;
#pragma unroll
        for (int m = 0; m < 17; ++m) oacc[rb][m] = (float4_t)0.f;
    }

    lds_u8* L = (lds_u8*)lds;
    const unsigned lds_base = (unsigned)(uintptr_t)L;
    const unsigned wofs = (unsigned)(w * kWaveBytes);  // this wave's double buffer
    // transposed-read lane address: lane pair (2r, 2r+1) of a 16-lane group names key slot r
    const int slot = li >> 1;
    const int tkey = slot < 4 ? 4 * lg + slot : 16 + 4 * lg + (slot - 4);
    const int tr_lane = 16 * tkey + 8 * (li & 1);

    // The block table is read-only for the kernel's lifetime: read it through the constant
    // address space so uniform lookups become scalar loads (they must not share the vector
    // memory counter with the K/V stream, or every lookup would drain the DMA pipeline).
    const_int_ptr bt_row = (const_int_ptr)(uintptr_t)(a.block_table + (int64_t)b * a.bt_stride);

    const int my_first = tb + w;
    const int nt = my_first < te ? (te - 1 - my_first) / kWaves + 1 : 0;
    const int rho = l & 31;

    auto compute_tile = [&](int tile, unsigned kofs, unsigned vofs) {
        // ---- S^T = K Q^T ----
        float4_t sacc[NRB][2];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) sacc[rb][0] = sacc[rb][1] = (float4_t)0.f;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint4_t kraw = *(const lds_uint4*)(L + kofs + 512 * (4 * c + lg) + 16 * (li + 16 * u));
                const half8_t k0 = widen_i8x8(kraw.x, kraw.y);
                const half8_t k1 = widen_i8x8(kraw.z, kraw.w);
#pragma unroll
                for (int rb = 0; rb < NRB; ++rb) {
                    sacc[rb][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, qop[rb][2 * c], sacc[rb][u], 0, 0, 0);
                    sacc[rb][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, qop[rb][2 * c + 1], sacc[rb][u], 0, 0, 0);
                }
            }
        }

        // ---- scales of this lane's 8 keys 16u + 4lg + j (k_scale at row byte 256, v_scale at 516) ----
        float ks[2][4], vs[2][4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int key = 16 * u + 4 * lg + j;
                ks[u][j] = *(const lds_float*)(L + vofs + 16 * key + (256 - kVFirst)) * a.scale_log2;
                vs[u][j] = *(const lds_float*)(L + vofs + 512 * 16 + 16 * key + (516 - kVFirst - 256)) * kPScale;
            }
        }

        // ---- online softmax, P' ----
        const int kb = tile * kTile;
        // Interior tile: every key is visible to every row (padding rows have Q = 0 and
        // are never written out), so no per-element mask is needed.
        bool interior = kb >= lo && kb + kTile <= hi;
        if (a.causal) interior = interior && kb + kTile - 1 <= ctx0;
        if (a.window > 0) interior = interior && (ctx0 + ql - 1) - kb < a.window;
        half8_t pop[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            float sv[2][4];
            bool vis[2][4];
            float mloc = kNegInf;
            if (interior) {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        vis[u][j] = true;
                        sv[u][j] = sacc[rb][u][j] * ks[u][j];
                        mloc = fmaxf(mloc, sv[u][j]);
                    }
                }
            } else {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int t = kb + 16 * u + 4 * lg + j;
                        bool ok = rvalid[rb] && t >= lo && t < hi;
                        if (a.causal) ok = ok && t <= rpos[rb];
                        if (a.window > 0) ok = ok && (rpos[rb] - t) < a.window;
                        vis[u][j] = ok;
                        sv[u][j] = ok ? sacc[rb][u][j] * ks[u][j] : kNegInf;
                        mloc = fmaxf(mloc, sv[u][j]);
                    }
                }
            }
            mloc = xor_max(mloc, 16);
            mloc = xor_max(mloc, 32);
            const bool raise = mloc > m_run[rb] + kLazy;
            // wave-uniform; after the first tile it is rarely taken
            const int any_raise = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_ballot_w64(raise) != 0);
            {
                const float m_new = raise ? mloc : m_run[rb];
                const float alpha = m_run[rb] == kNegInf ? 0.f : __builtin_amdgcn_exp2f(m_run[rb] - m_new);
                l_run[rb] *= alpha;
                m_run[rb] = m_new;
#pragma unroll
                for (int m = 0; m < 17; ++m) scale_acc_if(oacc[rb][m], alpha, any_raise);
            }
            float psum = 0.f;
            _Float16 pv[8];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float p = vis[u][j] ? __builtin_amdgcn_exp2f(sv[u][j] - m_run[rb]) : 0.f;
                    psum += p;
                    pv[4 * u + j] = (_Float16)(vis[u][j] ? p * vs[u][j] : 0.f);
                }
            }
            l_run[rb] += psum;
            pop[rb] = half8_t{pv[0], pv[1], pv[2], pv[3], pv[4], pv[5], pv[6], pv[7]};
        }

        // ---- O^T += V^T P^T ----
#pragma unroll
        for (int m = 0; m < 17; ++m) {
            const int2_t raw = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_int2*)(L + vofs + 512 * m + tr_lane));
            const half8_t vop = widen_i8x8((unsigned)raw.x, (unsigned)raw.y);
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb)
                oacc[rb][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop[rb], oacc[rb][m], 0, 0, 0);
        }
    };

    if (nt > 0) {
        TilePages pg = tile_pages<kFastBT>(a, bt_row, my_first, lo, hi);
        issue_tile(tile_row<kFastBT>(a, bt_row, pg, rho, g), h, lds_base + wofs, lds_base + wofs + kKBytes);
        if (nt > 1) pg = tile_pages<kFastBT>(a, bt_row, my_first + kWaves, lo, hi);
        for (int n = 0; n < nt; ++n) {
            const unsigned cur = wofs + (unsigned)((n & 1) * kTileBytes);
            if (n + 1 < nt) {
                const unsigned nxt = wofs + (unsigned)(((n + 1) & 1) * kTileBytes);
                issue_tile(tile_row<kFastBT>(a, bt_row, pg, rho, g), h, lds_base + nxt, lds_base + nxt + kKBytes);
                if (n + 2 < nt) pg = tile_pages<kFastBT>(a, bt_row, my_first + (n + 2) * kWaves, lo, hi);
                wait_vm<kDmaPerTile>();
            } else {
                wait_vm<0>();
            }
            compute_tile(my_first + n * kWaves, cur, cur + kKBytes);
        }
    }
    // ---- merge the 4 waves ----
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
        float lt = xor_sum(l_run[rb], 16);
        l_run[rb] = xor_sum(lt, 32);
    }
    float* wm = reinterpret_cast<float*>(lds + kLdsStats);
    float* wl = wm + kWaves * 16 * kMaxRowBlocks;
    __syncthreads();  // every wave is done with its loop buffers (the merge buffer aliases them)
    if (lg == 0) {
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            wm[w * 16 * kMaxRowBlocks + 16 * rb + li] = m_run[rb];
            wl[w * 16 * kMaxRowBlocks + 16 * rb + li] = l_run[rb];
        }
    }
    __syncthreads();
    float* obuf = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
        const int row = 16 * rb + li;
        float M = kNegInf;
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, wm[ww * 16 * kMaxRowBlocks + row]);
        const float f = m_run[rb] == kNegInf ? 0.f : exp2f(m_run[rb] - M) * (1.0f / kPScale);
        float* ob = obuf + (w * 16 + li) * kOPitch;
#pragma unroll
        for (int m = 0; m < 17; ++m) {
            const int d0 = 16 * m - (260 - kVFirst) + 4 * lg;  // block m covers dims 16m-12 .. 16m+3
            if (d0 >= 0 && d0 < kDim) *reinterpret_cast<float4_t*>(ob + d0) = oacc[rb][m] * f;
        }
        __syncthreads();
        {
            const int orow = tid >> 4, dq = (tid & 15) * 16;
            const int r = 16 * rb + orow;
            if (r < R) {
                float Mr = kNegInf;
#pragma unroll
                for (int ww = 0; ww < kWaves; ++ww) Mr = fmaxf(Mr, wm[ww * 16 * kMaxRowBlocks + r]);
                float* dst = a.part_o + prow(r) * kDim + dq;
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    float4_t acc = (float4_t)0.f;
#pragma unroll
                    for (int ww = 0; ww < kWaves; ++ww)
                        acc += *reinterpret_cast<const float4_t*>(obuf + (ww * 16 + orow) * kOPitch + dq + 4 * q4);
                    *reinterpret_cast<float4_t*>(dst + 4 * q4) = acc;
                }
                if ((tid & 15) == 0) {
                    float L = 0.f;
#pragma unroll
                    for (int ww = 0; ww < kWaves; ++ww) {
                        const float mw = wm[ww * 16 * kMaxRowBlocks + r];
                        if (mw != kNegInf) L += exp2f(mw - Mr) * wl[ww * 16 * kMaxRowBlocks + r];
                    }
                    a.part_m[prow(r)] = Mr;
                    a.part_l[prow(r)] = L;
                }
            }
        }
        __syncthreads();
    }
}

// One workgroup per (token, q head): 4 groups of 64 threads split the partials, each thread
// owns 4 output dims; the groups are merged through LDS. Follows pth_dec.cu:245-283.
__global__ void __launch_bounds__(256) pd_combine_kernel(const CombineParams a) {
    __shared__ float sm_acc[4][64][5];
    const int tok = blockIdx.x, head = blockIdx.y, Hq = gridDim.y;
    const int tid = threadIdx.x, d4 = tid & 63, grp = tid >> 6;
    int b = 0;
    while (b < a.num_seqs && a.qsl[b + 1] <= tok) ++b;
    if (b >= a.num_seqs || tok < a.qsl[b]) return;  // padding token
    if (a.seq_lens[b] <= 0) return;
    if (tok - a.qsl[b] >= a.qmax) return;  // rows past qmax are not computed
    const int64_t base = ((int64_t)tok * Hq + head) * a.nseg;
    float M = kNegInf;
    for (int p = 0; p < a.nsplit; ++p) M = fmaxf(M, a.part_m[base + p]);
    float L = 0.f;
    float4_t acc = (float4_t)0.f;
    if (M != kNegInf) {
        for (int p = 0; p < a.nsplit; ++p) {
            const float mp = a.part_m[base + p];
            if (mp == kNegInf) continue;
            const float wgt = exp2f(mp - M);
            L += wgt * a.part_l[base + p];
            if ((p & 3) == grp)
                acc += wgt * reinterpret_cast<const float4_t*>(a.part_o + (base + p) * kDim)[d4];
        }
    }
    sm_acc[grp][d4][0] = acc.x;
    sm_acc[grp][d4][1] = acc.y;
    sm_acc[grp][d4][2] = acc.z;
    sm_acc[grp][d4][3] = acc.w;
    __syncthreads();
    if (grp == 0) {
        const float inv = L > 0.f ? 1.f / L : 0.f;
        _Float16* o = a.out + (int64_t)tok * a.o_st + (int64_t)head * a.o_sh + 4 * d4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float v = sm_acc[0][d4][j] + sm_acc[1][d4][j] + sm_acc[2][d4][j] + sm_acc[3][d4][j];
            o[j] = (_Float16)(v * inv);
        }
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

bool fast_block_table(int bs) { return bs == 16 || bs >= 32; }

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
    if (fast)
        hipLaunchKernelGGL((pd_partial_kernel<NRB, true>), grid, dim3(kThreads), 0, stream, p);
    else
        hipLaunchKernelGGL((pd_partial_kernel<NRB, false>), grid, dim3(kThreads), 0, stream, p);
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
    const int rows = x.qmax * p.G;
    const dim3 grid(x.nsplit, x.heads_kv, x.num_seqs);
    const bool fast = fast_block_table(x.block_size);
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
    hipLaunchKernelGGL(pd_combine_kernel, dim3(x.num_tokens, x.heads_q), dim3(256), 0, stream, c);
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

const char* pth_dec_version(void) { return "pth_dec-gfx950 0.1"; }

}  // extern "C"
