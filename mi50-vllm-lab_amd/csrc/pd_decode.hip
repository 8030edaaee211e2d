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
//   DFlash2) are held as 16-row blocks, so one read of a K/V tile serves every row. Windowed
//   groups of more than 16 rows are instead sliced into 16-row workgroups (grid z = slice x
//   sequence) when nsplit x Hkv x num_seqs x slices fits the CUs and num_seqs x window is at most
//   16,384 keys: then the slices' repeated reads of the tiles cost less than the split partials
//   they save.
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
//     exactly by SDWA byte conversions, with no bias, so the fp32 accumulators only ever hold
//     partial scores), B = Q^T held in registers; the four accumulation chains (2 key blocks x
//     2 row blocks) are interleaved.
//   softmax: base 2, fp32, online. A row's running max is raised only when a tile exceeds it
//     by > 2^4: each lane tests its own 8 scores and one ballot decides; only then is the row
//     max reduced across lanes and O rescaled (rare after the first tile). P' = p * v_scale * 16
//     in fp16 has the range of p * v_scale * 256 with p <= 1. Masked weights are chosen by
//     select, so a NaN scale on a masked row cannot leak in.
//   O^T += V^T P^T: ds_read_b64_tr_b8 hands each lane 8 keys of one V column (A operand,
//     16 dims x 32 keys, widened exactly like K); P^T never leaves registers: the S^T
//     accumulator layout (lane = query
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
// The tile copies, the raw slot image and the widening are shared with the chunked prefill
// (pd_prefill.hip) through pd_tile.hpp.
//
// Nothing is allocated, nothing waits for the host, and every split range is derived on
// the device from seq_lens / query_start_loc, so launches can be captured in a HIP graph.
#include <atomic>
#include <mutex>

#include "pd_tile.hpp"

namespace pd {

constexpr int kWaveLds = 2 * kSlot;                // LDS bytes per wave
constexpr int kWaves = 4;                          // independent tile streams per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kBtCache = 1024;                     // block-table entries of a split kept in LDS
// With Q staged in LDS as well (block sizes that are multiples of 16) the block-table slice
// is smaller:
constexpr int kBtEarly = 384;                      // per-block row offsets (48 tiles per wave)
constexpr int kBtRaw = 384;                        // raw block-table entries (96 per wave)
constexpr int kBtWave = kBtEarly / 4;              // 16-key blocks staged per wave

// The 17 DMAs of one tile into the slot at LDS address `slot` (8 K blocks, 8 V blocks, tail).
template <bool kFast, class P>
__device__ __forceinline__ void issue_tile(const P& a, const TileSrc& src, const DmaLane& d,
                                           unsigned slot, int lane) {
    if constexpr (kFast) {
        static_for<0, 8>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            dma16_so<kImgK + i * kBlk>(src.base[i >> 2] + (int64_t)(4 * (i & 3)) * a.k_ss, d.kvo, slot);
        });
        static_for<0, 8>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            dma16_so<kImgV + i * kBlk>(src.base[i >> 2] + (int64_t)(i & 3) * a.k_ss, d.vvo, slot);
        });
        const int64_t delta = src.base[1] - src.base[0];
        dma16_vo<kImgT>(src.base[0] + (delta & -(int64_t)d.tsel) + d.toff, slot);
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
    // (three row blocks: Q is staged in the V images of slot 1 of waves 0..2 instead, 16 rows
    // each; those slots receive their V copies only after Q is in registers)
    constexpr bool kQInSlots = NRB >= 3;
    constexpr int kQBytes = kEarly && !kQInSlots ? 16 * NRB * 2 * kDim : 0;
    constexpr int kLdsBytes = kLdsQ + kQBytes;
    static_assert(2 * 17 * 1024 <= kWaveLds && kWaveLds % 16 == 0,
                  "two row blocks of accumulator blocks fit the slots of their wave");
    static_assert(kLdsBytes <= 160 * 1024, "gfx950 has 160 KiB of LDS per CU");
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];

    // grid z = row slice x sequence: with rslices > 1 the workgroup takes rows [row0, row0 + 16 NRB)
    // of its GQA group, and the group's other slices read the same tiles
    const int s = blockIdx.x, g = blockIdx.y;
    const int rs = a.rslices > 1 ? (int)blockIdx.z / a.num_seqs : 0;
    const int b = (int)blockIdx.z - rs * a.num_seqs;
    const int row0 = 16 * NRB * rs;
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
    const int R = min(16 * NRB, ql * G - row0);  // rows of this workgroup: group rows row0 + [0, R)
    if (R <= 0) return;                          // a slice past the sequence's rows
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
        const int i = (row0 + r) / G, hh = (row0 + r) - i * G;
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
    bool rvalid[NRB];
    int rpos[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
        const int r = 16 * rb + li;
        rvalid[rb] = r < R;
        const int qi = (row0 + r) / G, qh = (row0 + r) - qi * G;
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
    // then 4 rows from the v_scale bytes in lane group 3, never stored).
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
            const int r = row0 + min(2 * i + (l >> 5), R - 1);
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
            static_for<0, 8>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
                dma16_so<kSlot + kImgK + i * kBlk>(src1.base[i >> 2] + (int64_t)(4 * (i & 3)) * a.k_ss, dl.kvo, wslots);
            });
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
            static_for<0, 8>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
                dma16_so<kSlot + kImgV + i * kBlk>(src1.base[i >> 2] + (int64_t)(i & 3) * a.k_ss, dl.vvo, wslots);
            });
            const int64_t delta = src1.base[1] - src1.base[0];
            dma16_vo<kSlot + kImgT>(src1.base[0] + (delta & -(int64_t)dl.tsel) + dl.toff, wslots);
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

    // ---- S^T = K Q^T for every row block (K exact in fp16, the widening bias removed before the
    //      products), times k_scale, relative to the running max: sv = s - m (log2 units; s itself
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
                    // K exact in fp16 (no widening bias): the accumulator holds only partial
                    // scores, whose rounding is ~1152 / |k| times smaller than with the bias
                    // removed at the end
                    const half8_t kf = hh == 0 ? widen_i8x8_exact(kr[u].x, kr[u].y) : widen_i8x8_exact(kr[u].z, kr[u].w);
#pragma unroll
                    for (int rb = 0; rb < NRB; ++rb)
                        sacc[rb][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            kf, qop[rb][2 * c + hh], (c | hh) ? sacc[rb][u] : (float4_t)0.f, 0, 0, 0);
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
            // the scores are formed in place in both cases (no copies where the paths meet); a tile
            // at the edge of the visible range then masks its invisible keys to -inf
#pragma unroll
            for (int e = 0; e < 8; ++e) sv[rb][e] = __builtin_fmaf(sacc[rb][e >> 2][e & 3], ks[e], nm);
            if (!interior) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int t = kb + 16 * (e >> 2) + 4 * lg + (e & 3);
                    const int rp = rpos[rb];
                    const bool vis = rvalid[rb] & (t >= lo) & (t < hi) & (!a.causal | (t <= rp)) &
                                     ((a.window <= 0) | ((rp - t) < a.window));
                    sv[rb][e] = vis ? sv[rb][e] : kNegInf;
                }
            }
            float mx = kNegInf;
#pragma unroll
            for (int e = 0; e < 8; ++e) mx = fmaxf(mx, sv[rb][e]);
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
            // O is still zero while every row of the block is fresh, and a row that keeps its
            // max would be multiplied by 1: rescale only when a row with state raises
            if (__builtin_amdgcn_ballot_w64(raise && !fresh) != 0) {
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
    //      rows); then O^T += V^T hi^T + V^T lo^T for every row block, V widened exactly (no
    //      bias: the fp32 accumulators hold only the products' own sums) ----
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
            for (int e = 0; e < 8; e += 2) {
                const float p0 = __builtin_amdgcn_exp2f(sv[rb][e]);  // masked: 2^-inf = 0
                const float p1 = __builtin_amdgcn_exp2f(sv[rb][e + 1]);
                psum += p0;
                psum += p1;
                half2_t h, lo;
                split_fp16x2(p0, vsc[e], p1, vsc[e + 1], h, lo);
                phi[rb][e] = h.x;
                phi[rb][e + 1] = h.y;
                plo[rb][e] = lo.x;
                plo[rb][e + 1] = lo.y;
            }
            l_run[rb] += psum;
        }
#pragma unroll
        for (int m = 0; m < 17; ++m) {
            const half8_t vf = widen_i8x8_exact((unsigned)o.v[m].x, (unsigned)o.v[m].y);
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb)
                oacc[rb][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, phi[rb], oacc[rb][m], 0, 0, 0);
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb)
                oacc[rb][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, plo[rb], oacc[rb][m], 0, 0, 0);
        }
    };

    // ---- every operand of a tile from its slot into registers, so the slot can be refilled
    //      before the tile is computed: v_scale of this lane's keys, the K operand, k_scale, and
    //      the 17 transposed V reads ----
    auto read_ops = [&](lds_u8* T, TileOps& o) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) o.vs[4 * u + j] = *(const lds_float*)(T + vso[u] + 16 * j);
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
            static_for<0, 8>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
                dma16_so<kImgK + i * kBlk>(nsrc.base[i >> 2] + (int64_t)(4 * (i & 3)) * a.k_ss, dl.kvo, slot);
            });
        };
        // While the stream ramps up (the refills of its first kRampTiles tiles) the first four V
        // blocks go between the scores and the values, the rest after the values.
        constexpr int kRampTiles = 2;
        auto ramp = [&](int n) { return n - 2 < kRampTiles; };  // refill n is issued by iteration n - 2
        auto issue_v0 = [&](int n) __attribute__((always_inline)) {
            const unsigned slot = wslots + (unsigned)((n & 1) * kSlot);
            static_for<0, 4>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
                dma16_so<kImgV + i * kBlk>(nsrc.base[i >> 2] + (int64_t)(i & 3) * a.k_ss, dl.vvo, slot);
            });
        };
        auto issue_v = [&](int n) __attribute__((always_inline)) {
            const unsigned slot = wslots + (unsigned)((n & 1) * kSlot);
            if (!ramp(n)) {
                static_for<0, 4>([&](auto ic) {
                    constexpr int i = decltype(ic)::value;
                    dma16_so<kImgV + i * kBlk>(nsrc.base[i >> 2] + (int64_t)(i & 3) * a.k_ss, dl.vvo, slot);
                });
            }
            static_for<4, 8>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
                dma16_so<kImgV + i * kBlk>(nsrc.base[i >> 2] + (int64_t)(i & 3) * a.k_ss, dl.vvo, slot);
            });
            const int64_t delta = nsrc.base[1] - nsrc.base[0];
            dma16_vo<kImgT>(nsrc.base[0] + (delta & -(int64_t)dl.tsel) + dl.toff, slot);
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
        // tiles are done, with its per-row max and sum. Row blocks go through the slots two at a
        // time (kRawRounds rounds). Dims of an accumulator block: block m < 16 holds dims
        // 16 m - 4 + 4 lg .. + 3 in lane group lg (row li), block 16 holds 244..255 in lane
        // groups 0-2. Row factors: M = max_w m_w, e_w = 2^(m_w - M), O = sum_w e_w O_w / 16,
        // L = sum_w e_w l_w.
        //
        // Two or three row blocks: thread (row, 32 dims) derives the factors of its row, sums the
        // four waves' blocks with them and writes its part of the row (a block holds the float4 of
        // (lg, row rr) at 16 lg + rr).
        //
        // One row block (at most 16 rows, single-token decodes): each wave takes whole rows, so
        // the lanes of rows that do not exist issue nothing. For one row the 64 lanes read dims
        // 4 L .. 4 L + 3 (block (L + 1) / 4, group (L + 1) % 4) and store the row's 1 KiB with one
        // instruction. A block then holds the float4 of (lg, rr) at 16 lg + ((rr + lg + 4 (m & 3))
        // & 15), so that the row reads (position (rr + L + 1) & 15) and the stores (16 rows of
        // one lane group) both spread over all banks. (With two row blocks this layout measured
        // 0.26 us slower per launch at 24 rows.)
        constexpr bool kRowStores = NRB == 1;
        constexpr int kRawRounds = (NRB + 1) / 2;
        float* wm = reinterpret_cast<float*>(lds + kLdsStats);  // [wave][NRB][16] running max
        float* wl = wm + kWaves * NRB * 16;                     // [wave][NRB][16] row sum of p
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            const float l_row = xor_sum(xor_sum(l_run[rb], 16), 32);
            if (lg == 0) {
                wm[(w * NRB + rb) * 16 + li] = m_run[rb];
                wl[(w * NRB + rb) * 16 + li] = l_row;
            }
        }
        unsigned raw[4];  // this wave's slots, by block index m & 3
#pragma unroll
        for (int k = 0; k < 4; ++k)
            raw[k] = lds_base + (unsigned)(w * kWaveLds + 16 * (kRowStores ? 16 * lg + ((li + lg + 4 * k) & 15) : l));
        auto store_round = [&](int rd) __attribute__((always_inline)) {
#pragma unroll
            for (int rb = 2 * rd; rb < 2 * rd + 2 && rb < NRB; ++rb)
#pragma unroll
                for (int m = 0; m < 17; ++m)
                    asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(raw[m & 3]), "a"(oacc[rb][m]),
                                 "i"(((rb - 2 * rd) * 17 + m) * 1024)
                                 : "memory");
        };
        store_round(0);
        wait_lds();
        __syncthreads();  // every wave's stats and first accumulator blocks are in LDS
        auto factors = [&](int row, float* f) __attribute__((always_inline)) {
            float M = kNegInf;
#pragma unroll
            for (int v = 0; v < kWaves; ++v) M = fmaxf(M, wm[v * NRB * 16 + row]);
            float Lr = 0.f;
#pragma unroll
            for (int v = 0; v < kWaves; ++v) {
                const float mw = wm[v * NRB * 16 + row];
                const float e = mw == kNegInf ? 0.f : exp2f(mw - M);
                f[v] = e * (1.0f / kPScale);
                Lr += e * wl[v * NRB * 16 + row];
            }
            return float2_t{M, Lr};
        };
        if constexpr (kRowStores) {
            // wave w takes rows w + 4 j; lane j computes the factors of row j of its wave, which
            // are then read from it as scalars
            const int rown = w + 4 * (l & 3);
            float f[kWaves];
            const float2_t ml = factors(rown, f);
            if (l < 4 && rown < R) {
                const int64_t pr = prow(rown);
                a.part_m[pr] = ml.x;
                a.part_l[pr] = ml.y;
            }
            const int m_l = l < 63 ? (l + 1) >> 2 : 16;
            const int g_l = l < 63 ? (l + 1) & 3 : 2;
            const lds_u8* rd_base = L + (m_l * 1024 + 256 * g_l);
            const int c_l = g_l + 4 * (m_l & 3);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = w + 4 * j;  // uniform
                if (row >= R) break;
                const lds_u8* p = rd_base + 16 * ((row + c_l) & 15);
                float fs[kWaves];
#pragma unroll
                for (int v = 0; v < kWaves; ++v)
                    fs[v] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f[v]), j));
                float4_t acc = *(const lds_float4*)p * fs[0];
#pragma unroll
                for (int v = 1; v < kWaves; ++v) acc += *(const lds_float4*)(p + v * kWaveLds) * fs[v];
                *reinterpret_cast<float4_t*>(a.part_o + prow(row) * kDim + 4 * l) = acc;
            }
        } else {
#pragma unroll
            for (int rd = 0; rd < kRawRounds; ++rd) {
                if (rd > 0) {
                    store_round(rd);
                    wait_lds();
                    __syncthreads();
                }
                // thread: row 32 rd + (lane & 31), wave w's two 32-dim parts
                const int row = 32 * rd + (l & 31), part = 2 * w + (l >> 5);
                if (row < R) {
                    float f[kWaves];
                    const float2_t ml = factors(row, f);
                    const int64_t pr = prow(row);
                    if (part == 0) {
                        a.part_m[pr] = ml.x;
                        a.part_l[pr] = ml.y;
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
                        float4_t acc = rawp[blk] * f[0];
#pragma unroll
                        for (int v = 1; v < kWaves; ++v) acc += rawp[v * (kWaveLds / 16) + blk] * f[v];
                        *reinterpret_cast<float4_t*>(dst + d) = acc;
                    }
                }
                if (rd + 1 < kRawRounds) __syncthreads();  // the blocks are rewritten for the next round
            }
        }
    }
}

// Cross-row lane exchanges of gfx950 (v_permlane16/32_swap), as asm with both registers read and
// written. With a = b = x on entry: permlane16: a = rows (0, 0, 2, 2) of x, b = rows (1, 1, 3, 3);
// permlane32: a = (low, low) halves, b = (high, high). So a op b is x op x^16 (resp. x^32) in
// every lane, with no LDS crossbar round trip. The swap must not read a register a VALU
// instruction has just written, and the compiler inserts no wait states around asm: the
// s_nop before (and after, for the results) supply them.
__device__ __forceinline__ void permlane16_swap(float& a, float& b) {
    asm volatile("s_nop 4\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 4" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane32_swap(float& a, float& b) {
    asm volatile("s_nop 4\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 4" : "+v"(a), "+v"(b));
}
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xf, 0xf, false));
}
__device__ __forceinline__ float xor16_sum(float x) {
    float a = x, b = x;
    permlane16_swap(a, b);
    return a + b;
}
__device__ __forceinline__ float xor32_sum(float x) {
    float a = x, b = x;
    permlane32_swap(a, b);
    return a + b;
}
// Max over the 64 lanes, in every lane: DPP within 16-lane rows (quad swaps of 1 and 2 lanes, the
// half-row and row mirrors), then the two cross-row swaps.
__device__ __forceinline__ float wave_max64(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));   // quad_perm [1, 0, 3, 2]
    v = fmaxf(v, dpp_mov<0x4E>(v));   // quad_perm [2, 3, 0, 1]
    v = fmaxf(v, dpp_mov<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_mov<0x140>(v));  // row_mirror
    float a = v, b = v;
    permlane16_swap(a, b);
    v = fmaxf(a, b);
    a = v, b = v;
    permlane32_swap(a, b);
    return fmaxf(a, b);
}

// Sum over the 64 lanes, in every lane (the same DPP and swap steps as wave_max64).
__device__ __forceinline__ float wave_sum64(float v) {
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    v += dpp_mov<0x140>(v);
    return xor32_sum(xor16_sum(v));
}

// Sum of a float4 over the lanes of the wave that share lane % kCW (kCW = 4 or 8): rotations by 4
// and 8 lanes inside each 16-lane row (DPP row_ror), then the two cross-row swaps.
template <int kCW>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (kCW == 4) v += dpp_mov<0x124>(v);  // row_ror:4
    v += dpp_mov<0x128>(v);                          // row_ror:8
    return xor32_sum(xor16_sum(v));
}

// Log-sum-exp merge of the split partials (pth_dec.cu:245-283 semantics): M = max_p m_p,
// L = sum_p 2^(m_p - M) l_p, out = sum_p 2^(m_p - M) O_p / L, and 0 when L == 0. Grid
// (num_tokens, heads_q, 64 / kCols): a workgroup merges 4 kCols dims of one (token, head) row, and
// each of its 4 waves a quarter of them (kCW float4 columns) over every split, so the waves never
// exchange data: no LDS and no barrier. Lane (sg, c) of a wave owns column c of splits sg, sg +
// 64 / kCW, ...; M and L come from a second layout in which lane s holds split s's m and l, by
// wave reductions. Every partial load is issued before anything waits, so the merge costs one
// memory round trip.
// kCols: float4 columns per workgroup, 16 (a 64-dim quarter) or 32 (a half row); kPer: splits
// per lane loaded up front (the first kPer * 64 / (kCols / 4) splits), the smallest power of two
// that covers nsplit up to 64, so that few splits do not cost loads of clamped duplicates.
template <int kCols, int kPer>
__global__ void __launch_bounds__(256) pd_combine_kernel(const CombineParams a) {
    constexpr int kCW = kCols / 4;  // float4 columns per wave
    constexpr int kSG = 64 / kCW;   // lanes sharing a column (segment groups)
    static_assert(kPer * kSG <= 64, "the up-front loads cover at most the first 64 splits");
    const int tok = blockIdx.x, head = blockIdx.y, part = blockIdx.z, Hq = gridDim.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane % kCW, sg = lane / kCW;
    const int col = wave * kCW + c;  // float4 column within the workgroup's dims

    // Sequence of this token = number of sequences whose query rows end at or before it. The first
    // 64 sequences' ends are requested before the partial loads, so that waiting for them does not
    // wait for the partials; the entry of the token's sequence then comes by scalar loads while
    // the partial loads are in flight. The lookup only gates the final store (the merge of a
    // padding token reads allocated but unwritten partials and is discarded).
    // (Every load below is unconditional, from a clamped index with the value selected afterwards,
    // so that the compiler can count them and wait for exactly the one it needs.)
    const int q_end_ld = a.qsl[min(lane + 1, a.num_seqs)];
    asm volatile("" ::: "memory");  // issued before the partial loads
    // The partial loads are in bounds for every (token, head) of the grid.
    const int64_t base = ((int64_t)tok * Hq + head) * a.nseg;
    const float* pm = a.part_m + base;
    const float* pl = a.part_l + base;
    const float4_t* po = reinterpret_cast<const float4_t*>(a.part_o + base * kDim + part * 4 * kCols) + col;
    const int ns1 = a.nsplit - 1;
    const float m_ld = pm[min(lane, ns1)], l_ld = pl[min(lane, ns1)];  // lane s: split s
    float mv[kPer];
    float4_t ov[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int si = min(sg + kSG * i, ns1);
        const float m = pm[si];
        const float4_t o = po[(int64_t)si * (kDim / 4)];
        mv[i] = sg + kSG * i <= ns1 ? m : kNegInf;
        ov[i] = o;
    }

    const int q_end0 = lane + 1 <= a.num_seqs ? q_end_ld : 0x7fffffff;
    int b = __popcll(__ballot(q_end0 <= tok));
    for (int i0 = 64; i0 < a.num_seqs; i0 += 64) {
        const int i = i0 + lane + 1;
        const bool ended = i <= a.num_seqs && a.qsl[i] <= tok;
        b += __popcll(__ballot(ended));
    }
    const int bq = __builtin_amdgcn_readfirstlane(min(b, a.num_seqs - 1));
    const int q_b = ((const_int_ptr)(uintptr_t)a.qsl)[bq], len_b = ((const_int_ptr)(uintptr_t)a.seq_lens)[bq];
    const bool live = b < a.num_seqs && tok >= q_b && len_b > 0 && tok - q_b < a.qmax;

    // M and L over the splits, in the split-per-lane layout (splits 64.. one per lane more)
    const float m_s = lane <= ns1 ? m_ld : kNegInf;
    float mx = m_s;
    for (int p = 64 + lane; p <= ns1; p += 64) mx = fmaxf(mx, pm[p]);
    const float M = wave_max64(mx);
    float lw = 0.f;
    float4_t acc = (float4_t)0.f;
    if (M != kNegInf) {
        lw = m_s != kNegInf ? exp2f(m_s - M) * l_ld : 0.f;
        for (int p = 64 + lane; p <= ns1; p += 64) {
            const float mp = pm[p];
            if (mp != kNegInf) lw += exp2f(mp - M) * pl[p];
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const float w = mv[i] != kNegInf ? exp2f(mv[i] - M) : 0.f;
            acc += w != 0.f ? w * ov[i] : (float4_t)0.f;  // empty splits leave part_o unwritten
        }
        for (int p = sg + kSG * kPer; p <= ns1; p += kSG) {
            const float mp = pm[p];
            if (mp != kNegInf) acc += exp2f(mp - M) * po[(int64_t)p * (kDim / 4)];
        }
    }
    const float L = wave_sum64(lw);
    acc.x = group_sum<kCW>(acc.x);
    acc.y = group_sum<kCW>(acc.y);
    acc.z = group_sum<kCW>(acc.z);
    acc.w = group_sum<kCW>(acc.w);
    if (live && sg == 0) {
        const float inv = L > 0.f ? 1.f / L : 0.f;
        typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
        const half4_t h = {(_Float16)(acc.x * inv), (_Float16)(acc.y * inv), (_Float16)(acc.z * inv),
                           (_Float16)(acc.w * inv)};
        _Float16* o = a.out + (int64_t)tok * a.o_st + (int64_t)head * a.o_sh + part * 4 * kCols + 4 * col;
        __builtin_memcpy(o, &h, 8);
    }
}

// ---------------------------------------------------------------------------------------
// host side

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

// Compute units of the device a stream belongs to (looked up once per device; 0 if unknown).
static int compute_units(hipStream_t stream) {
    constexpr int kDevices = 64;
    static std::atomic<int> cached[kDevices];
    int dev = -1;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0 || dev >= kDevices) return 0;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
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
    const int nrb = rows <= 16 ? 1 : rows <= 32 ? 2 : 3;
    // Windowed groups of more than 16 rows are sliced into 16-row workgroups when that still
    // fits one round of workgroups and the batch's windows hold at most kSliceKeys keys: then
    // each slice re-reading the tiles costs less than the split partials it saves (4 x 8 rows
    // over 2,048-key windows: 23.8 -> 19.3 us per layer at 5 splits of 3 slices against 16
    // unsliced splits; past kSliceKeys, e.g. 4 x 8 rows over 8,192 keys, slicing lost).
    p.num_seqs = x.num_seqs;
    p.rslices = nrb > 1 && x.window > 0 && (int64_t)x.window * x.num_seqs <= kSliceKeys &&
                        (int64_t)x.nsplit * x.heads_kv * x.num_seqs * nrb <= compute_units(stream)
                    ? nrb
                    : 1;
    const dim3 grid(x.nsplit, x.heads_kv, x.num_seqs * p.rslices);
    const bool fast = fast_block_table(x.block_size, x.k_ss);
    if (rows <= 16 || p.rslices > 1) return launch_partial_nrb<1>(p, grid, stream, fast);
    if (rows <= 32) return launch_partial_nrb<2>(p, grid, stream, fast);
    return launch_partial_nrb<3>(p, grid, stream, fast);
}

template <int kCols>
static void launch_combine_cols(const CombineParams& c, dim3 grid, hipStream_t stream) {
    constexpr int kSG = 64 / (kCols / 4);
    const int need = (min(c.nsplit, 64) + kSG - 1) / kSG;  // splits per lane to cover
    if (need <= 1)
        hipLaunchKernelGGL((pd_combine_kernel<kCols, 1>), grid, dim3(256), 0, stream, c);
    else if (need <= 2)
        hipLaunchKernelGGL((pd_combine_kernel<kCols, 2>), grid, dim3(256), 0, stream, c);
    else if (need <= 4 || 64 / kSG < 8)
        hipLaunchKernelGGL((pd_combine_kernel<kCols, (64 / kSG < 4 ? 64 / kSG : 4)>), grid, dim3(256), 0, stream, c);
    else
        hipLaunchKernelGGL((pd_combine_kernel<kCols, (64 / kSG < 8 ? 64 / kSG : 8)>), grid, dim3(256), 0, stream, c);
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
    // workgroups (4 windowed sequences x 8 tokens x 24 heads, 768 rows: 31.3 -> 29.7 us per layer;
    // 24 rows: 12.2 against 12.6).
    if ((int64_t)x.num_tokens * x.heads_q <= 256)
        launch_combine_cols<16>(c, dim3(x.num_tokens, x.heads_q, 4), stream);
    else
        launch_combine_cols<32>(c, dim3(x.num_tokens, x.heads_q, 2), stream);
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

// Partials of pth_dec_launch_noalloc: part_o [T, Hq, nsplit, 256], then part_m and part_l
// [T, Hq, nsplit], in device memory the library holds (one copy per GPU, for the life of the
// process). Host code never passes `scratch` itself to a kernel (on the host it only names the
// symbol): each device's address comes from hipGetSymbolAddress, once per device.
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

}  // namespace pd
