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
// kExact (pth_fa_forward_exact) gives the decode kernel's numerics: K and V are widened without
// the bias (so the fp32 accumulators hold only the products' own sums) and P' enters the P.V
// products as fp16 hi + lo, which doubles them. The default instance keeps the bias in K and V
// and removes it per row (sum_d q_d (k_d + 1152) - 1152 sum_d q_d, sum_k P'_k (v_k + 1152) -
// 1152 sum_k P'_k).
#include <type_traits>

#include "pd_tile.hpp"

namespace pd {

constexpr int kFaRaw = 4;                       // raw (int8) tile slots
constexpr int kFaHK = 16 * 1024;                // fp16 K operands: (32-dim step, 16-key block) x 1 KiB
constexpr int kFaHV = 17 * 1024;                // fp16 V^T operands: 17 16-dim blocks x 1 KiB
constexpr int kFaHS = 256;                      // k_scale * scale * log2(e) [32], v_scale [32]
constexpr int kFaHBuf = kFaHK + kFaHV + kFaHS;
constexpr int kFaBt = 6144;                     // 16-key blocks (or pages) of the LDS block table

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

template <bool kFast, bool kExact, bool kSplit>
__global__ void __launch_bounds__(kFaWaves * 64, 1) pd_prefill_kernel(const FaParams a) {
    constexpr int kLdsRaw = 0;
    constexpr int kLdsH = kLdsRaw + kFaRaw * kSlot;
    // The unsplit default instance addresses its widening stores from bases held per tile (see
    // widen_load), starts its row sums from the first term and forms P' by v_fma_mix; the split
    // and exact instances measured slower with these (the split one 4.14 -> 4.23 ms at 2,560
    // tokens x 4 splits, fma_mix being the part that costs it) and keep per-store addresses and
    // a multiply and a conversion for P'.
    constexpr bool kPinned = !kExact && !kSplit;
    constexpr int kLdsBt = kLdsH + 2 * kFaHBuf;
    constexpr int kLdsBytes = kLdsBt + kFaBt * 4;
    static_assert(kLdsBytes <= 160 * 1024, "gfx950 has 160 KiB of LDS per CU");
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];

    // Workgroups are dispatched to the 8 XCDs round robin (linear id L to XCD L % 8), and each XCD
    // has its own L2. Every query tile of a (sequence, kv head) streams the same keys, so the
    // logical workgroup index (query tile fastest) is laid out XCD by XCD: XCD x takes a
    // contiguous range of it, and the query tiles sharing a kv head mostly share an L2 (a 2,048-token
    // chunk at 24 q / 4 kv heads: each kv head's 64 query tiles on two XCDs).
    const unsigned nx = gridDim.x, ny = gridDim.y, nwg = nx * ny * gridDim.z;
    const unsigned lin = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
    const unsigned xcd = lin % 8u;
    const unsigned lidx = xcd * (nwg / 8u) + min(xcd, nwg % 8u) + lin / 8u;
    // x = split * (query tiles) + query tile: the query tiles of one split and kv head (which
    // stream the same keys) stay neighbours in the XCD order
    const int x = (int)(lidx % nx), g = (int)((lidx / nx) % ny), b = (int)(lidx / (nx * ny));
    const int nqt = kSplit ? (int)nx / a.nsplit : (int)nx;
    const int qt = kSplit ? x % nqt : x, split = kSplit ? x / nqt : 0;
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
    // this workgroup's run of key tiles [t0, t1): all of them unless the keys are split
    const int per = kSplit ? (ntiles + a.nsplit - 1) / a.nsplit : ntiles;
    const int t0 = kSplit ? min(ntiles, split * per) : 0, t1 = kSplit ? min(ntiles, t0 + per) : ntiles;

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
            const int nblk = 2 * (t1 - t0);  // the workgroup's tiles t0 + i / 2
            pt.in_lds = a.bt32 && nblk <= kFaBt;
            if (pt.in_lds) {
                lds_int* dst = (lds_int*)(L + kLdsBt);
                for (int i = tid; i < nblk; i += kFaWaves * 64) {
                    const int kb = (t0 + (i >> 1)) * kTile;
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
        lds_u8 *h, *hk, *hv, *hs;  // destinations in fp16 buffer n & 1
    };
    auto widen_load = [&](int n, WidenRegs& r) __attribute__((always_inline)) {
        // The fp16 buffers lie above 64 KiB, beyond the 16-bit offset of an LDS instruction: the
        // unsplit default instance forms the destinations once per tile and holds them opaque,
        // so that every store carries only its small offset as an immediate (the exact instance,
        // which holds more registers across the products, measured slower carrying them: 4.03 ->
        // 4.18 ms for a 2,048-token chunk over 61,440 cached keys).
        if constexpr (kPinned) {
            r.h = hbuf(n) + 16 * l;
            r.hs = hbuf(n) + kFaHK + kFaHV + 4 * l;
            asm("" : "+v"(r.h), "+v"(r.hs));
            r.hk = r.h + 4096 * w;
            r.hv = r.h + kFaHK + 1024 * w;
        }
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
            half8_t kf;
            if constexpr (kExact)
                kf = hh == 0 ? widen_i8x8_exact(r.kr[u].x, r.kr[u].y) : widen_i8x8_exact(r.kr[u].z, r.kr[u].w);
            else
                kf = hh == 0 ? widen_i8x8(r.kr[u].x, r.kr[u].y) : widen_i8x8(r.kr[u].z, r.kr[u].w);
            lds_u8* const d = kPinned ? r.hk + (2 * hh + u) * 1024 : H + ((2 * w + hh) * 2 + u) * 1024 + 16 * l;
            *(lds_half8*)d = kf;
        } else if (j < 8) {
            // kExact: V widened exactly (no bias), so the fp32 P.V accumulators hold only the
            // products' own sums; else with the bias, removed per row at the end
            const int2_t vr = r.vr[j - 4];
            lds_u8* const d = kPinned ? r.hv + 4096 * (j - 4) : H + kFaHK + (w + 4 * (j - 4)) * 1024 + 16 * l;
            *(lds_half8*)d =
                kExact ? widen_i8x8_exact((unsigned)vr.x, (unsigned)vr.y) : widen_i8x8((unsigned)vr.x, (unsigned)vr.y);
        } else if (j == 8) {
            // rows 12..15 of the tail block are the v_scale bytes. kExact: the O^T rows they feed
            // (lane group 3 of accumulator block 16) are never stored. Else they are widened from
            // 0 to exactly 1152, so those rows accumulate 1152 * sum of P', the bias to remove
            if constexpr (kExact) {
                *(lds_half8*)(H + kFaHK + 16 * 1024 + 16 * l) = widen_i8x8_exact((unsigned)r.vr[4].x, (unsigned)r.vr[4].y);
            } else {
                const int2_t vt = li >= 12 ? int2_t{0, 0} : r.vr[4];
                lds_u8* const d = kPinned ? r.h + kFaHK + 16 * 1024 : H + kFaHK + 16 * 1024 + 16 * l;
                *(lds_half8*)d = widen_i8x8((unsigned)vt.x, (unsigned)vt.y);
            }
        } else {
            // k_scale * scale * log2(e) [32] then v_scale [32]; keys past seq_len may hold garbage
            // scales (even NaN): v_scale 0 makes their P' 0
            const bool dead = l >= 32 && n * kTile + sr >= hi;
            lds_float* const d = kPinned ? (lds_float*)r.hs : (lds_float*)(H + kFaHK + kFaHV + 4 * l);
            *d = dead ? 0.f : r.sc * sc_mul;
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
                                                                         st ? sacc[rb][u] : (float4_t)(kExact ? 0.f : qneg[rb]), 0, 0, 0);
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
            // O is still zero while every row of the block is fresh, and a row that keeps its
            // max would be multiplied by 1: rescale only when a row with state raises, four
            // accumulators per LDS round trip
            if (__builtin_amdgcn_ballot_w64(raise && !fresh) != 0) {
#pragma unroll
                for (int m = 0; m < 16; m += 4)
                    agpr_scale4_via_lds(oacc[rb][m], oacc[rb][m + 1], oacc[rb][m + 2], oacc[rb][m + 3], alpha, scr_addr);
                agpr_scale_via_lds(oacc[rb][16], alpha, scr_addr);
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
        half8_t pop[kFaRB], plo[kFaRB];
#pragma unroll
        for (int rb = 0; rb < kFaRB; ++rb) {
            float psum = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float p0 = __builtin_amdgcn_exp2f(sv[rb][e]);
                const float p1 = __builtin_amdgcn_exp2f(sv[rb][e + 1]);
                psum = e == 0 && kPinned ? p0 : psum + p0;
                psum += p1;
                if constexpr (kExact) {
                    half2_t ph, pl;
                    split_fp16x2(p0, vs[e], p1, vs[e + 1], ph, pl);
                    pop[rb][e] = ph.x;
                    pop[rb][e + 1] = ph.y;
                    plo[rb][e] = pl.x;
                    plo[rb][e + 1] = pl.y;
                } else if constexpr (kPinned) {
                    // p * v_scale rounded once to fp16 (v_fma_mix with a zero addend: one
                    // instruction per value, where a multiply and a packed conversion take 1.5)
                    pop[rb][e] = (_Float16)__builtin_fmaf(p0, vs[e], 0.f);
                    pop[rb][e + 1] = (_Float16)__builtin_fmaf(p1, vs[e + 1], 0.f);
                } else {
                    pop[rb][e] = (_Float16)(p0 * vs[e]);
                    pop[rb][e + 1] = (_Float16)(p1 * vs[e + 1]);
                }
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
            if constexpr (kExact) {
#pragma unroll
                for (int rb = 0; rb < kFaRB; ++rb)
                    oacc[rb][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[m], plo[rb], oacc[rb][m], 0, 0, 0);
            }
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
                const lds_int* e = pt.lds + 2 * (n - t0);
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
        for (int n = t0; n < min(t1, t0 + kFaRaw); ++n) issue(n);
        if (t1 > t0) {
            // tile t0 has landed; of the next three at most 2 are left in flight (conservative)
            wait_quarters(min(t1 - t0 - 1, 2), tail_wave);
            __syncthreads();
            widen(t0);
        }
        // Iteration n: tile n + 1 has landed and every wave is done with iteration n - 1, so
        // fp16 buffer n & 1 holds tile n and raw slot n & 3 (widened in iteration n - 1) is free
        // for tile n + 4.
        auto arrive = [&](int n) __attribute__((always_inline)) {
            if (n + 1 < t1) wait_quarters(min(2, t1 - 2 - n), tail_wave);
            __syncthreads();
            if (n + kFaRaw < t1) issue(n + kFaRaw);
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
        run(std::false_type{}, t0, min(n_int, t1));
        run(std::true_type{}, max(n_int, t0), t1);
    };
    if (pt.in_lds)
        tile_loop(std::true_type{});
    else
        tile_loop(std::false_type{});

    // ---- normalise and store: out[b, tq0 + tok, g G + hh, :]; with the keys split, the
    //      unnormalised partial O, the running max m and the sum l of the row instead ----
#pragma unroll
    for (int rb = 0; rb < kFaRB; ++rb) {
        const float l_row = xor_sum(xor_sum(l_run[rb], 16), 32);
        const float inv = l_row > 0.f ? 1.f / l_row : 0.f;
        // the V widening bias of the row, 1152 * sum of its P' (0 when V is widened exactly)
        const float corr = kExact ? 0.f : __shfl(oacc[rb][16].x, 48 + li, 64);

        if (rvalid[rb]) {
            const int r = 48 * w + 16 * rb + li;
            const int tok = r / G, hh = r - (r / G) * G;
            if constexpr (kSplit) {
                const int64_t pr = (((int64_t)b * a.Sq + tq0 + tok) * a.Hq + g * G + hh) * a.nsplit + split;
                float* prow = a.part_o + pr * kDim;
#pragma unroll
                for (int m = 0; m < 17; ++m) {
                    const int d0 = m < 16 ? 16 * m - 4 + 4 * lg : (lg == 2 ? 252 : -1);
                    if (d0 >= 0 && d0 < kDim) *reinterpret_cast<float4_t*>(prow + d0) = oacc[rb][m] - corr;
                }
                if (lg == 0) {
                    a.part_m[pr] = m_run[rb];
                    a.part_l[pr] = l_row;
                }
            } else {
                float* orow = a.out + (int64_t)b * a.o_sb + (int64_t)(tq0 + tok) * a.o_st + (int64_t)(g * G + hh) * a.o_sh;
#pragma unroll
                for (int m = 0; m < 17; ++m) {
                    const int d0 = m < 16 ? 16 * m - 4 + 4 * lg : (lg == 2 ? 252 : -1);
                    if (d0 >= 0 && d0 < kDim) *reinterpret_cast<float4_t*>(orow + d0) = (oacc[rb][m] - corr) * inv;
                }
            }
        }
    }
}

// Log-sum-exp merge of a split prefill's partials into out (fp32): one wave per row, lane l
// owns dims 4 l .. 4 l + 3. M = max_s m_s, out = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s,
// and 0 for a row no split saw a key of. Lane s reads split s's m and l (nsplit <= 64), the wave
// reduces M and L, and the O rows are loaded eight splits at a time before any is used, so a
// row costs about nsplit / 8 memory round trips. A split that saw no key of the row (m = -inf)
// is excluded by a select, not a product, so whatever its O holds cannot reach the output.
__global__ void __launch_bounds__(256) pd_prefill_combine_kernel(const FaParams a, int rows) {
    constexpr int kBatch = 8;
    const int r = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6), l = threadIdx.x & 63;
    if (r >= rows) return;
    const int ns = a.nsplit;
    const int64_t base = (int64_t)r * ns;
    const float m_mine = l < ns ? a.part_m[base + l] : kNegInf;
    const float l_mine = l < ns ? a.part_l[base + l] : 0.f;
    float M = m_mine;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    const float w_mine = m_mine != kNegInf ? exp2f(m_mine - M) : 0.f;
    float L = w_mine * l_mine;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) L += __shfl_xor(L, o, 64);
    float4_t acc = (float4_t)0.f;
    const float4_t* po = reinterpret_cast<const float4_t*>(a.part_o + base * kDim) + l;
    for (int s0 = 0; s0 < ns; s0 += kBatch) {
        float4_t o[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) o[i] = s0 + i < ns ? po[(int64_t)(s0 + i) * (kDim / 4)] : (float4_t)0.f;
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const float wi = __shfl(w_mine, min(s0 + i, 63), 64);
            acc += (s0 + i < ns && wi != 0.f) ? wi * o[i] : (float4_t)0.f;
        }
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const int hd = r % a.Hq, tok = (r / a.Hq) % a.Sq, b = r / (a.Hq * a.Sq);
    float* orow = a.out + (int64_t)b * a.o_sb + (int64_t)tok * a.o_st + (int64_t)hd * a.o_sh;
    *reinterpret_cast<float4_t*>(orow + 4 * l) = acc * inv;
}

// ---------------------------------------------------------------------------------------
// host side

template <bool kSplit>
static void launch_prefill_kernel(const FaParams& p, dim3 grid, hipStream_t stream, bool fast, bool exact) {
    const dim3 block(kFaWaves * 64);
    if (fast && !exact)
        hipLaunchKernelGGL((pd_prefill_kernel<true, false, kSplit>), grid, block, 0, stream, p);
    else if (!exact)
        hipLaunchKernelGGL((pd_prefill_kernel<false, false, kSplit>), grid, block, 0, stream, p);
    else if (fast)
        hipLaunchKernelGGL((pd_prefill_kernel<true, true, kSplit>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((pd_prefill_kernel<false, true, kSplit>), grid, block, 0, stream, p);
}

hipError_t launch_prefill(const FaParams& p, int batch, int heads_kv, hipStream_t stream, bool exact) {
    const dim3 grid(((p.Sq + p.tok_per_wg - 1) / p.tok_per_wg) * p.nsplit, heads_kv, batch);
    const bool fast = fast_block_table(p.block_size, p.k_ss);
    if (p.nsplit == 1) {
        launch_prefill_kernel<false>(p, grid, stream, fast, exact);
        return hipGetLastError();
    }
    launch_prefill_kernel<true>(p, grid, stream, fast, exact);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int rows = batch * p.Sq * p.Hq;
    hipLaunchKernelGGL(pd_prefill_combine_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, p, rows);
    return hipGetLastError();
}

}  // namespace pd
