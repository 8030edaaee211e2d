// KV-cache writer: the producer of the 520-byte rows (vLLM's cache update for int8
// per-token-head KV, called as do_kv_cache_update(layer, key, value, kv_cache, slot_mapping),
// upstream/pr-dflash2/0002-fix-gfx906-keep-the-drafter-s-sliding-window-in-the-.patch:81-87).
// Large calls (>= 4,096 rows (token, kv head)) take four rows per wave, 16 lanes per row: lane i
// of a row holds elements 4 (16 j + i) .. + 3 for j = 0..3 of K and of V, so each of its four
// loads and four stores per tensor covers a contiguous stretch of the row across the 16 lanes,
// and a wave keeps 4 KiB of loads in flight (one row per wave keeps 1 KiB, too little to cover
// the memory latency: 32,768 tokens x 4 kv heads 67.7 -> 49.9 us). Small calls keep one row per
// wave, 4 elements per lane, where the longer chain of divisions per lane would be exposed.
// Calls of at least 16,384 rows quantise through the row's inverse scale (quant4_inv), with the
// division kept where the result could differ.
// absmax by DPP rotations inside 16-lane rows (and two cross-row steps for whole-wave rows),
// scale = absmax / 127 (0 for an all-zero row), q = clamp(rint(x / scale), -127, 127) with
// x / scale correctly rounded; the row's K bytes, k_scale, V bytes and v_scale are written with
// 4-byte stores (the V bytes start at byte 260 of the row, 4-byte aligned). Tokens whose slot is
// negative (padding) or past the cache are skipped.
#include <type_traits>

#include "pd_tile.hpp"
#include "pth_dec.h"

namespace pd {

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

// quant4 through y = x * inv, inv = 1 / scale rounded once per row: y is within 2^-15 of the
// correctly rounded x / scale (|x / scale| <= 127, so both carry relative errors below 2^-23),
// hence rint(y) is the same integer unless y lies within 2^-14 of a half-integer. Those values,
// and rows whose inverse is not finite, take the division itself, so the bytes are exactly
// quant4's.
__device__ __forceinline__ unsigned quant4_inv(float4_t x, float scale, float inv) {
    if (scale == 0.f) return 0u;
    const float y[4] = {x.x * inv, x.y * inv, x.z * inv, x.w * inv};
    bool near = !__builtin_isfinite(inv);
#pragma unroll
    for (int e = 0; e < 4; ++e) near = near || fabsf(y[e] - __builtin_floorf(y[e]) - 0.5f) < 0x1p-14f;
    if (near) return quant4(x, scale);
    unsigned r = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        r |= ((unsigned)((int)fminf(fmaxf(__builtin_rintf(y[e]), -127.f), 127.f) & 0xff)) << (8 * e);
    return r;
}

// Max over the 16 lanes of a DPP row, in every lane of the row (rotations by 8, 4, 2, 1).
__device__ __forceinline__ float row16_max(float v) {
    auto ror = [](float x, auto ctrl) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                     decltype(ctrl)::value, 0xf, 0xf, false));
    };
    v = fmaxf(v, ror(v, std::integral_constant<int, 0x128>{}));  // row_ror:8
    v = fmaxf(v, ror(v, std::integral_constant<int, 0x124>{}));  // row_ror:4
    v = fmaxf(v, ror(v, std::integral_constant<int, 0x122>{}));  // row_ror:2
    return fmaxf(v, ror(v, std::integral_constant<int, 0x121>{}));  // row_ror:1
}

__device__ __forceinline__ float absmax4(float4_t x) {
    return fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
}

// Rows (token, kv head) from which a call takes four rows per wave, and from which it quantises
// through the row's inverse scale (32,768 tokens x 4 kv heads 50.4 -> 47.8 us, 8,192 tokens
// 16.9 -> 16.5; below the bound the longer code measured slower: 1,024 tokens 5.25 -> 5.64 us,
// 2,048 tokens 7.15 -> 7.41).
constexpr int64_t kKvwRowsSplit = 4096;
constexpr int64_t kKvwRowsInv = 16384;

// kRows rows per wave, 64 / kRows lanes per row.
template <class In, int kRows, bool kInv>
__global__ void __launch_bounds__(256) pd_cache_write_kernel(const CacheWriteParams a) {
    constexpr int kLanes = 64 / kRows;
    const int l = threadIdx.x & 63, i = l % kLanes;
    const int row = (blockIdx.x * 4 + (threadIdx.x >> 6)) * kRows + l / kLanes;
    if (row >= a.T * a.Hkv) return;
    const int t = row / a.Hkv, h = row - t * a.Hkv;
    const int64_t slot = a.slots[t];
    if (slot < 0 || slot >= a.num_slots) return;
    // (the lanes of a row are all present or all gone, so the reductions only read lanes of
    // their own row)
    const In* kin = static_cast<const In*>(a.key) + t * a.k_st + h * a.k_sh + 4 * i;
    const In* vin = static_cast<const In*>(a.value) + t * a.v_st + h * a.v_sh + 4 * i;
    float4_t k[kRows], v[kRows];
#pragma unroll
    for (int j = 0; j < kRows; ++j) k[j] = load4(kin + 4 * kLanes * j);
#pragma unroll
    for (int j = 0; j < kRows; ++j) v[j] = load4(vin + 4 * kLanes * j);
    float km = absmax4(k[0]), vm = absmax4(v[0]);
#pragma unroll
    for (int j = 1; j < kRows; ++j) {
        km = fmaxf(km, absmax4(k[j]));
        vm = fmaxf(vm, absmax4(v[j]));
    }
    km = row16_max(km);
    vm = row16_max(vm);
    if constexpr (kRows == 1) {
#pragma unroll
        for (int o = 16; o <= 32; o <<= 1) {
            km = fmaxf(km, __shfl_xor(km, o, 64));
            vm = fmaxf(vm, __shfl_xor(vm, o, 64));
        }
    }
    const float ks = km / 127.f, vs = vm / 127.f;
    const int64_t blk = slot / a.block_size, off = slot - blk * a.block_size;
    int8_t* r = a.kc + blk * a.k_sb + off * a.k_ss + h * a.k_sh_c;
    // kInv (calls of at least kKvwRowsInv rows): quantise through the row's inverse scale.
    auto quant = [&](float4_t x, float scale, float inv) {
        if constexpr (kInv)
            return quant4_inv(x, scale, inv);
        else
            return quant4(x, scale);
    };
    const float kinv = 1.f / ks, vinv = 1.f / vs;
#pragma unroll
    for (int j = 0; j < kRows; ++j) reinterpret_cast<unsigned*>(r)[kLanes * j + i] = quant(k[j], ks, kinv);
#pragma unroll
    for (int j = 0; j < kRows; ++j) reinterpret_cast<unsigned*>(r + 260)[kLanes * j + i] = quant(v[j], vs, vinv);
    if (i == 0) {
        *reinterpret_cast<float*>(r + 256) = ks;
        *reinterpret_cast<float*>(r + 516) = vs;
    }
}

// ---------------------------------------------------------------------------------------
// host side

template <int kRows, bool kInv>
static void launch_rows(const CacheWriteParams& p, int dtype, hipStream_t stream) {
    const int64_t rows_per_wg = 4 * kRows;
    const dim3 grid((unsigned)(((int64_t)p.T * p.Hkv + rows_per_wg - 1) / rows_per_wg));
    if (dtype == PD_DTYPE_FP16)
        hipLaunchKernelGGL((pd_cache_write_kernel<_Float16, kRows, kInv>), grid, dim3(256), 0, stream, p);
    else if (dtype == PD_DTYPE_BF16)
        hipLaunchKernelGGL((pd_cache_write_kernel<__bf16, kRows, kInv>), grid, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL((pd_cache_write_kernel<float, kRows, kInv>), grid, dim3(256), 0, stream, p);
}

hipError_t launch_cache_write(const CacheWriteParams& p, int dtype, hipStream_t stream) {
    const int64_t rows = (int64_t)p.T * p.Hkv;
    if (rows >= kKvwRowsInv)
        launch_rows<4, true>(p, dtype, stream);
    else if (rows >= kKvwRowsSplit)
        launch_rows<4, false>(p, dtype, stream);
    else
        launch_rows<1, false>(p, dtype, stream);
    return hipGetLastError();
}

}  // namespace pd
