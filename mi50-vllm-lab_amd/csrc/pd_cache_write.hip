// KV-cache writer: the producer of the 520-byte rows (vLLM's cache update for int8
// per-token-head KV, called as do_kv_cache_update(layer, key, value, kv_cache, slot_mapping),
// upstream/pr-dflash2/0002-fix-gfx906-keep-the-drafter-s-sliding-window-in-the-.patch:81-87).
// One wave per (token, kv head): 64 lanes x 4 elements of K and of V; absmax by a wave
// reduction, scale = absmax / 127 (0 for an all-zero row), q = clamp(rint(x / scale), -127, 127)
// with x / scale correctly rounded; the row's K bytes, k_scale, V bytes and v_scale are written
// with 4-byte stores. Tokens whose slot is negative (padding) or past the cache are skipped.
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

hipError_t launch_cache_write(const CacheWriteParams& p, int dtype, hipStream_t stream) {
    const dim3 grid((unsigned)(((int64_t)p.T * p.Hkv + 3) / 4));
    if (dtype == PD_DTYPE_FP16)
        hipLaunchKernelGGL((pd_cache_write_kernel<_Float16>), grid, dim3(256), 0, stream, p);
    else if (dtype == PD_DTYPE_BF16)
        hipLaunchKernelGGL((pd_cache_write_kernel<__bf16>), grid, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL((pd_cache_write_kernel<float>), grid, dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace pd
