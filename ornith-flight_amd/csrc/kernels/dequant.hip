// SPDX-License-Identifier: MIT
//
// GGUF dequantization on the device, bit-exact with the reference:
//   whole tensor   gguf.c:605-638  (F32 copy, F16, Q4_K, Q6_K)
//   expert slice   gguf.c:652-711  (interleaved: slice[i] = full[i*E + e])
//
// Exactness: d*sc has <= 17 significant bits (Q4_K) and d*sc*q <= 24 bits
// (Q6_K), so every product below is exact in fp32; the only rounding is
// Q4_K's final "- dmin*m", which this code performs exactly as the reference
// does.  The half decode is the reference's integer mapping (common.h).
// Whole tensors: each thread writes 4 consecutive elements with one 16-byte
// store, reading its 4 quants with one 4-byte (Q4_K: 144-byte blocks keep
// 4-byte alignment) or two 2-byte loads (Q6_K: 210-byte blocks are only
// 2-byte aligned inside a tensor); pointers without that alignment take the
// one-element-per-thread kernels, which read bytes.
#include "common.h"
#include "launch.h"

namespace {

__device__ __forceinline__ float q4k_elem(const uint8_t *blk, int pos)
{
    const int sub = pos >> 5, chunk = pos >> 6, half = (pos >> 5) & 1, l = pos & 31;
    const uint8_t *s = blk + ORN_Q4K_OFF_SCALES;
    uint32_t sc, m;
    if (sub < 4) {
        sc = s[sub] & 63u;
        m = s[sub + 4] & 63u;
    } else {
        sc = (s[sub + 4] & 0xFu) | (((uint32_t)s[sub - 4] >> 6) << 4);
        m = ((uint32_t)s[sub + 4] >> 4) | (((uint32_t)s[sub] >> 6) << 4);
    }
    const float d_val = orn_half_to_float(orn_ld_u16(blk + ORN_Q4K_OFF_D)) * (float)sc;
    const float min_val = orn_half_to_float(orn_ld_u16(blk + ORN_Q4K_OFF_DMIN)) * (float)m;
    const uint32_t b = blk[ORN_Q4K_OFF_QS + chunk * 32 + l];
    const uint32_t q = half ? (b >> 4) : (b & 0x0Fu);
    return d_val * (float)q - min_val;
}

__device__ __forceinline__ float q6k_elem(const uint8_t *blk, int pos)
{
    const int pass = pos >> 7, lane = (pos >> 5) & 3, l = pos & 31, is = l >> 4;
    const float d = orn_half_to_float(orn_ld_u16(blk + ORN_Q6K_OFF_D));
    const uint32_t qlb = blk[ORN_Q6K_OFF_QL + pass * 64 + ((lane & 1) ? 32 + l : l)];
    const uint32_t qhb = blk[ORN_Q6K_OFF_QH + pass * 32 + l];
    const uint32_t lo = (lane < 2) ? (qlb & 0x0Fu) : (qlb >> 4);
    const int q = (int)(lo | (((qhb >> (2 * lane)) & 3u) << 4)) - 32;
    const int sc = (int)(int8_t)blk[ORN_Q6K_OFF_SCALES + pass * 8 + lane * 2 + is];
    return d * (float)sc * (float)q;
}

// Elements pos0..pos0+3 (pos0 % 4 == 0: one sub-block, one qs run) of the
// block at blk, with q4k_elem's arithmetic.
__device__ __forceinline__ float4 q4k_quad(const uint8_t *blk, int pos0)
{
    const int sub = pos0 >> 5, chunk = pos0 >> 6, half = (pos0 >> 5) & 1, l = pos0 & 31;
    const uint8_t *s = blk + ORN_Q4K_OFF_SCALES;
    uint32_t sc, m;
    if (sub < 4) {
        sc = s[sub] & 63u;
        m = s[sub + 4] & 63u;
    } else {
        sc = (s[sub + 4] & 0xFu) | (((uint32_t)s[sub - 4] >> 6) << 4);
        m = ((uint32_t)s[sub + 4] >> 4) | (((uint32_t)s[sub] >> 6) << 4);
    }
    const float d_val = orn_half_to_float(orn_ld_u16(blk + ORN_Q4K_OFF_D)) * (float)sc;
    const float min_val = orn_half_to_float(orn_ld_u16(blk + ORN_Q4K_OFF_DMIN)) * (float)m;
    const uint32_t w = *reinterpret_cast<const uint32_t *>(blk + ORN_Q4K_OFF_QS + chunk * 32 + l);
    const uint32_t q = half ? (w >> 4) & 0x0F0F0F0Fu : w & 0x0F0F0F0Fu;
    return make_float4(d_val * (float)(q & 0xFFu) - min_val, d_val * (float)((q >> 8) & 0xFFu) - min_val,
                       d_val * (float)((q >> 16) & 0xFFu) - min_val, d_val * (float)(q >> 24) - min_val);
}

// The same for Q6_K (pos0 % 4 == 0: one pass, lane and scale).
__device__ __forceinline__ float4 q6k_quad(const uint8_t *blk, int pos0)
{
    const int pass = pos0 >> 7, lane = (pos0 >> 5) & 3, l = pos0 & 31, is = l >> 4;
    const float d = orn_half_to_float(orn_ld_u16(blk + ORN_Q6K_OFF_D));
    const uint8_t *qlp = blk + ORN_Q6K_OFF_QL + pass * 64 + ((lane & 1) ? 32 + l : l);
    const uint8_t *qhp = blk + ORN_Q6K_OFF_QH + pass * 32 + l;
    // every offset here is even, and the launcher checked that src is
    const uint16_t *ql16 = reinterpret_cast<const uint16_t *>(qlp);
    const uint16_t *qh16 = reinterpret_cast<const uint16_t *>(qhp);
    const uint32_t qlw = (uint32_t)ql16[0] | ((uint32_t)ql16[1] << 16);
    const uint32_t qhw = (uint32_t)qh16[0] | ((uint32_t)qh16[1] << 16);
    const uint32_t lo = (lane < 2) ? (qlw & 0x0F0F0F0Fu) : ((qlw >> 4) & 0x0F0F0F0Fu);
    const uint32_t hi = ((qhw >> (2 * lane)) & 0x03030303u) << 4;
    const uint32_t q = lo | hi;  // four 6-bit values, one per byte
    const float ds = d * (float)(int)(int8_t)blk[ORN_Q6K_OFF_SCALES + pass * 8 + lane * 2 + is];
    return make_float4(ds * (float)((int)(q & 0xFFu) - 32), ds * (float)((int)((q >> 8) & 0xFFu) - 32),
                       ds * (float)((int)((q >> 16) & 0xFFu) - 32), ds * (float)((int)(q >> 24) - 32));
}

// 64 threads per block of 256 elements, four blocks per work group pass.
// Outputs are written once and not read here again: non-temporal stores,
// each instruction 1 KB contiguous per wave.
template <bool Q6>
__global__ void __launch_bounds__(256) k_dequant_quad(const uint8_t *src, float4 *dst, uint64_t n_blocks)
{
    const int sub_blk = threadIdx.x >> 6, pos0 = 4 * (threadIdx.x & 63);
    for (uint64_t b = (uint64_t)blockIdx.x * 4 + sub_blk; b < n_blocks; b += (uint64_t)gridDim.x * 4) {
        const float4 v = Q6 ? q6k_quad(src + b * ORN_Q6K_BYTES, pos0)
                            : q4k_quad(src + b * ORN_Q4K_BYTES, pos0);
        __builtin_nontemporal_store(__builtin_bit_cast(v4f, v),
                                    reinterpret_cast<v4f *>(dst + b * (ORN_QK_K / 4) + (pos0 >> 2)));
    }
}

// Q4_K, src and dst 16-byte aligned (a 144-byte block is nine 16-byte
// words): 16 lanes per block and a header word (d, dmin, scales) they share.
// Store i of lane l writes outputs 64i + 4l .. +3, so that each store
// instruction covers 256 contiguous bytes per block (1 KB per wave, written
// non-temporally): sub-block j = 2i + l/8, from the quant word at bytes
// 16 + 32i + 4(l&7) (low nibbles for even j, high for odd), with the
// reference's arithmetic: d1 = d*sc, m1 = dmin*m, y = d1*q - m1
// (gguf.c:43-61).  (Lane l writing outputs 16l..16l+15, 64-byte strided per
// instruction, ran at 3.4 TB/s; this at 6.2.)
__global__ void __launch_bounds__(256) k_dequant_q4k16(const uint4 *__restrict__ src,
                                                       v4f *__restrict__ dst, uint64_t n_blocks)
{
    const int l = threadIdx.x & 15;
    for (uint64_t b = (uint64_t)blockIdx.x * 16 + (threadIdx.x >> 4); b < n_blocks;
         b += (uint64_t)gridDim.x * 16) {
        const uint4 *blk = src + b * (ORN_Q4K_BYTES / 16);
        const uint4 hd = blk[0];
        const uint32_t *qs = reinterpret_cast<const uint32_t *>(blk + 1);
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = qs[8 * i + (l & 7)];
        const float d = orn_half_to_float(hd.x & 0xFFFFu), dm = orn_half_to_float(hd.x >> 16);
        const uint32_t sh = 4u * (uint32_t)(l >> 3);
        v4f *o = dst + b * (ORN_QK_K / 4) + l;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t sc, m;
            orn_scale_min_k4(2 * i + (l >> 3), hd.y, hd.z, hd.w, sc, m);
            const float d1 = d * (float)sc, m1 = dm * (float)m;
            const uint32_t q = (w[i] >> sh) & 0x0F0F0F0Fu;
            const v4f r = {d1 * (float)(q & 0xFFu) - m1, d1 * (float)((q >> 8) & 0xFFu) - m1,
                           d1 * (float)((q >> 16) & 0xFFu) - m1, d1 * (float)(q >> 24) - m1};
            __builtin_nontemporal_store(r, &o[16 * i]);
        }
    }
}

__global__ void k_dequant_q4k(const uint8_t *src, float *dst, uint64_t n_blocks)
{
    for (uint64_t b = blockIdx.x; b < n_blocks; b += gridDim.x)
        __builtin_nontemporal_store(q4k_elem(src + b * ORN_Q4K_BYTES, (int)threadIdx.x),
                                    dst + b * ORN_QK_K + threadIdx.x);
}

__global__ void k_dequant_q6k(const uint8_t *src, float *dst, uint64_t n_blocks)
{
    for (uint64_t b = blockIdx.x; b < n_blocks; b += gridDim.x)
        __builtin_nontemporal_store(q6k_elem(src + b * ORN_Q6K_BYTES, (int)threadIdx.x),
                                    dst + b * ORN_QK_K + threadIdx.x);
}

__global__ void k_dequant_f16(const uint8_t *src, float *dst, uint64_t n)
{
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        __builtin_nontemporal_store(orn_half_to_float(orn_ld_u16(src + 2 * i)), dst + i);
}

// One output element per thread: linear = i*E + e, then the single-element
// extractor of the block that holds it (gguf.c:686-706).
__global__ void k_slice(const uint8_t *src, int type, uint64_t per, uint64_t n_experts,
                        uint64_t e, float *dst)
{
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < per; i += stride) {
        const uint64_t lin = i * n_experts + e;
        float v;
        if (type == ORN_TYPE_Q4_K)
            v = q4k_elem(src + (lin / ORN_QK_K) * ORN_Q4K_BYTES, (int)(lin % ORN_QK_K));
        else if (type == ORN_TYPE_Q6_K)
            v = q6k_elem(src + (lin / ORN_QK_K) * ORN_Q6K_BYTES, (int)(lin % ORN_QK_K));
        else if (type == ORN_TYPE_F16)
            v = orn_half_to_float(orn_ld_u16(src + 2 * lin));
        else
            v = reinterpret_cast<const float *>(src)[lin];
        __builtin_nontemporal_store(v, dst + i);
    }
}

inline int grid_cap(uint64_t n, uint64_t per_block)
{
    uint64_t g = (n + per_block - 1) / per_block;
    return g > 65536 ? 65536 : (int)(g ? g : 1);
}

}  // namespace

extern "C" int ornk_dequant(const void *src, int type, uint64_t n_elems, float *dst, hipStream_t s)
{
    const uint8_t *p = static_cast<const uint8_t *>(src);
    const uint64_t nb = n_elems / ORN_QK_K;
    switch (type) {
    case ORN_TYPE_F32:
        if (n_elems == 0) return hipSuccess;
        return hipMemcpyAsync(dst, src, n_elems * 4, hipMemcpyDeviceToDevice, s);
    case ORN_TYPE_F16:
        if (n_elems == 0) return hipSuccess;
        hipLaunchKernelGGL(k_dequant_f16, dim3(grid_cap(n_elems, 256)), dim3(256), 0, s, p, dst,
                           n_elems);
        return hipGetLastError();
    case ORN_TYPE_Q4_K:
        if (nb == 0) return hipSuccess;
        if (((uintptr_t)p & 15) == 0 && ((uintptr_t)dst & 15) == 0)
            hipLaunchKernelGGL(k_dequant_q4k16, dim3(grid_cap(nb, 16)), dim3(256), 0, s,
                               reinterpret_cast<const uint4 *>(p), reinterpret_cast<v4f *>(dst), nb);
        else if (((uintptr_t)p & 3) == 0 && ((uintptr_t)dst & 15) == 0)
            hipLaunchKernelGGL(k_dequant_quad<false>, dim3(grid_cap(nb, 4)), dim3(256), 0, s, p,
                               reinterpret_cast<float4 *>(dst), nb);
        else
            hipLaunchKernelGGL(k_dequant_q4k, dim3(grid_cap(nb, 1)), dim3(ORN_QK_K), 0, s, p, dst, nb);
        return hipGetLastError();
    case ORN_TYPE_Q6_K:
        if (nb == 0) return hipSuccess;
        if (((uintptr_t)p & 1) == 0 && ((uintptr_t)dst & 15) == 0)
            hipLaunchKernelGGL(k_dequant_quad<true>, dim3(grid_cap(nb, 4)), dim3(256), 0, s, p,
                               reinterpret_cast<float4 *>(dst), nb);
        else
            hipLaunchKernelGGL(k_dequant_q6k, dim3(grid_cap(nb, 1)), dim3(ORN_QK_K), 0, s, p, dst, nb);
        return hipGetLastError();
    default:
        return hipErrorInvalidValue;
    }
}

extern "C" int ornk_dequant_slice(const void *src, int type, uint64_t n_elems, uint64_t n_experts,
                                  int expert, float *dst, hipStream_t s)
{
    if (n_experts == 0 || expert < 0 || (uint64_t)expert >= n_experts) return hipErrorInvalidValue;
    if (type != ORN_TYPE_F32 && type != ORN_TYPE_F16 && type != ORN_TYPE_Q4_K &&
        type != ORN_TYPE_Q6_K)
        return hipErrorInvalidValue;
    const uint64_t per = n_elems / n_experts;
    if (per == 0) return hipSuccess;
    hipLaunchKernelGGL(k_slice, dim3(grid_cap(per, 256)), dim3(256), 0, s,
                       static_cast<const uint8_t *>(src), type, per, n_experts, (uint64_t)expert,
                       dst);
    return hipGetLastError();
}
