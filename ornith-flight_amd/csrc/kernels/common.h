// SPDX-License-Identifier: MIT
//
// Device-side helpers shared by the gfx950 kernels: the reference's fp16
// conversion, K-quant scale unpacking, wave reductions, and the fixed
// super-block geometry.  Only included from .hip translation units.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../../include/ornith/kquant.h"

#define ORN_WAVE 64

// Kernel launch of a forward step: with the step's profiling events set
// (ornk_moe_args ev_start/ev_stop), hipExtLaunchKernel stamps the kernel's
// own start and end into them; otherwise a plain launch.  ORN_LAUNCH_EV2
// takes the two events explicitly (a step of two kernels passes the start
// event to its first and the stop event to its last).
#define ORN_LAUNCH_EV2(st, sp, K, grid, block, shmem, s, ...)                                  \
    do {                                                                                       \
        if ((st) || (sp))                                                                      \
            hipExtLaunchKernelGGL(K, grid, block, shmem, s, st, sp, 0u, __VA_ARGS__);          \
        else                                                                                   \
            hipLaunchKernelGGL(K, grid, block, shmem, s, __VA_ARGS__);                         \
    } while (0)
#define ORN_LAUNCH_EV(a, K, grid, block, shmem, s, ...) \
    ORN_LAUNCH_EV2((a)->ev_start, (a)->ev_stop, K, grid, block, shmem, s, __VA_ARGS__)

// Native 4-wide vector.  Loads through it are single vector loads; copying
// HIP's float4 struct from global memory lowers to a memcpy, which keeps
// register arrays of it in scratch memory.
typedef float v4f __attribute__((ext_vector_type(4)));

// gguf.c:16-26.  0x0000 -> 0; every other pattern is decoded as a normal
// number with exponent bias 112 (0x8000 -> -2^-15, subnormal patterns ->
// 2^-15*(1+m/1024), exp=31 -> 2^16*(1+m/1024)).  Pure integer work, so the
// result is bit-identical to the reference on every input.
__device__ __forceinline__ float orn_half_to_float(uint32_t h)
{
    h &= 0xFFFFu;
    const uint32_t u = ((h & 0x8000u) << 16) | ((((h & 0x7C00u) >> 10) + 112u) << 23) |
                       ((h & 0x03FFu) << 13);
    // Zero via a mask (all ones iff h != 0), not a select: the compiler
    // turns the select into a branch, which splits the callers' loops.
    const uint32_t nz = 0u - ((h + 0xFFFFu) >> 16);
    return __uint_as_float(u & nz);
}

// The same sum over a compile-time count of NB batches, fully unrolled: the
// reads of batch b+1 are issued before the adds of batch b and every add
// issues back to back (no loop counter, no per-batch wait beyond the data).
template <int NB>
__device__ __forceinline__ float orn_lds_seq_sum32_n(const v4f *p4)
{
    float ss = 0.0f;
    v4f A[8], B[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) A[i] = p4[i];
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) {
        v4f(&cur)[8] = (bt & 1) ? B : A;
        v4f(&nxt)[8] = (bt & 1) ? A : B;
        if (bt + 1 < NB) {
#pragma unroll
            for (int i = 0; i < 8; ++i) nxt[i] = p4[8 * (bt + 1) + i];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            ss += cur[i].x;
            ss += cur[i].y;
            ss += cur[i].z;
            ss += cur[i].w;
        }
        asm volatile("" : "+v"(ss));  // each batch's adds stay in their batch
    }
    return ss;
}

// Sequential fp32 sum ((0 + p[0]) + p[1]) + ... of the 32 * nb floats at p4
// (LDS), for one lane: batches of 32 in two register buffers, the reads of one
// batch issued before the adds of the other, so only the chain of adds is
// serial.  (The order and roundings of a plain loop over p.)
__device__ __forceinline__ float orn_lds_seq_sum32(const v4f *p4, int nb)
{
    float ss = 0.0f;
    v4f A[8], B[8];
    auto rd = [&](v4f(&r)[8], int bt) {
        const int b = bt < nb ? bt : nb - 1;  // past the end: re-read the last batch, unused
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = p4[8 * b + i];
    };
    auto add = [&](const v4f(&r)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            ss += r[i].x;
            ss += r[i].y;
            ss += r[i].z;
            ss += r[i].w;
        }
    };
    if (nb > 0) rd(A, 0);
    for (int bt = 0; bt < nb; bt += 2) {
        rd(B, bt + 1);
        __builtin_amdgcn_sched_barrier(0);
        add(A);
        if (bt + 1 >= nb) break;
        rd(A, bt + 2);
        __builtin_amdgcn_sched_barrier(0);
        add(B);
    }
    return ss;
}

// Empty volatile asm that reads and writes v[0..7] and clobbers memory: every
// computation of these values is ordered before it, and no load or store
// moves across it.  Used to keep a ring slot's refill after the slot's last
// use, so the refill can write the slot's own registers.
__device__ __forceinline__ void orn_pin8(float *v)
{
    asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                 "+v"(v[6]), "+v"(v[7])::"memory");
}

__device__ __forceinline__ void orn_pin2(float &a, float &b)
{
    asm volatile("" : "+v"(a), "+v"(b)::"memory");
}

// Marks the point where a ring slot's loaded registers are first used: the
// wait for the slot's loads lands here, and no use of them moves above it.
__device__ __forceinline__ void orn_pin_u4(uint4 &a)
{
    asm volatile("" : "+v"(a.x), "+v"(a.y), "+v"(a.z), "+v"(a.w));
}

// Byte i (0..3) of w as a float: one v_cvt_f32_ubyte<i>.  The word passes
// through an empty asm first, so the compiler cannot fold an earlier mask
// into a per-byte bit-field extract (two instructions per byte).
__device__ __forceinline__ void orn_bytes_to_float(uint32_t w, float *f)
{
    asm("" : "+v"(w));
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = (float)((w >> (8 * i)) & 0xFFu);
}

__device__ __forceinline__ uint32_t orn_byte(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }

// gguf.c:31-40, with the 12 packed scale bytes held as three little-endian
// dwords s0 (bytes 0-3), s1 (bytes 4-7), s2 (bytes 8-11).  Both encodings
// are computed and selected, so a wave whose lanes need different sub-blocks
// does not diverge.
__device__ __forceinline__ void orn_scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                                 uint32_t &sc, uint32_t &m)
{
    const int i = j & 3;
    const uint32_t b0 = orn_byte(s0, i), b1 = orn_byte(s1, i), b2 = orn_byte(s2, i);
    const uint32_t sc_lo = b0 & 63u, m_lo = b1 & 63u;
    const uint32_t sc_hi = (b2 & 0xFu) | ((b0 >> 6) << 4);
    const uint32_t m_hi = (b2 >> 4) | ((b1 >> 6) << 4);
    sc = j < 4 ? sc_lo : sc_hi;
    m = j < 4 ? m_lo : m_hi;
}

// Unaligned-safe little-endian byte reads (for the GGUF AoS Q6_K stream whose
// 210-byte blocks are only 2-byte aligned).
__device__ __forceinline__ uint32_t orn_ld_u8(const uint8_t *p) { return (uint32_t)(*p); }
__device__ __forceinline__ uint32_t orn_ld_u16(const uint8_t *p)
{
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8);
}

// Sum over the 64 lanes of a wave (fixed butterfly order -> deterministic).
__device__ __forceinline__ float orn_wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, ORN_WAVE);
    return v;
}
