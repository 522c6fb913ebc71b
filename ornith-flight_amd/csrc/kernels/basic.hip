// SPDX-License-Identifier: MIT
//
// fp32 element-wise and small dense kernels behind the gpu.h backend API.
// Compiled with -ffp-contract=off: every mul/add below rounds separately, in
// the order written, like the reference CPU backend (gpu.c:104-238).
#include "common.h"
#include "launch.h"

namespace {

__global__ void k_fill(float *p, float v, size_t n)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = v;
}

// gpu.c:104-115: C[i][j] = sum_k A[i][k] * B[k][j], a sequential fp32 sum
// from 0.0f with k ascending and separately rounded products, so results are
// bit-identical to the CPU backend.  A thread owns NC adjacent columns for MT
// rows (a block-row of A, MT <= 16), so every B element is read once per MT
// rows: the kernel streams B, which is what bounds it at small M (an LM head
// reads K*N floats per token), and with NC = 4 a lane's B load is one 16-byte
// word.  A is staged in LDS in chunks of MM_KC columns (every lane reads the
// same words: broadcast); the MM_U B loads of a turn are issued before their
// products.  Rows past M are zero in LDS and never stored.
constexpr int MM_KC = 256, MM_U = 8;

template <int NC>
struct ColVec;
template <>
struct ColVec<1> {
    typedef float T;
    static __device__ __forceinline__ float at(float v, int) { return v; }
};
template <>
struct ColVec<4> {
    typedef v4f T;
    static __device__ __forceinline__ float at(v4f v, int c) { return v[c]; }
};

template <int MT, int NC>
__global__ void __launch_bounds__(256) k_matmul(float *C, const float *A, const float *B, int M,
                                                int N, int K)
{
    typedef typename ColVec<NC>::T bvec;
    __shared__ __align__(16) float As[MT][MM_KC];
    const int j = (blockIdx.x * 256 + threadIdx.x) * NC;  // first column of this thread
    const int i0 = blockIdx.y * MT;
    const bool live = j < N;  // NC > 1 only when N % NC == 0: all NC columns exist
    const bvec *b = reinterpret_cast<const bvec *>(B + (live ? j : 0));
    const size_t ldb = (size_t)N / NC;  // row stride of B in bvec units
    float acc[MT][NC];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[i][c] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += MM_KC) {
        const int kc = K - k0 < MM_KC ? K - k0 : MM_KC;
        __syncthreads();  // the previous chunk is consumed
        for (int e = threadIdx.x; e < MT * MM_KC; e += 256) {
            const int i = e / MM_KC, k = e - i * MM_KC;
            As[i][k] = (i0 + i < M && k < kc) ? A[(size_t)(i0 + i) * K + k0 + k] : 0.0f;
        }
        __syncthreads();
        int k = 0;
        for (; k + MM_U <= kc; k += MM_U) {
            bvec bv[MM_U];
#pragma unroll
            for (int u = 0; u < MM_U; ++u) bv[u] = b[(size_t)(k0 + k + u) * ldb];
#pragma unroll
            for (int u = 0; u < MM_U; ++u)
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int c = 0; c < NC; ++c)
                        acc[i][c] += As[i][k + u] * ColVec<NC>::at(bv[u], c);
        }
        for (; k < kc; ++k) {
            const bvec bk = b[(size_t)(k0 + k) * ldb];
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int c = 0; c < NC; ++c) acc[i][c] += As[i][k] * ColVec<NC>::at(bk, c);
        }
    }
    if (!live) return;
#pragma unroll
    for (int i = 0; i < MT; ++i)
        if (i0 + i < M)
#pragma unroll
            for (int c = 0; c < NC; ++c) C[(size_t)(i0 + i) * N + j + c] = acc[i][c];
}

// gpu.c:144-156 per row: ss is the reference's sequential fp32 sum of the
// fp32 products x[i]*x[i], i ascending, then out = w * (x * inv_rms).  The
// products are formed by all threads into LDS (dim floats of dynamic shared
// memory); one lane then adds them in order (orn_lds_seq_sum32), so only the
// chain of adds is serial and the roundings are the reference's.
__global__ void __launch_bounds__(256) k_rmsnorm(float *out, const float *x, const float *w, int dim)
{
    extern __shared__ __align__(16) float s_p[];
    __shared__ float inv_s;
    const float *xr = x + (size_t)blockIdx.x * dim;
    float *orow = out + (size_t)blockIdx.x * dim;
    // Vector path (dim a multiple of 4, at most 16384): a thread's x and w
    // are loaded in one round trip, before the first product.
    const bool vec = (dim & 3) == 0 && dim <= 16 * 1024;
    const int n4 = dim >> 2;
    v4f xv[16], wv[16];
    if (vec) {
        const v4f *x4 = reinterpret_cast<const v4f *>(xr);
        const v4f *w4 = reinterpret_cast<const v4f *>(w);
        v4f *p4 = reinterpret_cast<v4f *>(s_p);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int i = (int)threadIdx.x + 256 * j;
            if (i < n4) {
                xv[j] = x4[i];
                wv[j] = w4[i];
            }
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int i = (int)threadIdx.x + 256 * j;
            if (i < n4) p4[i] = xv[j] * xv[j];
        }
    } else {
        for (int i = threadIdx.x; i < dim; i += blockDim.x) {
            const float v = xr[i];
            s_p[i] = v * v;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int nb = dim >> 5;
        float ss = orn_lds_seq_sum32(reinterpret_cast<const v4f *>(s_p), nb);
        for (int i = 32 * nb; i < dim; ++i) ss += s_p[i];
        inv_s = 1.0f / sqrtf(ss / (float)dim + 1e-6f);
    }
    __syncthreads();
    const float inv = inv_s;
    if (vec) {
        v4f *o4 = reinterpret_cast<v4f *>(orow);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int i = (int)threadIdx.x + 256 * j;
            if (i < n4) o4[i] = wv[j] * (xv[j] * inv);
        }
    } else {
        for (int i = threadIdx.x; i < dim; i += blockDim.x) orow[i] = w[i] * (xr[i] * inv);
    }
}

__global__ void k_silu(float *out, const float *x, int n)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        float v = x[i];
        out[i] = v / (1.0f + expf(-v));
    }
}

__global__ void k_silu_mul(float *out, const float *g, const float *u, int n)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        float v = g[i];
        out[i] = (v / (1.0f + expf(-v))) * u[i];
    }
}

__global__ void k_add(float *out, const float *a, const float *b, int n)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

// Streaming read of n16 16-byte words (grid-stride, 8 loads in flight per
// thread), folded with xor into one word per thread so the loads are live.
__global__ void __launch_bounds__(256) k_stream_read(const uint4 *__restrict__ p, size_t n16,
                                                     uint32_t *__restrict__ out)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 7 * stride < n16; i += 8 * stride) {
        uint4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = p[i + j * stride];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    for (; i < n16; i += stride) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

inline int blocks_for(size_t n, int bs) { return (int)((n + (size_t)bs - 1) / (size_t)bs); }

}  // namespace

// out: ORNK_STREAM_GRID * 256 words.
extern "C" int ornk_stream_read(const void *p, size_t bytes, uint32_t *out, hipStream_t s)
{
    hipLaunchKernelGGL(k_stream_read, dim3(ORNK_STREAM_GRID), dim3(256), 0, s,
                       reinterpret_cast<const uint4 *>(p), bytes / 16, out);
    return hipGetLastError();
}

extern "C" int ornk_fill_f32(float *p, float v, size_t n, hipStream_t s)
{
    if (n == 0) return hipSuccess;
    size_t nb = (n + 255) / 256;
    int grid = nb > 65536 ? 65536 : (int)nb;
    hipLaunchKernelGGL(k_fill, dim3(grid), dim3(256), 0, s, p, v, n);
    return hipGetLastError();
}

extern "C" int ornk_matmul_f32(float *C, const float *A, const float *B, int M, int N, int K,
                               hipStream_t s)
{
    if (M <= 0 || N <= 0) return hipSuccess;
    // rows per block-row: the smallest power of two >= M, at most 16 (a
    // register per row and column); larger M runs ceil(M/16) block-rows.
    // Up to 4 rows a thread takes 4 columns (one 16-byte B load per step)
    // where N allows it (N % 4 == 0 keeps every row 16-byte aligned).
    const int mt = M > 8 ? 16 : M > 4 ? 8 : M > 2 ? 4 : M;
    const int nc = (mt <= 4 && N % 4 == 0 && ((uintptr_t)B & 15) == 0) ? 4 : 1;
    const dim3 grid(blocks_for(((size_t)N + nc - 1) / nc, 256), (M + mt - 1) / mt);
#define ORN_MM(MT_, NC_) hipLaunchKernelGGL((k_matmul<MT_, NC_>), grid, dim3(256), 0, s, C, A, B, M, N, K)
    if (nc == 4) {
        switch (mt) {
        case 1: ORN_MM(1, 4); break;
        case 2: ORN_MM(2, 4); break;
        default: ORN_MM(4, 4); break;
        }
    } else {
        switch (mt) {
        case 1: ORN_MM(1, 1); break;
        case 2: ORN_MM(2, 1); break;
        case 4: ORN_MM(4, 1); break;
        case 8: ORN_MM(8, 1); break;
        default: ORN_MM(16, 1); break;
        }
    }
#undef ORN_MM
    return hipGetLastError();
}

extern "C" int ornk_rmsnorm(float *out, const float *x, const float *w, int rows, int dim,
                            hipStream_t s)
{
    if (rows <= 0 || dim <= 0) return hipSuccess;
    if (dim > 16384) return hipErrorInvalidValue;  // the products live in LDS
    hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(256), (size_t)dim * sizeof(float), s, out, x,
                       w, dim);
    return hipGetLastError();
}

extern "C" int ornk_silu(float *out, const float *x, int n, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_silu, dim3(blocks_for((size_t)n, 256)), dim3(256), 0, s, out, x, n);
    return hipGetLastError();
}

extern "C" int ornk_silu_mul(float *out, const float *g, const float *u, int n, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_silu_mul, dim3(blocks_for((size_t)n, 256)), dim3(256), 0, s, out, g, u, n);
    return hipGetLastError();
}

extern "C" int ornk_add(float *out, const float *a, const float *b, int n, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_add, dim3(blocks_for((size_t)n, 256)), dim3(256), 0, s, out, a, b, n);
    return hipGetLastError();
}
