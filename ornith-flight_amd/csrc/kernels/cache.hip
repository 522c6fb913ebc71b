// SPDX-License-Identifier: MIT
//
// Expert loads of a streamed store (csrc/host/cache.c): the decode-layout
// blocks of each missing expert are read straight from the host tier
// (pinned host memory mapped into the device's address space) by one
// kernel for all of a forward's misses, instead of four DMA copies per
// expert.  Each load is (key, slot): expert `key` of the tier goes to device
// slot `slot`.
#include "common.h"
#include "launch.h"

namespace {

// blockIdx.y = load; the x blocks of a load stride over its 16-byte chunks:
// gate (nb*144 B), up (nb*144 B), down bodies (nb*208 B), down d (nb*2 B).
// Block 0 of a load also records the slot (for the packer) and zeroes the
// slot's dmax entries (the packer's atomic maxima start from 0).
__global__ void __launch_bounds__(256)
    k_cache_gather(const int2 *__restrict__ loads, int n, const uint4 *__restrict__ hg,
                   const uint4 *__restrict__ hu, const uint4 *__restrict__ hb,
                   const uint4 *__restrict__ hd, uint4 *__restrict__ g, uint4 *__restrict__ u,
                   uint4 *__restrict__ b, uint4 *__restrict__ d, int *__restrict__ slots_out,
                   float *__restrict__ dmax, size_t nb)
{
    const int i = blockIdx.y;
    if (i >= n) return;
    const int2 ld = loads[i];
    const size_t key = (size_t)ld.x, slot = (size_t)ld.y;
    const size_t n1 = nb * 9, n2 = nb * 13, n3 = nb / 8;  // 16-byte chunks per array
    const size_t total = 2 * n1 + n2 + n3;
    for (size_t j = (size_t)blockIdx.x * blockDim.x + threadIdx.x; j < total;
         j += (size_t)gridDim.x * blockDim.x) {
        if (j < n1) {
            g[slot * n1 + j] = hg[key * n1 + j];
        } else if (j < 2 * n1) {
            const size_t o = j - n1;
            u[slot * n1 + o] = hu[key * n1 + o];
        } else if (j < 2 * n1 + n2) {
            const size_t o = j - 2 * n1;
            b[slot * n2 + o] = hb[key * n2 + o];
        } else {
            const size_t o = j - 2 * n1 - n2;
            d[slot * n3 + o] = hd[key * n3 + o];
        }
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) slots_out[i] = (int)slot;
    if (dmax && blockIdx.x == 0 && threadIdx.x < 3) dmax[slot * 3 + threadIdx.x] = 0.0f;
}

}  // namespace

extern "C" int ornk_cache_gather(const ornk_gather_args *a, hipStream_t s)
{
    if (a->n <= 0) return hipSuccess;
    if (a->nb % 8) return hipErrorInvalidValue;
    // ~4 MB of blocks in flight per load at the Ornith shape: 64 work groups
    // of 256 threads each (8 chunks a thread)
    const unsigned gx = (unsigned)((a->nb * 31 / 8 + 255) / 256 < 64 ? (a->nb * 31 / 8 + 255) / 256
                                                                      : 64);
    hipLaunchKernelGGL(k_cache_gather, dim3(gx, (unsigned)a->n), dim3(256), 0, s,
                       reinterpret_cast<const int2 *>(a->loads), a->n,
                       reinterpret_cast<const uint4 *>(a->h_gate),
                       reinterpret_cast<const uint4 *>(a->h_up),
                       reinterpret_cast<const uint4 *>(a->h_body),
                       reinterpret_cast<const uint4 *>(a->h_d), reinterpret_cast<uint4 *>(a->gate),
                       reinterpret_cast<uint4 *>(a->up), reinterpret_cast<uint4 *>(a->body),
                       reinterpret_cast<uint4 *>(a->d), a->slots_out, a->dmax, a->nb);
    return hipGetLastError();
}
