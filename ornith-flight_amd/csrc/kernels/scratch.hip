// SPDX-License-Identifier: MIT
//
// Fixed device scratch for the MoE forward entry point that allocates
// nothing (gpu_moe_forward_noalloc).  The forward's work buffers (logits,
// selection, dispatch tables, split-K partials, mid rows, counters) are
// carved from this array instead of the context's grow-only workspace.
//
// The array is one file-scope device variable: every GPU the library runs
// on holds its own copy, at its own address, until the process ends.  The
// array's name is only a host-side stand-in for that memory: passing it to a
// kernel compiles but faults.  Host code therefore resolves each device's
// address once, with that device current (ornk_scratch_resolve, called by
// the entry point's first call on a context), and only ever passes the
// resolved address to kernels.
//
// Every call on one GPU shares that GPU's array and leaves its contents in
// place; the forward clears what must start at zero itself (its counters are
// zeroed by the routing kernel).  Calls that overlap on one GPU race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "launch.h"

// External linkage on purpose: a `static` (internal) device variable is a
// LOCAL symbol of the code object, which the loader does not export, and
// HIP's symbol lookup then aborts the process instead of returning an
// error.  The name is unique to this library.  `used`: no kernel names the
// array, so without it the device compiler would drop it.
__attribute__((used)) __device__ __align__(256) uint8_t ornk_noalloc_scratch[ORNK_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
void *g_addr[kMaxDevices];
std::mutex g_lock;

}  // namespace

extern "C" int ornk_scratch_resolve(int device, void **addr)
{
    *addr = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> guard(g_lock);
    if (!g_addr[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(ornk_noalloc_scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_addr[device] = p;
    }
    *addr = g_addr[device];
    return hipSuccess;
}
