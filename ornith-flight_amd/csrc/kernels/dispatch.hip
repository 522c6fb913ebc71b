// SPDX-License-Identifier: MIT
//
// Top-k selection and token -> expert dispatch of the routed-MoE step.
//
// Selection (model.c:301-317 renormalised, model.c:1027-1049 literal) is
// exchange selection with strict '>'.  When the top k+1 logits are finite
// and pairwise distinct, exchange selection returns them in value order, so
// a wave finds them with k+1 rounds of "wave max, check it is unique,
// remove it" (DPP reductions, ballots); in the literal mode their gaps must
// also exceed 1e-5, so that their probabilities keep that order.  Otherwise
// (ties, NaN/Inf) one lane runs the reference's selection literally on this
// device's values.
//
// Dispatch (one work group): list position j = 0 is the shared expert
// (expert id E), j >= 1 routed expert j-1.  It produces the active slots
// (shared first, then experts in ascending id), their row ranges, the work
// items (<= tchunk rows each, expert id in the 4th word) and the
// row <-> (token, selection slot) maps.  Pairs with w < 1e-6 are skipped
// (model.c:1066).  Scans are wave-level DPP scans joined through LDS.
//
// One token: a single wave selects and dispatches (k_select_dispatch1).  Up
// to ORN_FUSED_SELECT_T tokens, selection and dispatch run in one work group
// of 16 waves (one launch); above, k_select (a wave per token) then
// k_dispatch.
#include "common.h"
#include "launch.h"
#include "select.h"

#include <climits>
#include <math.h>

// Fused selection + dispatch up to 16 tokens (one token per wave): a wave
// selects one token in ~2 us, so from 17 tokens on the separate k_select
// (a wave per token over many work groups) and k_dispatch launches are
// faster (measured at 64 tokens: 13.6 against 24.4 us).
#define ORN_FUSED_SELECT_T 16

namespace {

using namespace orn_sel;

__global__ void __launch_bounds__(256)
    k_select(const float *__restrict__ logits, int T, int E, int k, int mode,
             uint32_t *__restrict__ idx_out, float *__restrict__ w_out, int *n_slow)
{
    __shared__ float sv[4][256];
    __shared__ int si[4][256];
    const int wave = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wave;
    if (t >= T) return;  // a wave is a token: no block-wide barrier
    select_token(logits + (size_t)t * E, E, k, mode, idx_out + (size_t)t * k,
                 w_out + (size_t)t * k, nullptr, nullptr, sv[wave], si[wave], n_slow);
}

// ---------------------------------------------------------------------------
// Dispatch core, one work group of 1024 threads; sel_idx/sel_w may live in
// LDS or global memory (visible to the whole group on entry).
// ---------------------------------------------------------------------------


#define ORN_DU 8  // pairs read per thread at a time in dispatch_group

// Keys of pairs p0 + 1024 u, u < ORN_DU (0xFFFFFFFF past P).  The loads
// are unconditional, at an index clamped to P - 1 (P >= 1 when called), so
// that all of them are in flight before the first is used.
template <typename IdxT>
__device__ __forceinline__ void dispatch_keys(uint32_t (&ev)[ORN_DU], int p0, int P,
                                              const IdxT *sel_idx, const float *sel_w, int ep_lo,
                                              int ep_n)
{
    IdxT iv[ORN_DU];
    float wv[ORN_DU];
#pragma unroll
    for (int u = 0; u < ORN_DU; ++u) {
        const int p = min(p0 + u * 1024, P - 1);
        iv[u] = sel_idx[p];
        wv[u] = sel_w[p];
    }
#pragma unroll
    for (int u = 0; u < ORN_DU; ++u)
        ev[u] = p0 + u * 1024 < P ? dispatch_key(iv[u], wv[u], ep_lo, ep_n) : 0xFFFFFFFFu;
}

template <typename IdxT>
__device__ void dispatch_group(DispatchLds &L, const IdxT *sel_idx, const float *sel_w, int T,
                               int k, int E, int ep_lo, int ep_n, int has_shared, int *ctl,
                               int *slot_expert,
                               int *slot_off, int *slot_cnt, int *row_token, int *pair_row,
                               int4 *items, int items_max, int tchunk)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int NJ = E + 1;
    const int P = T * k;
    L.cnt[tid] = 0;
    L.cursor[tid] = 0;
    __syncthreads();
    // Pairs are read ORN_DU at a time per thread, so that a thread has that
    // many loads in flight rather than one per loop turn (16 turns at 2048
    // tokens).  An index outside [0, E) cannot come out of the router; it
    // lies outside every share, so it is skipped rather than trusted.
    for (int p0 = tid; p0 < P; p0 += ORN_DU * 1024) {
        uint32_t ev[ORN_DU];
        dispatch_keys(ev, p0, P, sel_idx, sel_w, ep_lo, ep_n);
#pragma unroll
        for (int u = 0; u < ORN_DU; ++u)
            if (ev[u] != 0xFFFFFFFFu) atomicAdd(&L.cnt[ev[u] + 1], 1);
    }
    if (tid == 0) L.cnt[0] = has_shared ? T : 0;
    __syncthreads();

    const int c = tid < NJ ? L.cnt[tid] : 0;
    const int flag = c > 0 ? 1 : 0;
    const int nit = (c + tchunk - 1) / tchunk;
    const int s_flag = wave_incl_scan(flag), s_c = wave_incl_scan(c), s_nit = wave_incl_scan(nit);
    if (lane == 63) {
        L.wtot[0][wave] = s_flag;
        L.wtot[1][wave] = s_c;
        L.wtot[2][wave] = s_nit;
    }
    __syncthreads();
    int o_flag = 0, o_c = 0, o_nit = 0, n_slots = 0, n_rows = 0, n_items = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
        const int a = L.wtot[0][w], b = L.wtot[1][w], d = L.wtot[2][w];
        if (w < wave) {
            o_flag += a;
            o_c += b;
            o_nit += d;
        }
        n_slots += a;
        n_rows += b;
        n_items += d;
    }
    const int slot = o_flag + s_flag - flag;
    const int roff = o_c + s_c - c;
    const int ioff = o_nit + s_nit - nit;
    L.rowoff[tid] = roff;
    if (flag) {
        const int ex = tid == 0 ? E : tid - 1;
        slot_expert[slot] = ex;
        slot_off[slot] = roff;
        slot_cnt[slot] = c;
        for (int q = 0; q < nit && ioff + q < items_max; ++q) {
            const int r0 = q * tchunk;
            items[ioff + q] = make_int4(slot, roff + r0, min(tchunk, c - r0), ex);
        }
    }
    if (tid == 0) {
        ctl[0] = n_slots;
        ctl[1] = n_items < items_max ? n_items : items_max;
        ctl[2] = n_rows;
    }
    __syncthreads();

    for (int p0 = tid; p0 < P; p0 += ORN_DU * 1024) {
        uint32_t ev[ORN_DU];
        dispatch_keys(ev, p0, P, sel_idx, sel_w, ep_lo, ep_n);
#pragma unroll
        for (int u = 0; u < ORN_DU; ++u) {
            const int p = p0 + u * 1024;
            if (p >= P) break;
            if (ev[u] == 0xFFFFFFFFu) {  // skipped, or another rank's expert
                pair_row[p] = -1;
                continue;
            }
            const int j = (int)ev[u] + 1;
            const int r = L.rowoff[j] + atomicAdd(&L.cursor[j], 1);
            row_token[r] = p / k;
            pair_row[p] = r;
        }
    }
    if (has_shared)
        for (int t = tid; t < T; t += 1024) row_token[L.rowoff[0] + t] = t;
}

__global__ void __launch_bounds__(1024)
    k_dispatch(const uint32_t *__restrict__ idx, const float *__restrict__ w, int T, int k, int E,
               int ep_lo, int ep_n, int has_shared, int *ctl, int *slot_expert, int *slot_off, int *slot_cnt,
               int *row_token, int *pair_row, int4 *items, int items_max,
               int tchunk)
{
    __shared__ DispatchLds L;
    dispatch_group(L, idx, w, T, k, E, ep_lo, ep_n, has_shared, ctl, slot_expert, slot_off, slot_cnt,
                   row_token, pair_row, items, items_max, tchunk);
}

// Selection of T <= ORN_FUSED_SELECT_T tokens (wave w: token w) followed by
// the dispatch, in one work group.
__global__ void __launch_bounds__(1024)
    k_select_dispatch(const float *__restrict__ logits, int T, int E, int k, int mode,
                      uint32_t *__restrict__ idx_out, float *__restrict__ w_out, int ep_lo,
                      int ep_n, int has_shared, int *ctl, int *slot_expert, int *slot_off,
                      int *slot_cnt, int *row_token, int *pair_row, int4 *items, int items_max,
                      int tchunk)
{
    __shared__ DispatchLds L;
    __shared__ float sv[16][256];
    __shared__ int si[16][256];
    __shared__ int lidx[ORN_FUSED_SELECT_T * 16];
    __shared__ float lw[ORN_FUSED_SELECT_T * 16];
    const int wave = threadIdx.x >> 6;
    if (wave < T)  // T <= 16: one token per wave
        select_token(logits + (size_t)wave * E, E, k, mode, idx_out + (size_t)wave * k,
                     w_out + (size_t)wave * k, lidx + wave * k, lw + wave * k, sv[wave], si[wave],
                     ctl + 3);
    __syncthreads();
    // the dispatch of <= 256 pairs by one wave (measured at 16 tokens: the
    // kernel 0.6 us shorter than with the 16-wave dispatch_group; the
    // group is faster from ~500 pairs)
    if (wave == 0)
        dispatch_wave(L, lidx, lw, T, k, E, ep_lo, ep_n, has_shared, ctl, slot_expert, slot_off,
                      slot_cnt, row_token, pair_row, items, items_max, tchunk);
}

// One token: selection and dispatch by a single wave, with no work-group
// barrier (orn_sel::dispatch_one).
__global__ void __launch_bounds__(64)
    k_select_dispatch1(const float *__restrict__ logits, int E, int k, int mode,
                       uint32_t *__restrict__ idx_out, float *__restrict__ w_out, int ep_lo,
                       int ep_n, int has_shared, int *ctl, int *slot_expert, int *slot_off,
                       int *slot_cnt, int *row_token, int *pair_row, int4 *items, int items_max)
{
    __shared__ float sv[256];
    __shared__ int si[256];
    __shared__ int lidx[16];
    __shared__ float lw[16];
    select_token(logits, E, k, mode, idx_out, w_out, lidx, lw, sv, si, ctl + 3);
    wave_sync();
    dispatch_one(lidx, lw, E, k, ep_lo, ep_n, has_shared, ctl, slot_expert, slot_off, slot_cnt,
                 row_token, pair_row, items, items_max, nullptr);
}

// Expert ids -> cache slots, in place, for a store that streams its experts
// through a fixed set of device slots: items[i].w for the forward's items and
// slot_expert[s] for its slots.  Every id the dispatch wrote has an entry
// (the host filled remap from slot_expert itself).
__global__ void k_remap_items(int4 *items, int *slot_expert, const int *ctl,
                              const int *__restrict__ remap, int items_max, int slots_max)
{
    const int n_items = min(ctl[1], items_max), n_slots = min(ctl[0], slots_max);
    for (int i = threadIdx.x; i < n_items; i += blockDim.x) items[i].w = remap[items[i].w];
    for (int i = threadIdx.x; i < n_slots; i += blockDim.x) slot_expert[i] = remap[slot_expert[i]];
}

}  // namespace

extern "C" int ornk_remap_items(int *items, int *slot_expert, const int *ctl, const int *remap,
                                int items_max, int slots_max, hipStream_t s)
{
    hipLaunchKernelGGL(k_remap_items, dim3(1), dim3(1024), 0, s, reinterpret_cast<int4 *>(items),
                       slot_expert, ctl, remap, items_max, slots_max);
    return hipGetLastError();
}

// Selection + dispatch step of the MoE forward (after the router).
extern "C" int ornk_moe_dispatch(const ornk_moe_args *a, hipStream_t s)
{
    const int T = a->T, E = a->E, k = a->k;
    if (T <= 0) return hipSuccess;
    if (E < 1 || E > 256 || k < 1 || k > 16 || k > E) return hipErrorInvalidValue;
    if (a->ep_lo < 0 || a->ep_n < 0 || a->ep_lo + a->ep_n > E) return hipErrorInvalidValue;
    int4 *items = reinterpret_cast<int4 *>(a->items);
    if (T == 1) {
        ORN_LAUNCH_EV(a, k_select_dispatch1, dim3(1), dim3(64), 0, s, a->logits, E, k, a->mode,
                           a->idx, a->w, a->ep_lo, a->ep_n, a->has_shared, a->ctl, a->slot_expert, a->slot_off,
                           a->slot_cnt, a->row_token, a->pair_row, items, a->items_max);
        return hipGetLastError();
    }
    if (T <= ORN_FUSED_SELECT_T) {
        ORN_LAUNCH_EV(a, k_select_dispatch, dim3(1), dim3(1024), 0, s, a->logits, T, E, k,
                           a->mode, a->idx, a->w, a->ep_lo, a->ep_n, a->has_shared, a->ctl, a->slot_expert,
                           a->slot_off, a->slot_cnt, a->row_token, a->pair_row, items,
                           a->items_max, a->tchunk);
        return hipGetLastError();
    }
    ORN_LAUNCH_EV2(a->ev_start, nullptr, k_select, dim3((T + 3) / 4), dim3(256), 0, s, a->logits,
                   T, E, k, a->mode, a->idx, a->w, a->ctl + 3);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    ORN_LAUNCH_EV2(nullptr, a->ev_stop, k_dispatch, dim3(1), dim3(1024), 0, s, a->idx, a->w, T, k,
                   E, a->ep_lo, a->ep_n, a->has_shared, a->ctl, a->slot_expert, a->slot_off,
                   a->slot_cnt, a->row_token, a->pair_row, items, a->items_max, a->tchunk);
    return hipGetLastError();
}
