// SPDX-License-Identifier: MIT
//
// Top-k selection of one token by one wave, with the reference's
// exchange-selection semantics, and the one-token dispatch; shared by the
// dispatch kernels (dispatch.hip) and the one-token gate/up kernel that
// selects in its prologue (expert_dec.hip).
//
// Selection (model.c:301-317 renormalised, model.c:1027-1049 literal) is
// exchange selection with strict '>'.  When the top k+1 logits are finite
// and pairwise distinct, exchange selection returns them in value order, so
// a wave finds them with k+1 rounds of "wave max, check it is unique,
// remove it" (DPP reductions, ballots); in the literal mode their gaps must
// also exceed 1e-5, so that their probabilities keep that order.  Otherwise
// (ties, NaN/Inf) one lane runs the reference's selection literally on this
// device's values.
#pragma once

#include <climits>
#include <math.h>

#include "common.h"

namespace orn_sel {

// ---------------------------------------------------------------------------
// Wave reductions through DPP (every lane receives the result).
// ---------------------------------------------------------------------------
template <int CTRL, bool BC = false>
__device__ __forceinline__ int dpp_i(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, BC);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}
__device__ __forceinline__ float readlane_f(float v, int l)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Wave max of the selection keys (every lane receives it): quad_perm
// [1,0,3,2], [2,3,0,1], then row_ror 4, 8 give every lane of a 16-lane row
// the row's value; the four rows are joined with readlane.
__device__ __forceinline__ int wave_max_key(int v)
{
    v = max(v, __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_mov_dpp(v, 0x124, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false));
    return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Order-preserving integer key of a finite float (a < b <=> key(a) <
// key(b)); -0 is folded into +0, so a -0/+0 pair compares equal, as the
// two do under '>'.
__device__ __forceinline__ int sel_key(float f)
{
    int b = __builtin_bit_cast(int, f);
    b = b == INT_MIN ? 0 : b;
    return b >= 0 ? b : b ^ 0x7FFFFFFF;
}

__device__ __forceinline__ float key_value(int k)
{
    return __builtin_bit_cast(float, k >= 0 ? k : k ^ 0x7FFFFFFF);
}

__device__ __forceinline__ float wave_sum(float v)
{
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x124>(v);
    v += dpp_f<0x128>(v);
    return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

// Inclusive prefix sum over the wave: row_shr 1, 2, 4, 8 within 16-lane rows
// (lanes before the row start read 0), then the earlier rows' totals.
__device__ __forceinline__ int wave_incl_scan(int v)
{
    const int lane = threadIdx.x & 63;
    v += dpp_i<0x111, true>(v);
    v += dpp_i<0x112, true>(v);
    v += dpp_i<0x114, true>(v);
    v += dpp_i<0x118, true>(v);
    const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31);
    const int r2 = __builtin_amdgcn_readlane(v, 47);
    const int row = lane >> 4;
    return v + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}

__device__ __forceinline__ void wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------------------
// Selection of one token by one wave (E <= 256: lane holds experts lane +
// 64*i).  Writes k indices and weights to io/wo and, if given, to the LDS
// copies lio/lwo.  val/ix: E floats/ints of LDS for the literal path.
// ---------------------------------------------------------------------------
__device__ inline void select_token(const float *__restrict__ lg, int E, int k, int mode,
                             uint32_t *__restrict__ io, float *__restrict__ wo, int *lio,
                             float *lwo, float *val, int *ix, int *n_slow)
{
    const int lane = threadIdx.x & 63;
    float vo[4];
    int key[4];  // selection keys; INT_MIN: no expert, or already selected
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = lane + 64 * i;
        const bool valid = e < E;
        vo[i] = valid ? lg[e] : -INFINITY;
        if (valid && !isfinite(vo[i])) bad = true;
        key[i] = valid ? sel_key(vo[i]) : INT_MIN;
    }
    bool slow = __ballot(bad) != 0ull;

    // Lane r < k ends up holding the r-th selected (value, index).  The
    // rounds compare integer keys of the finite logits (same order, one
    // integer max per reduction step).
    float my_v = 0.0f, mx = 0.0f, prev = 0.0f;
    int my_e = 0;
    if (!slow) {
        const int rounds = k < E ? k + 1 : k;
        for (int r = 0; r < rounds; ++r) {
            const int mk = wave_max_key(max(max(key[0], key[1]), max(key[2], key[3])));
            const float m = key_value(mk);
            uint64_t b[4];
            int cnt = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                b[i] = __ballot(key[i] == mk);
                cnt += __popcll(b[i]);
            }
            if (cnt != 1) {  // a tie (or a -0/+0 pair): take the literal path
                slow = true;
                break;
            }
            int e = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (b[i]) e = 64 * i + __ffsll((unsigned long long)b[i]) - 1;
            const bool hit = lane == (e & 63);  // the winner's lane; e >> 6 is uniform
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (hit && (e >> 6) == i) key[i] = INT_MIN;
            if (r == 0) {
                mx = m;
            } else {
                if (!(prev > m)) slow = true;
                if (mode == 1 && !((double)prev - (double)m > 1e-5)) slow = true;
            }
            if (lane == r) {
                my_v = m;
                my_e = e;
            }
            prev = m;
        }
    }

    if (!slow) {
        float w;
        if (mode == 0) {
            // model.c:307-317: s_i = expf(v_i - v_0), sequential sum, divide.
            const float s_i = expf(my_v - mx);
            float sum = 0.0f;
            for (int i = 0; i < k; ++i) sum += readlane_f(s_i, i);
            w = s_i / sum;
        } else {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) s += expf(vo[i] - mx);  // -inf (no expert) -> 0
            w = expf(my_v - mx) / wave_sum(s);
        }
        if (lane < k) {
            io[lane] = (uint32_t)my_e;
            wo[lane] = w;
            if (lio) {
                lio[lane] = my_e;
                lwo[lane] = w;
            }
        }
        return;
    }

    // Literal path: the reference's selection, run by lane 0 on this
    // device's values.
    if (lane == 0 && n_slow) atomicAdd(n_slow, 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = lane + 64 * i;
        if (e < E) {
            val[e] = vo[i];
            ix[e] = e;
        }
    }
    wave_sync();
    if (lane == 0) {
        if (mode == 1) {
            // model.c:1027-1036: max by strict '>', expf, sequential sum, divide.
            float m = val[0];
            for (int e = 1; e < E; ++e)
                if (val[e] > m) m = val[e];
            float sum = 0.0f;
            for (int e = 0; e < E; ++e) {
                val[e] = expf(val[e] - m);
                sum += val[e];
            }
            for (int e = 0; e < E; ++e) val[e] = val[e] / sum;
        }
        // k passes of exchange selection (model.c:301-305 / 1040-1048).
        for (int i = 0; i < k && i < E - 1; ++i)
            for (int j = i + 1; j < E; ++j)
                if (val[j] > val[i]) {
                    const float ft = val[i];
                    val[i] = val[j];
                    val[j] = ft;
                    const int it = ix[i];
                    ix[i] = ix[j];
                    ix[j] = it;
                }
        if (mode == 0) {
            const float m = val[0];
            float sum = 0.0f;
            for (int i = 0; i < k; ++i) sum += expf(val[i] - m);
            for (int i = 0; i < k; ++i) val[i] = expf(val[i] - m) / sum;
        }
        for (int i = 0; i < k; ++i) {
            io[i] = (uint32_t)ix[i];
            wo[i] = val[i];
            if (lio) {
                lio[i] = ix[i];
                lwo[i] = val[i];
            }
        }
    }
    wave_sync();
}


// The dispatch of one token by one wave from its selection (lidx, lw in
// LDS, k entries): what the general dispatch produces for T = 1.  Every
// active slot holds one row (row index = slot index): the shared expert
// first, then the selected experts with w >= 1e-6 (model.c:1066) of this
// share in ascending id; one item per slot.  With slot_e (LDS, k + 1
// entries) the slot experts are also written there, and the returned slot
// count is valid in every lane.
__device__ __forceinline__ int dispatch_one(const int *lidx, const float *lw, int E, int k,
                                            int ep_lo, int ep_n, int has_shared, int *ctl,
                                            int *slot_expert, int *slot_off, int *slot_cnt,
                                            int *row_token, int *pair_row, int4 *items,
                                            int items_max, int *slot_e)
{
    const int lane = threadIdx.x & 63;
    auto kept = [&](int j) {  // pair j survives the skip rule (model.c:1066) and is this share's
        return !(lw[j] < 1e-6f) && (uint32_t)(lidx[j] - ep_lo) < (uint32_t)ep_n;
    };
    const bool valid = lane < k && kept(lane);
    const int e = lane < k ? lidx[lane] : 0;
    int rank = 0;  // among the kept pairs, by expert id (the ids are distinct)
    for (int j = 0; j < k; ++j) rank += (kept(j) && lidx[j] < e) ? 1 : 0;
    const int hs = has_shared ? 1 : 0;
    const int n_slots = hs + __popcll(__ballot(valid));
    if (valid) {
        const int sl = hs + rank;
        if (slot_e) slot_e[sl] = e;
        if (slot_expert) {
            slot_expert[sl] = e;
            slot_off[sl] = sl;
            slot_cnt[sl] = 1;
            if (sl < items_max) items[sl] = make_int4(sl, sl, 1, e);
            row_token[sl] = 0;
        }
    }
    if (slot_expert && lane < k) pair_row[lane] = valid ? hs + rank : -1;
    if (lane == 0) {
        if (hs && slot_e) slot_e[0] = E;
        if (slot_expert) {
            if (hs) {
                slot_expert[0] = E;
                slot_off[0] = 0;
                slot_cnt[0] = 1;
                if (items_max > 0) items[0] = make_int4(0, 0, 1, E);
                row_token[0] = 0;
            }
            ctl[0] = n_slots;
            ctl[1] = n_slots < items_max ? n_slots : items_max;
            ctl[2] = n_slots;
        }
    }
    return n_slots;
}

}  // namespace orn_sel
