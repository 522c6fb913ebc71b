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
    // integer max per reduction step).  Each lane sorts its four (key, e)
    // descending once and offers its head; a round's maximum must be offered
    // by one lane only (equal heads: a tie), and the winner drops its head.
    // An expert equal to the winner in the winner's own lane comes up as
    // the next round's maximum, equal to the previous one, which the
    // strict-order check catches (after the k-th it no longer matters).
    float my_v = 0.0f, mx = 0.0f, prev = 0.0f;
    int my_e = 0;
    if (!slow) {
        int sk[4], se[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sk[i] = key[i];
            se[i] = lane + 64 * i;
        }
        auto cs = [&](int a, int b) {
            const bool sw = sk[b] > sk[a];
            const int ka = sk[a], kb = sk[b], ea = se[a], eb = se[b];
            sk[a] = sw ? kb : ka;
            sk[b] = sw ? ka : kb;
            se[a] = sw ? eb : ea;
            se[b] = sw ? ea : eb;
        };
        cs(0, 1);
        cs(2, 3);
        cs(0, 2);
        cs(1, 3);
        cs(1, 2);
        const int rounds = k < E ? k + 1 : k;
        for (int r = 0; r < rounds; ++r) {
            const int mk = wave_max_key(sk[0]);
            const uint64_t bl = __ballot(sk[0] == mk);
            if (__popcll(bl) != 1) {  // a tie (or a -0/+0 pair): take the literal path
                slow = true;
                break;
            }
            const int owner = __ffsll((unsigned long long)bl) - 1;
            const int e = __builtin_amdgcn_readlane(se[0], owner);
            const float m = key_value(mk);
            if (lane == owner) {
                sk[0] = sk[1];
                se[0] = se[1];
                sk[1] = sk[2];
                se[1] = se[2];
                sk[2] = sk[3];
                se[2] = se[3];
                sk[3] = INT_MIN;
            }
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
    const int e = lane < k ? lidx[lane] : 0;
    const float wl = lane < k ? lw[lane] : 0.0f;
    // pair `lane` survives the skip rule (model.c:1066) and is this share's
    const bool valid = lane < k && !(wl < 1e-6f) && (uint32_t)(e - ep_lo) < (uint32_t)ep_n;
    const uint64_t kb = __ballot(valid);
    int rank = 0;  // among the kept pairs, by expert id (the ids are distinct)
    for (int j = 0; j < k; ++j)
        rank += (((kb >> j) & 1ull) && __builtin_amdgcn_readlane(e, j) < e) ? 1 : 0;
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

// ---------------------------------------------------------------------------
// Dispatch helpers shared by the dispatch kernels (dispatch.hip) and the
// certified routing kernel (router_cert.hip).
// ---------------------------------------------------------------------------
struct DispatchLds {
    int cnt[1024];
    int cursor[1024];
    int rowoff[1024];
    int wtot[3][16];
};

// Expert of a selected pair if it is dispatched here, else 0xFFFFFFFF: the
// pair is skipped when w < 1e-6 (model.c:1066) or its expert lies outside
// this forward's share [ep_lo, ep_lo + ep_n) (another rank's).
template <typename IdxT>
__device__ __forceinline__ uint32_t dispatch_key(IdxT idx, float w, int ep_lo, int ep_n)
{
    const uint32_t e = (uint32_t)idx;
    return !(w < 1e-6f) && e - (uint32_t)ep_lo < (uint32_t)ep_n ? e : 0xFFFFFFFFu;
}

// The dispatch of a small batch (T * k <= 1024 pairs, E + 1 <= 320 slot
// candidates) by one wave: no work-group barrier, the same outputs as
// dispatch_group (slot j = 0 the shared expert, j = e + 1 routed expert e;
// slots, row ranges and items in j order; rows of an expert in any order).
// Lane l takes the candidates j = 5l .. 5l+4, so the scans over j are a
// lane-local sum and one wave scan.
template <typename IdxT>
__device__ void dispatch_wave(DispatchLds &L, const IdxT *lidx, const float *lw, int T, int k,
                              int E, int ep_lo, int ep_n, int has_shared, int *ctl,
                              int *slot_expert, int *slot_off, int *slot_cnt, int *row_token,
                              int *pair_row, int4 *items, int items_max, int tchunk)
{
    constexpr int JPL = 5;
    const int lane = threadIdx.x & 63;
    const int NJ = E + 1, P = T * k, j0 = JPL * lane;
#pragma unroll
    for (int i = 0; i < JPL; ++i) {
        L.cnt[j0 + i] = 0;
        L.cursor[j0 + i] = 0;
    }
    wave_sync();
    for (int p = lane; p < P; p += 64) {
        const uint32_t key = dispatch_key(lidx[p], lw[p], ep_lo, ep_n);
        if (key != 0xFFFFFFFFu) atomicAdd(&L.cnt[key + 1], 1);
    }
    wave_sync();
    int c[JPL], nit[JPL], sc = 0, sn = 0, sf = 0;
#pragma unroll
    for (int i = 0; i < JPL; ++i) {
        const int j = j0 + i;
        c[i] = j >= NJ ? 0 : j == 0 ? (has_shared ? T : 0) : L.cnt[j];
        nit[i] = (c[i] + tchunk - 1) / tchunk;
        sc += c[i];
        sn += nit[i];
        sf += c[i] > 0 ? 1 : 0;
    }
    const int ic = wave_incl_scan(sc), in = wave_incl_scan(sn), iflag = wave_incl_scan(sf);
    int roff = ic - sc, ioff = in - sn, slot = iflag - sf;
#pragma unroll
    for (int i = 0; i < JPL; ++i) {
        const int j = j0 + i;
        L.rowoff[j] = roff;
        if (c[i] > 0) {
            const int ex = j == 0 ? E : j - 1;
            slot_expert[slot] = ex;
            slot_off[slot] = roff;
            slot_cnt[slot] = c[i];
            for (int q = 0; q < nit[i] && ioff + q < items_max; ++q) {
                const int r0 = q * tchunk;
                items[ioff + q] = make_int4(slot, roff + r0, min(tchunk, c[i] - r0), ex);
            }
            ++slot;
        }
        roff += c[i];
        ioff += nit[i];
    }
    if (lane == 63) {
        ctl[0] = iflag;
        ctl[1] = in < items_max ? in : items_max;
        ctl[2] = ic;
    }
    wave_sync();
    for (int p = lane; p < P; p += 64) {
        const uint32_t key = dispatch_key(lidx[p], lw[p], ep_lo, ep_n);
        if (key == 0xFFFFFFFFu) {  // skipped, or another rank's expert
            pair_row[p] = -1;
            continue;
        }
        const int j = (int)key + 1;
        const int r = L.rowoff[j] + atomicAdd(&L.cursor[j], 1);
        row_token[r] = p / k;
        pair_row[p] = r;
    }
    if (has_shared)
        for (int t = lane; t < T; t += 64) row_token[L.rowoff[0] + t] = t;
}

}  // namespace orn_sel
