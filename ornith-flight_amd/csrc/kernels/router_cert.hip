// SPDX-License-Identifier: MIT
//
// Certified routing of the smallest decode batches (T <= 4 tokens): router
// logits, top-k selection and the token -> expert dispatch in ONE launch,
// with the reference's routing decisions reproduced exactly.
//
// The reference's logit (model.c:1017-1025) is a sequential fp32 chain
//   s^_1 = p_1,  s^_i = fl(s^_{i-1} + p_i),  p_i = fl(x_i * W(i, e)),
// n = D dependent adds (plus one for a router bias): 4.3 us of dependent
// adds at D = 2048 however many lanes run.  Here the same fp32 products p_i
// are summed in parallel, in fp64, giving S (relative error ~1e-14),
// together with a rigorous bound on the chain's distance from it:
//   |s^_n - s_n| <= u * sum_{i>=2} |s_i| / (1 - n u),   u = 2^-24,
// s_i the exact partial sums.  (Each step rounds by at most u of |s^_i|,
// and |s^_i| <= |s_i| + that same error, hence the 1 / (1 - n u).)  The
// partial sums are formed per lane over a chunk of L = D/64 consecutive
// values (running sum l_i in fp64) and bounded chunk by chunk as
//   sum_{i in chunk} |O + l_i| <= L |O| + sum_i |l_i|,
// O the sum of the chunks before, so that all chunks run in parallel.  The
// bound gets a 1e-3 margin for its own fp32/fp64 roundings (which also
// covers the error of S itself), plus 1e-30 for underflow.
//
// Selection (one wave per token).  With the intervals [S - B, S + B]:
//   certified  if the top k by S are ordered with gaps (lo_r > hi_{r+1}) and
//              the k-th lies above every other expert's hi -- then the
//              exchange selection of model.c:301-317 / 1040-1048 returns
//              exactly these k in this order (in the literal mode every gap
//              must exceed 1e-5 as well, so that the probabilities keep the
//              order: the condition dispatch.hip's fast path uses);
//   otherwise  the candidates (every expert whose hi reaches the k-th
//              largest lo; everything below is beaten by k experts) get the
//              reference's exact fp32 chain and the test runs again: the
//              candidates are now exact points, so it fails only on exact
//              ties or a literal-mode gap under 1e-5;
//   then       every logit of the token gets its exact chain and the
//              reference's selection runs on them (select.h select_token,
//              which handles ties, NaN and Inf literally).
// Non-finite sums skip straight to the last case.  The weights are formed
// from the fp32-rounded sums with select.h's formulas (exact logits where a
// chain ran); the logits buffer receives the same values.
//
// One launch: E/4 work groups of 4 waves; work group eg forms the sums of
// experts 4eg..4eg+3 for every token; the last work group to finish (a
// counter) selects (wave t: token t) and dispatches (select.h dispatch_one /
// dispatch_wave).
//
// With the layer's rmsnorm (ORN_MOE_NORM, gpu.c:144-156) the reference's
// products are p_i = fl(fl(w_i * fl(x_i * inv)) * W(i, e)), inv from a
// sequential fp32 sum of squares (another 2048 dependent adds).  That chain
// runs in one extra work group, in parallel with the sums, which take the
// scale out: the groups sum q_i = fl(fl(x_i * w_i) * W(i, e)) into T and
// bound |chain - inv T| <= inv B_T with
//   B_T = u (A_q + 5.0001 n u Q) / (1 - n u) + 5.0001 u Q,
// A_q = sum |partial sums of q|, Q = sum |q_i| (p_i and inv q_i differ by
// at most 5 roundings of |p_i|, which moves every partial sum by at most
// 5.0001 u inv Q).  The extra group publishes inv (a tagged word), the
// normalised rows and their max |x|; the selecting group waits for inv and
// forms S = inv T (+ bias) and B = inv B_T (+ the bias add's rounding) --
// exact products of fp32 values in fp64 -- before the selection, and
// rebuilds the normalised rows for the exact chains.  Measured at T = 16 the serial
// per-wave phases (selection ~3 us, dispatch ~2-3 us) and the handoffs
// between token groups cost more than the exact chains save, so larger
// batches keep the exact routers (router.hip, dispatch.hip).
// The counter and a generation word live in a 4 KB area that starts zeroed.
#include "common.h"
#include "launch.h"
#include "mfma_ops.h"
#include "select.h"

#include <climits>
#include <math.h>

namespace {

using namespace orn_sel;

constexpr int CERT_TPG = ORN_CERT_MAX_T;  // the batch (wave w selects token w)
constexpr int CERT_EPG = 4;  // experts per work group in the sum phase
constexpr int CERT_NCH = 64; // chunks per logit (one per lane group)

// sync area: int 0: work groups done; 64-bit word 1: the generation.
enum { SYNC_GROUP = 0 };
enum { SYNC64_GEN = 1 };

struct CertArgs {
    const float *x, *router, *bias, *norm_w;
    float *xn, *x_amax, *logits;
    uint64_t *est;   // [T][E] tagged (S, B) words, then [T] tagged rmsnorm scales
    int *sync;
    uint32_t *idx;
    float *w;
    int *ctl, *slot_expert, *slot_off, *slot_cnt, *row_token, *pair_row;
    int4 *items;
    int T, E, k, mode, ep_lo, ep_n, has_shared, items_max, tchunk;
    int ngroups;  // expert work groups (with the rmsnorm, one more group runs its chain)
};

__device__ __forceinline__ double readlane_d(double v, int l)
{
    const long long bits = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)(bits & 0xFFFFFFFFll), l);
    const int hi = __builtin_amdgcn_readlane((int)(bits >> 32), l);
    return __longlong_as_double(((long long)hi << 32) | (long long)(unsigned int)lo);
}

// row_shr:n within 16-lane rows, lanes before the row start reading 0 (a
// double of zero bits is +0.0)
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v)
{
    const long long bits = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(bits & 0xFFFFFFFFll), CTRL, 0xF, 0xF, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(bits >> 32), CTRL, 0xF, 0xF, true);
    return __longlong_as_double(((long long)hi << 32) | (long long)(unsigned int)lo);
}

// Inclusive prefix sum over each 16-lane row.
__device__ __forceinline__ double row_incl_scan_d(double v)
{
    v += dpp_d<0x111>(v);
    v += dpp_d<0x112>(v);
    v += dpp_d<0x114>(v);
    v += dpp_d<0x118>(v);
    return v;
}

// fp32 bounds of a double, without branches: f_down(v) <= v <= f_up(v).
// The fp32 rounding moves v by at most half an ulp (<= |v| 2^-24), so a
// shift of |v| 2^-22 (plus 1e-38 for the subnormal range) before it cannot
// be undone; the bounds are ~4 ulp looser than the tightest.
__device__ __forceinline__ float f_down(double v)
{
    return (float)(v - fabs(v) * 0x1p-22 - 1e-38);
}
__device__ __forceinline__ float f_up(double v)
{
    return (float)(v + fabs(v) * 0x1p-22 + 1e-38);
}

__device__ __forceinline__ int max4(const int (&k)[4])
{
    return max(max(k[0], k[1]), max(k[2], k[3]));
}

// The reference's logit of expert e for the token row xs (LDS, nq quads):
// acc = 0; acc = acc + x[d] * W(d, e), d ascending; then + bias[e]
// (model.c:1017-1025).  W quads stream through a ring of NB batches of 4
// (NB - 1 batches in flight while a batch's 16 adds run; a deeper ring costs
// the whole kernel registers, and this path runs only for the few tokens
// whose bounds do not decide the selection).
__device__ __forceinline__ float exact_chain(const v4f *xs4, const v4f *Wq4, int e, int E, int nq,
                             const float *bias)
{
    constexpr int QB = 4, NB = 4;
    const int nb = nq / QB;  // nq is a multiple of 64
    v4f ring[NB][QB];
    auto ld = [&](v4f(&r)[QB], int b) {
#pragma unroll
        for (int i = 0; i < QB; ++i) r[i] = Wq4[(size_t)(QB * b + i) * E + e];
    };
#pragma unroll
    for (int s = 0; s < NB - 1; ++s) ld(ring[s], min(s, nb - 1));
    float acc = 0.0f;
#pragma unroll 1
    for (int b0 = 0; b0 < nb; b0 += NB) {
#pragma unroll
        for (int s = 0; s < NB; ++s) {
            const int b = b0 + s;
            ld(ring[(s + NB - 1) % NB], min(b + NB - 1, nb - 1));
            if (b < nb) {
#pragma unroll
                for (int i = 0; i < QB; ++i) {
                    const v4f xv = xs4[QB * b + i];
                    const v4f w = ring[s][i];
                    acc = acc + xv.x * w.x;
                    acc = acc + xv.y * w.y;
                    acc = acc + xv.z * w.z;
                    acc = acc + xv.w * w.w;
                }
            }
        }
    }
    if (bias) acc = acc + bias[e];
    return acc;
}

// Per-wave LDS of the selection.
struct SelLds {
    int cand[256];    // experts whose exact chain runs
    float cval[256];  // their chains' results
    float val[256];   // select_token's literal path
    int ix[256];
    int lidx[16];
    float lw[16];
};

// ---------------------------------------------------------------------------
// Handoffs between work groups.  An agent-scope release fence costs an L2
// writeback on this part (measured: 3.5 us at 64 work groups, 17 us at
// 256), so nothing here is fenced: every value one work group passes to
// another travels in ONE 64-bit agent-scope atomic word together with the
// launch's tag (the low 7 bits of a generation counter that the last work
// group of each launch advances, plus bit 7), and the reader re-reads a
// word until its tag is this launch's.
// The counters that elect the last work groups are relaxed agent-scope
// read-modify-writes issued after the writer's stores have completed
// (s_waitcnt), so the reader's first read almost always finds the tag.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void st_word(uint64_t *p, uint64_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t ld_word(const uint64_t *p)
{
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}

// Read a tagged word: until its low byte is `tag` (bounded by 20 ms of the
// 100 MHz real-time counter; false if the bound ran out, which the callers
// treat as "no value").
__device__ __forceinline__ bool ld_tagged(const uint64_t *p, uint32_t tag, uint64_t &v)
{
    v = ld_word(p);
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    while ((uint32_t)(v & 0xFFu) != tag && __builtin_amdgcn_s_memrealtime() - t0 < 2000000ull) {
        __builtin_amdgcn_s_sleep(1);
        v = ld_word(p);
    }
    return (uint32_t)(v & 0xFFu) == tag;
}

// An expert's (S, B) as one word: S rounded to fp32 (the rounding added to
// B) in the high half; B rounded up to fp32, then up to a multiple of 256
// ulp, its low 8 bits then holding the tag (B only grows), in the low half.
__device__ __forceinline__ uint64_t pack_est(double S, double B, uint32_t tag)
{
    const float sf = (float)S;
    uint32_t bb;
    if (!(B < 1e30) || !(fabs(S) < 3e38)) {
        bb = 0x7F000000u;  // ~1.7e38: never certifies
    } else {
        const float bf = f_up(B + fabs(S - (double)sf));
        bb = (__float_as_uint(bf) + 0xFFu) & ~0xFFu;
    }
    return ((uint64_t)__float_as_uint(sf) << 32) | (uint64_t)(bb | tag);
}

__device__ __forceinline__ void unpack_est(uint64_t w, float &sf, float &bf)
{
    sf = __uint_as_float((uint32_t)(w >> 32));
    bf = __uint_as_float((uint32_t)w);  // the tag bits only enlarge B
}

// Exchange of four (key, lo, hi, s, e) slots, descending key.
struct Slot {
    int key;
    float lo, hi, sf;
    int e;
};
__device__ __forceinline__ void cswap(Slot &a, Slot &b)
{
    const bool sw = b.key > a.key;
    const Slot ta = a, tb = b;
    a.key = sw ? tb.key : ta.key;
    a.lo = sw ? tb.lo : ta.lo;
    a.hi = sw ? tb.hi : ta.hi;
    a.sf = sw ? tb.sf : ta.sf;
    a.e = sw ? tb.e : ta.e;
    b.key = sw ? ta.key : tb.key;
    b.lo = sw ? ta.lo : tb.lo;
    b.hi = sw ? ta.hi : tb.hi;
    b.sf = sw ? ta.sf : tb.sf;
    b.e = sw ? ta.e : tb.e;
}

// Selection of one token by one wave from its experts' (sf, bf) (lane l
// holds experts l + 64 i); see the file comment.  Writes the k indices and
// weights to io/wo and S.lidx/S.lw; logits_row gets the fp32 values the
// weights come from.  Returns 0 (certified), 1 (candidates chained) or 2
// (every logit chained).
template <class PrepRow, class Rescale>
__device__ __forceinline__ int select_cert(float (&sfv)[4], float (&bfv)[4], bool bad,
                                           const float *xrow, PrepRow prep_row, Rescale rescale,
                                           const v4f *Wq4, const float *bias,
                                           int D, int E, int k, int mode, uint32_t *io, float *wo,
                                           float *logits_row, SelLds &S, int *n_lit)
{
    const int lane = threadIdx.x & 63;
    bool valid[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) valid[i] = lane + 64 * i < E;
    const double m = mode == 1 ? 1e-5 : 0.0;
    int my_e = 0;
    float my_v = 0.0f;

    // k rounds of "largest fp32 sum not yet taken" over each lane's four
    // slots sorted by key (the lane offers its head; the owner of the
    // round's maximum drops it), checking on the way, in fp32 bounds
    // rounded outward, that each selected lo exceeds the next one's hi + m,
    // and finally that the k-th lo exceeds every remaining hi + m.  A tie
    // of the fp32 keys fails (the doubles behind them lie within an ulp,
    // far inside the bounds).
    auto certify = [&]() -> bool {
        Slot sl[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sl[i].key = valid[i] ? sel_key(sfv[i]) : INT_MIN;
            sl[i].lo = f_down((double)sfv[i] - (double)bfv[i]);
            sl[i].hi = valid[i] ? f_up((double)sfv[i] + (double)bfv[i] + m) : -INFINITY;
            sl[i].sf = sfv[i];
            sl[i].e = lane + 64 * i;
        }
        cswap(sl[0], sl[1]);
        cswap(sl[2], sl[3]);
        cswap(sl[0], sl[2]);
        cswap(sl[1], sl[3]);
        cswap(sl[1], sl[2]);
        float prev_lo = 0.0f;
        for (int r = 0; r < k; ++r) {
            const int mk = wave_max_key(sl[0].key);
            const uint64_t bl = __ballot(sl[0].key == mk);
            if (__popcll(bl) != 1) return false;
            const int owner = __ffsll((unsigned long long)bl) - 1;
            const float w_lo = readlane_f(sl[0].lo, owner);
            const float w_hi = readlane_f(sl[0].hi, owner);
            const float w_sf = readlane_f(sl[0].sf, owner);
            const int w_e = __builtin_amdgcn_readlane(sl[0].e, owner);
            if (r > 0 && !(prev_lo > w_hi)) return false;
            prev_lo = w_lo;
            if (lane == r) {
                my_e = w_e;
                my_v = w_sf;
            }
            if (lane == owner) {
                sl[0] = sl[1];
                sl[1] = sl[2];
                sl[2] = sl[3];
                sl[3].key = INT_MIN;
                sl[3].hi = -INFINITY;
            }
        }
        const float hr = fmaxf(fmaxf(sl[0].hi, sl[1].hi), fmaxf(sl[2].hi, sl[3].hi));
        const int mh = wave_max_key(hr == -INFINITY ? INT_MIN : sel_key(hr));
        return mh == INT_MIN || prev_lo > key_value(mh);
    };
    // the k-th largest lower bound (k rounds over fp32 keys)
    auto kth_lo = [&]() -> float {
        int key[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            key[i] = valid[i] ? sel_key(f_down((double)sfv[i] - (double)bfv[i])) : INT_MIN;
        int mk = INT_MIN;
        for (int r = 0; r < k; ++r) {
            mk = wave_max_key(max4(key));
            int win = -1;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint64_t bl = __ballot(key[i] == mk);
                if (win < 0 && bl) win = 64 * i + __ffsll((unsigned long long)bl) - 1;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if ((win >> 6) == i && lane == (win & 63)) key[i] = INT_MIN;
        }
        return key_value(mk);
    };

    // One call site each for the certificate and the chains (the loop runs
    // at most twice: every inlined copy costs registers).
    int path = 0;
    bool row_ready = false, scaled = false;
    for (;;) {
        const bool ok = !bad && certify();
        if (!scaled) {
            // values given up to a positive scale (the caller's T-space):
            // the certificate holds for any scale; the weights and chains
            // need the values themselves
            bool nf = false;
            const float sc = rescale(nf);
            if (sc != 0.0f) my_v = (float)((double)sc * (double)my_v);
            if (nf) bad = true;
            scaled = true;
            if (ok && !bad) break;
        } else if (ok) {
            break;
        }
        int n = 0;
        bool isc[4] = {false, false, false, false};
        int pos[4] = {0, 0, 0, 0};
        if (path == 0 && !bad) {
            // candidates: hi + m reaches the k-th largest lo
            const float th = kth_lo();
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                isc[i] = valid[i] && f_up((double)sfv[i] + (double)bfv[i] + m) >= th;
                const uint64_t bl = __ballot(isc[i]);
                pos[i] = n + __popcll(bl & ((1ull << lane) - 1ull));
                n += __popcll(bl);
            }
            path = n <= 64 ? 1 : 2;
        } else {
            path = 2;
        }
        if (path == 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (isc[i]) S.cand[pos[i]] = lane + 64 * i;
        } else {
            n = E;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (valid[i]) S.cand[lane + 64 * i] = lane + 64 * i;
        }
        if (!row_ready) {
            prep_row();  // the row the chains read (the rmsnorm's: rebuilt here)
            row_ready = true;
        }
        wave_sync();
        for (int c = lane; c < n; c += 64)
            S.cval[c] = exact_chain(reinterpret_cast<const v4f *>(xrow), Wq4, S.cand[c], E, D / 4,
                                    bias);
        wave_sync();
        if (path == 2) break;
        bool fin = true;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (isc[i]) {
                sfv[i] = S.cval[pos[i]];
                bfv[i] = 0.0f;
                if (!isfinite(sfv[i])) fin = false;
            }
        bad = __ballot(!fin) != 0ull;
    }
    if (path == 2) {
        // S.cval[e] = the reference's logit e: its selection, literally
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (valid[i]) logits_row[lane + 64 * i] = S.cval[lane + 64 * i];
        select_token(S.cval, E, k, mode, io, wo, S.lidx, S.lw, S.val, S.ix, n_lit);
        return 2;
    }

    // weights from the fp32 values (select.h select_token's formulas)
    float vo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        vo[i] = valid[i] ? sfv[i] : -INFINITY;
        if (valid[i]) logits_row[lane + 64 * i] = vo[i];
    }
    const float mx = readlane_f(my_v, 0);
    float w;
    if (mode == 0) {
        const float s_i = expf(my_v - mx);
        float sum = 0.0f;
        for (int i = 0; i < k; ++i) sum += readlane_f(s_i, i);
        w = s_i / sum;
    } else {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) t += expf(vo[i] - mx);
        w = expf(my_v - mx) / wave_sum(t);
    }
    if (lane < k) {
        io[lane] = (uint32_t)my_e;
        wo[lane] = w;
        S.lidx[lane] = my_e;
        S.lw[lane] = w;
    }
    wave_sync();
    return path;
}

template <int NQ>
__global__ void __launch_bounds__(256) k_route_cert(CertArgs P)
{
    constexpr int D = 256 * NQ, L = 4 * NQ;  // L: values per chunk (lane)
    __shared__ __align__(16) float xs[CERT_TPG][D];
    // the chunk sums are dead once the per-expert sums are formed; the
    // selection and dispatch LDS reuse them
    union Lds2 {
        struct {
            double t[CERT_TPG][CERT_NCH][CERT_EPG];
            float a[CERT_TPG][CERT_NCH][CERT_EPG];
            float q[CERT_TPG][CERT_NCH][CERT_EPG];
        } parts;
        struct {
            SelLds sel[CERT_TPG];
            DispatchLds dl;
            int pidx[CERT_TPG * 16];
            float pw[CERT_TPG * 16];
        } sd;
        v4f sq[CERT_TPG * D / 4];  // the rmsnorm's squares
    };
    __shared__ Lds2 U;
    auto &part_t = U.parts.t;
    auto &part_a = U.parts.a;
    auto &part_q = U.parts.q;
    auto &sel = U.sd.sel;
    __shared__ float mx_s[CERT_TPG][4];
    __shared__ int flag_s, lit_s, chain_s;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int eg = blockIdx.x;
    const int E = P.E, T = P.T, k = P.k;
    const int t0 = 0, nt = T;  // T <= CERT_TPG: one token group
    const v4f *Wq4 = reinterpret_cast<const v4f *>(P.router);
    uint64_t *const sync64 = reinterpret_cast<uint64_t *>(P.sync);
    // this launch's tag (the generation the previous launch left)
    // (bit 7 set: a zeroed word never carries a tag)
    const uint32_t tag = ((uint32_t)ld_word(&sync64[SYNC64_GEN]) & 0x7Fu) | 0x80u;
    uint64_t *const inv_word = P.est + (size_t)T * E;  // [T] tagged rmsnorm scales
    const bool norm = P.norm_w != nullptr;

    if (norm && eg == P.ngroups) {
        // ---- the rmsnorm's group (gpu.c:144-156): the sequential sum of
        // squares by lane 0 of wave t (the squares first, by every thread,
        // so that the chain is adds only), then xn = w * (x * inv) and max
        // |xn| for the expert steps, and inv for the selecting group ----
        __shared__ float inv_s[CERT_TPG];
        v4f *sq = U.sq;
        for (int i = tid; i < nt * (D / 4); i += 256) {
            const int t = i / (D / 4), c = i % (D / 4);
            const v4f v = reinterpret_cast<const v4f *>(P.x + (size_t)(t0 + t) * D)[c];
            reinterpret_cast<v4f *>(xs[t])[c] = v;
            sq[i] = v * v;
        }
        __syncthreads();
        if (wave < nt && lane == 0) {
            const float ss = orn_lds_seq_sum32_n<D / 32>(sq + wave * (D / 4));
            inv_s[wave] = 1.0f / sqrtf(ss / (float)D + 1e-6f);
        }
        __syncthreads();
        if (tid < nt)
            st_word(&inv_word[t0 + tid],
                    ((uint64_t)__float_as_uint(inv_s[tid]) << 32) | (uint64_t)tag);
        for (int t = 0; t < nt; ++t) {
            float mx = 0.0f;
            for (int c = tid; c < D / 4; c += 256) {
                const v4f wn = reinterpret_cast<const v4f *>(P.norm_w)[c];
                const v4f v = wn * (reinterpret_cast<const v4f *>(xs[t])[c] * inv_s[t]);
                reinterpret_cast<v4f *>(P.xn + (size_t)(t0 + t) * D)[c] = v;
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            }
            if (P.x_amax) {
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
                if (lane == 0) mx_s[t][wave] = mx;
            }
        }
        __syncthreads();
        if (P.x_amax && tid < nt)
            P.x_amax[t0 + tid] =
                fmaxf(fmaxf(mx_s[tid][0], mx_s[tid][1]), fmaxf(mx_s[tid][2], mx_s[tid][3]));
        return;
    }

    // ---- sums: lane (j, el) covers chunk j (values L*j ..) of expert el ----
    const int el = lane & 3, j = 16 * wave + (lane >> 2);
    const int e = CERT_EPG * eg + el;
    const int ec = min(e, E - 1);  // lanes past E compute a copy, never stored
    v4f wr[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) wr[q] = Wq4[(size_t)(NQ * j + q) * E + ec];
    // the rows (with the rmsnorm: x * w, whose products with W differ from
    // the reference's by the scale inv and 5 roundings)
    for (int i = tid; i < nt * (D / 4); i += 256) {
        const int t = i / (D / 4), c = i % (D / 4);
        v4f v = reinterpret_cast<const v4f *>(P.x + (size_t)(t0 + t) * D)[c];
        if (norm) v = v * reinterpret_cast<const v4f *>(P.norm_w)[c];
        reinterpret_cast<v4f *>(xs[t])[c] = v;
    }
    __syncthreads();
    if (P.x_amax && eg == 0 && !norm) {
        // max |x| per token for the MFMA activation scaling
        for (int t = 0; t < nt; ++t) {
            float mx = 0.0f;
            for (int c = tid; c < D; c += 256) mx = fmaxf(mx, fabsf(xs[t][c]));
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
            if (lane == 0) mx_s[t][wave] = mx;
        }
        __syncthreads();
        if (tid < nt)
            P.x_amax[t0 + tid] =
                fmaxf(fmaxf(mx_s[tid][0], mx_s[tid][1]), fmaxf(mx_s[tid][2], mx_s[tid][3]));
    }

    for (int t = 0; t < nt; ++t) {
        const v4f *xr = reinterpret_cast<const v4f *>(xs[t]) + NQ * j;
        double l = 0.0;
        float A = 0.0f, Q = 0.0f;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const v4f p = xr[q] * wr[q];  // the reference's fp32 products (rmsnorm: q_i)
            l += (double)p.x;
            A += fabsf((float)l);
            l += (double)p.y;
            A += fabsf((float)l);
            l += (double)p.z;
            A += fabsf((float)l);
            l += (double)p.w;
            A += fabsf((float)l);
            if (norm) Q += (fabsf(p.x) + fabsf(p.y)) + (fabsf(p.z) + fabsf(p.w));
        }
        part_t[t][j][el] = l;
        part_a[t][j][el] = A;
        if (norm) part_q[t][j][el] = Q;
    }
    __syncthreads();

    // ---- per (token, expert): S and the bound; wave t <-> token t, lanes
    // (ce, r) with r covering chunks 4r .. 4r+3 of expert ce ----
    if (wave < nt) {
        const int t = wave, ce = lane >> 4, r = lane & 15;
        double tc[4], tl = 0.0, ql = 0.0;
        float ac[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            tc[i] = part_t[t][4 * r + i][ce];
            ac[i] = part_a[t][4 * r + i][ce];
            tl += tc[i];
            if (norm) ql += (double)part_q[t][4 * r + i][ce];
        }
        // DPP row scans (a row = one expert): O = the sum before lane r's
        // chunks; row totals land in lane 15
        const double inc = row_incl_scan_d(tl);
        double O = dpp_d<0x111>(inc);
        double sabs = 0.0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sabs += (double)L * fabs(O) + (double)ac[i];
            O += tc[i];
        }
        sabs = row_incl_scan_d(sabs);
        if (norm) ql = row_incl_scan_d(ql);
        double Sv = inc;
        const int eo = CERT_EPG * eg + ce;
        if (r == 15 && eo < E) {
            double n = (double)D;
            const double u = 0x1p-24;
            double Bv;
            if (norm) {
                // T and B_T (the bias and inv join in the selecting group)
                const double qa = ql * (1.0 + 1e-3);
                Bv = u * (sabs + 5.0001 * n * u * qa) * (1.0 + 1e-3) / (1.0 - n * u) +
                     5.0001 * u * qa + 1e-30;
            } else {
                if (P.bias) {
                    Sv += (double)P.bias[eo];
                    sabs += fabs(Sv);
                    n += 1.0;
                }
                Bv = u * sabs * (1.0 + 1e-3) / (1.0 - n * u) + 1e-30;
                P.logits[(size_t)(t0 + t) * E + eo] = (float)Sv;
            }
            // a partial sum beyond 1e38 could overflow the fp32 chain
            if (!(sabs < 1e38)) Bv = INFINITY;
            st_word(&P.est[(size_t)(t0 + t) * E + eo], pack_est(Sv, Bv, tag));
        }
    }

    // ---- the last work group of the token group selects its tokens ----
    __builtin_amdgcn_s_waitcnt(0);  // this wave's words have completed
    __syncthreads();
    if (tid == 0) {
        const int old = __hip_atomic_fetch_add(&P.sync[SYNC_GROUP], 1, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
        flag_s = old == P.ngroups - 1;
        if (flag_s)
            __hip_atomic_store(&P.sync[SYNC_GROUP], 0, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        lit_s = 0;
        chain_s = 0;
    }
    __syncthreads();
    if (!flag_s) return;
    if (wave < nt) {
        const int t = t0 + wave;
        float sfv[4], bfv[4];
        bool bad = false;
        // all four words in flight at once; a stale one is re-read alone
        uint64_t wv[4];
        const uint64_t *er = P.est + (size_t)t * E;
#pragma unroll
        for (int i = 0; i < 4; ++i) wv[i] = ld_word(&er[min(lane + 64 * i, E - 1)]);
        // with the rmsnorm: the token's scale, which its group publishes once
        // its chain (run beside the sums) ends; read while the words above
        // are in flight
        // with the rmsnorm: the token's scale, which its group publishes once
        // its chain (run beside the sums) ends.  Without a bias and in the
        // renormalising mode the selection is scale-invariant, so the first
        // certificate runs on (T, B_T) before the scale is read (select_cert
        // calls rescale() after it); otherwise the scale comes first.
        const bool tspace = norm && !P.bias && P.mode == 0;
        float inv = 1.0f;
        auto get_inv = [&]() {
            uint64_t iw = ld_word(&inv_word[t]);
            if ((uint32_t)(iw & 0xFFu) != tag && !ld_tagged(&inv_word[t], tag, iw)) {
                // not published within the bound: the chain here (lane 0)
                float ss = 0.0f;
                if (lane == 0) {
                    const float *xr = P.x + (size_t)t * D;
                    for (int c = 0; c < D; ++c) ss = ss + xr[c] * xr[c];
                }
                ss = __shfl(ss, 0, 64);
                inv = 1.0f / sqrtf(ss / (float)D + 1e-6f);
            } else {
                inv = __uint_as_float((uint32_t)(iw >> 32));
            }
        };
        // S = inv T + bias and B = inv B_T + the bias add's rounding
        auto apply_scale = [&]() {
            const double u = 0x1p-24;
            bool nf = false;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ee = lane + 64 * i;
                if (ee >= E) continue;
                double Sc = (double)inv * (double)sfv[i];  // exact
                double Bc = (double)inv * (double)bfv[i];
                if (P.bias) {
                    Sc += (double)P.bias[ee];
                    Bc += u * (fabs(Sc) + Bc) * (1.0 + 1e-6) + 1e-30;
                }
                const float sf = (float)Sc;
                sfv[i] = sf;
                bfv[i] = (fabs(Sc) < 3e38 && Bc < 1e30) ? f_up(Bc + fabs(Sc - (double)sf))
                                                         : 1.7e38f;
                P.logits[(size_t)t * E + ee] = sf;
                if (!(fabsf(sf) < 3e38f)) nf = true;
            }
            return __ballot(nf) != 0ull;
        };
        if (norm && !tspace) get_inv();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ee = lane + 64 * i;
            sfv[i] = 0.0f;
            bfv[i] = 0.0f;
            if (ee < E) {
                if ((uint32_t)(wv[i] & 0xFFu) != tag && !ld_tagged(&er[ee], tag, wv[i])) bad = true;
                unpack_est(wv[i], sfv[i], bfv[i]);
                if (!(fabsf(sfv[i]) < 3e38f)) bad = true;
            }
        }
        if (norm && !tspace && apply_scale()) bad = true;
        // after select_cert's first certificate (T-space only): the scale,
        // then the values in logit units; returns the scale (0: nothing done)
        auto rescale = [&](bool &nf) -> float {
            if (!tspace) return 0.0f;
            get_inv();
            nf = apply_scale();
            return inv;
        };
        bad = __ballot(bad) != 0ull;
        uint32_t *io = P.idx + (size_t)t * k;
        float *wo = P.w + (size_t)t * k;
        // the exact chains read the reference's normalised row: rebuilt from
        // x, w and the published scale only if a chain runs
        auto prep_row = [&]() {
            if (!norm) return;
            const v4f *x4 = reinterpret_cast<const v4f *>(P.x + (size_t)t * D);
            const v4f *w4 = reinterpret_cast<const v4f *>(P.norm_w);
            v4f *r4 = reinterpret_cast<v4f *>(xs[wave]);
#pragma unroll
            for (int c = lane; c < D / 4; c += 64) r4[c] = w4[c] * (x4[c] * inv);
        };
        const int path = select_cert(sfv, bfv, bad, xs[wave], prep_row, rescale, Wq4, P.bias, D,
                                     E, k, P.mode, io, wo, P.logits + (size_t)t * E, sel[wave],
                                     &lit_s);
        if (lane == 0 && path) atomicAdd(&chain_s, 1);
    }
    __syncthreads();

    // ---- ... and dispatches the batch ----
    if (T > 1) {
        // the batch's selections, from the waves' LDS copies
        for (int p = tid; p < T * k; p += 256) {
            U.sd.pidx[p] = sel[p / k].lidx[p % k];
            U.sd.pw[p] = sel[p / k].lw[p % k];
        }
        __syncthreads();
    }
    if (wave == 1 && lane >= 3 && lane < 16)
        P.ctl[lane] = lane == 3 ? lit_s : lane == 4 ? chain_s : 0;  // ctl[0..2]: the dispatch's
    if (wave == 0) {
        if (T == 1)
            dispatch_one(sel[0].lidx, sel[0].lw, E, k, P.ep_lo, P.ep_n, P.has_shared, P.ctl,
                         P.slot_expert, P.slot_off, P.slot_cnt, P.row_token, P.pair_row,
                         P.items, P.items_max, nullptr);
        else
            dispatch_wave(U.sd.dl, U.sd.pidx, U.sd.pw, T, k, E, P.ep_lo, P.ep_n, P.has_shared,
                          P.ctl, P.slot_expert, P.slot_off, P.slot_cnt, P.row_token, P.pair_row,
                          P.items, P.items_max, P.tchunk);
    }
    // the next launch's tag: every work group of this one read the current
    // generation before it counted itself in
    if (tid == 0)
        __hip_atomic_fetch_add(&sync64[SYNC64_GEN], (uint64_t)1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

extern "C" int ornk_route_cert_supported(int T, int D, int E, int k)
{
    const int nq = D / 256;
    return T >= 1 && T <= ORN_CERT_MAX_T && D % 256 == 0 && (nq == 1 || nq == 2 || nq == 4 ||
           nq == 8 || nq == 16) && E >= 1 && E <= 256 && k >= 1 && k <= 16 && k <= E;
}

extern "C" int ornk_moe_route_cert(const ornk_moe_args *a, hipStream_t s)
{
    const int T = a->T, D = a->D, E = a->E;
    if (!ornk_route_cert_supported(T, D, E, a->k)) return hipErrorInvalidValue;
    if (a->ep_lo < 0 || a->ep_n < 0 || a->ep_lo + a->ep_n > E || !a->route_est || !a->sync)
        return hipErrorInvalidValue;
    if (T * a->k > ORN_CERT_MAX_T * 16 || a->tchunk < 1) return hipErrorInvalidValue;
    CertArgs P;
    P.x = a->x;
    P.router = a->router;
    P.bias = a->bias;
    P.norm_w = a->apply_norm ? a->norm_w : nullptr;
    P.xn = a->xn;
    P.x_amax = a->router_amax ? a->x_amax : nullptr;
    P.logits = a->logits;
    P.est = reinterpret_cast<uint64_t *>(a->route_est);
    P.sync = a->sync;
    P.idx = a->idx;
    P.w = a->w;
    P.ctl = a->ctl;
    P.slot_expert = a->slot_expert;
    P.slot_off = a->slot_off;
    P.slot_cnt = a->slot_cnt;
    P.row_token = a->row_token;
    P.pair_row = a->pair_row;
    P.items = reinterpret_cast<int4 *>(a->items);
    P.T = T;
    P.E = E;
    P.k = a->k;
    P.mode = a->mode;
    P.ep_lo = a->ep_lo;
    P.ep_n = a->ep_n;
    P.has_shared = a->has_shared;
    P.items_max = a->items_max;
    P.tchunk = a->tchunk;
    P.ngroups = (E + CERT_EPG - 1) / CERT_EPG;
    const dim3 grid(P.ngroups + (P.norm_w ? 1 : 0));  // + the rmsnorm's group
    switch (D / 256) {
    case 1: ORN_LAUNCH_EV(a, k_route_cert<1>, grid, dim3(256), 0, s, P); break;
    case 2: ORN_LAUNCH_EV(a, k_route_cert<2>, grid, dim3(256), 0, s, P); break;
    case 4: ORN_LAUNCH_EV(a, k_route_cert<4>, grid, dim3(256), 0, s, P); break;
    case 8: ORN_LAUNCH_EV(a, k_route_cert<8>, grid, dim3(256), 0, s, P); break;
    case 16: ORN_LAUNCH_EV(a, k_route_cert<16>, grid, dim3(256), 0, s, P); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
