"""CPU check of the fast path of the device's exact top-k selection
(select.h select_token): each of the 64 lanes sorts its four (key, expert)
pairs (expert = lane + 64*i) once and offers its head; a round takes the
maximum head, requires that one lane alone offers it (else: a tie, the
literal path), and the winning lane drops its head; k+1 rounds, each
maximum strictly below the previous one (in the literal mode by more than
1e-5).  An expert equal to a winner inside the winner's own lane is not
seen by the head check; it comes up as the next round's maximum and fails
the strict-order check.  Whenever this emulation keeps the fast path, its
k experts must be the reference's exchange selection (oracle.topk, the
reference's own code path model.c:301-317 / 1040-1048); the crafted ties
below must leave it exactly when they matter.
"""
import numpy as np
import pytest

from oracle import oracle as O

INT_MIN = -(2 ** 31)


def sel_key(f):
    b = int(np.float32(f).view(np.int32))
    b = 0 if b == INT_MIN else b
    return b if b >= 0 else b ^ 0x7FFFFFFF


def tournament(logits, k, mode):
    """(indices, slow) as select_token's fast path forms them."""
    E = logits.size
    lanes = []
    for lane in range(64):
        sl = []
        for i in range(4):
            e = lane + 64 * i
            sl.append((sel_key(logits[e]), e) if e < E else (INT_MIN, e))
        # the compare-swap network cs(0,1) cs(2,3) cs(0,2) cs(1,3) cs(1,2),
        # swapping when the second key is strictly larger
        for a, b in ((0, 1), (2, 3), (0, 2), (1, 3), (1, 2)):
            if sl[b][0] > sl[a][0]:
                sl[a], sl[b] = sl[b], sl[a]
        lanes.append(sl)
    if not np.all(np.isfinite(logits)):
        return None, True
    out, prev = [], None
    rounds = k + 1 if k < E else k
    for r in range(rounds):
        heads = [l[0][0] for l in lanes]
        mk = max(heads)
        owners = [i for i, h in enumerate(heads) if h == mk]
        if len(owners) != 1:
            return None, True
        o = owners[0]
        e = lanes[o][0][1]
        m = np.float32(logits[e])
        lanes[o] = lanes[o][1:] + [(INT_MIN, -1)]
        if r > 0:
            if not prev > m:
                return None, True
            if mode == 1 and not (float(prev) - float(m) > 1e-5):
                return None, True
        out.append(e)
        prev = m
    return np.array(out[:k], np.uint32), False


def check(logits, k, mode):
    idx, slow = tournament(logits, k, mode)
    if not slow:
        ref, _ = O.topk(logits, k, mode)
        assert np.array_equal(idx, ref), (idx, ref)
    return slow


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("E", [256, 100, 9])
def test_random_logits_take_the_fast_path(E, mode):
    rng = np.random.default_rng(10 + E + mode)
    for _ in range(50):
        lg = (2.0 * rng.standard_normal(E)).astype(np.float32)
        assert not check(lg, 8, mode)


def base(seed=3):
    return (2.0 * np.random.default_rng(seed).standard_normal(256)).astype(np.float32)


def with_rank(lg, order, r, e, value=None):
    """Place expert e at value of the current rank-r expert (a tie)."""
    lg = lg.copy()
    lg[e] = lg[order[r]] if value is None else value
    return lg


def test_tie_across_lanes_goes_literal():
    lg = base()
    order = np.argsort(-lg, kind="stable")
    top = order[0]
    other = (top + 1) % 256 if ((top + 1) % 64) != (top % 64) else (top + 2) % 256
    assert other % 64 != top % 64
    assert check(with_rank(lg, order, 0, other), 8, 0)


@pytest.mark.parametrize("r", [0, 3, 7])
def test_tie_inside_a_lane_goes_literal(r):
    """The tied partner sits in the same lane (expert + 64): the head check
    cannot see it, the next round's strict-order check must."""
    lg = base()
    order = np.argsort(-lg, kind="stable")
    e = order[r]
    partner = (e + 64) % 256
    assert check(with_rank(lg, order, r, partner), 8, 0)


def test_tie_below_the_boundary_keeps_the_fast_path():
    """Ranks k+1 and k+2 tied inside one lane: the top k are unaffected and
    the fast path must still return the reference's selection."""
    lg = base()
    order = np.argsort(-lg, kind="stable")
    e = order[8]
    partner = (e + 64) % 256
    lg2 = lg.copy()
    # put the partner just below rank 8's value (rank 9), then tie them
    lg2[partner] = lg2[e]
    idx, slow = tournament(lg2, 8, 0)
    assert not slow
    ref, _ = O.topk(lg2, 8, 0)
    assert np.array_equal(idx, ref)


def test_signed_zero_pair_is_a_tie():
    lg = np.full(256, -1.0, np.float32)
    lg[5] = 0.0
    lg[6] = -0.0
    assert check(lg, 8, 0)


def test_literal_mode_small_gap_goes_literal():
    lg = base()
    order = np.argsort(-lg, kind="stable")
    lg2 = lg.copy()
    lg2[order[2]] = np.nextafter(lg2[order[1]], np.float32(-np.inf))
    assert check(lg2, 8, 1)
    # the same gap is fine in the renormalising mode (strict order holds)
    assert not check(lg2, 8, 0)
