"""CPU check of the bound the certified router (router_cert.hip) puts on the
distance between the reference's sequential fp32 logit chain
(model.c:1017-1025) and the fp64 sum of the same fp32 products.

The kernel splits the D products into 64 chunks of L = D/64 consecutive
values and forms, per chunk c, its sum T_c and A_c = sum_i |l_i| over the
chunk's running sums l_i; then, with O_c the sum of the chunks before c,
    S_abs = sum_c (L |O_c| + A_c),   B = u S_abs (1 + 1e-3) / (1 - n u).
numpy's float32 add.accumulate is the sequential fp32 chain itself, so the
bound is checked against the chain directly, on random router-shaped rows
and on adversarial ones (steady one-directional rounding, heavy
cancellation, huge leading terms), and two plausible mistakes -- dropping
the L |O_c| term, or bounding by u |S| alone -- are shown to fail.
"""
import numpy as np

U = 2.0 ** -24


def chain(p):
    """The reference's sequential fp32 sum from 0 (model.c:1017-1025)."""
    return np.add.accumulate(np.asarray(p, np.float32), dtype=np.float32)[-1]


def cert(p, nch=64, drop_offset=False):
    """(S, B) as router_cert.hip forms them."""
    p = np.asarray(p, np.float32).astype(np.float64)
    n = p.size
    L = n // nch
    chunks = p.reshape(nch, L)
    l = np.cumsum(chunks, axis=1)                   # running sums (fp64)
    T = l[:, -1]
    A = np.abs(l.astype(np.float32)).sum(axis=1, dtype=np.float32).astype(np.float64)
    O = np.concatenate([[0.0], np.cumsum(T)[:-1]])
    sabs = (A.sum() if drop_offset else (L * np.abs(O) + A).sum())
    S = T.sum()
    B = U * sabs * (1.0 + 1e-3) / (1.0 - n * U) + 1e-30
    return S, B


def violations(rows, **kw):
    bad = 0
    worst = 0.0
    for p in rows:
        S, B = cert(p, **kw)
        err = abs(float(chain(p)) - S)
        worst = max(worst, err / B)
        bad += err > B
    return bad, worst


def router_rows(rng, n_rows, D=2048):
    x = rng.standard_normal(D).astype(np.float32)
    W = (0.02 * rng.standard_normal((n_rows, D))).astype(np.float32)
    return [(x * w).astype(np.float32) for w in W]


def adversarial_rows(D=2048):
    rows = []
    # steady upward rounding: 1 + many terms of 0.75 ulp(1)
    p = np.full(D, 1.5 * 2.0 ** -24, np.float32)
    p[0] = 1.0
    rows.append(p)
    # the same below a large leading term, then cancelled
    q = np.full(D, 1.5 * 2.0 ** -14, np.float32)
    q[0] = 1024.0
    q[-1] = -1024.0
    rows.append(q)
    # alternating huge terms that cancel, small ones in between
    r = np.tile(np.array([3.0e4, 1.0e-3, -3.0e4, 7.0e-4], np.float32), D // 4)
    rows.append(r)
    # geometric growth
    rows.append((1.001 ** np.arange(D)).astype(np.float32))
    # positive squares (the rmsnorm's sum)
    rng = np.random.default_rng(3)
    rows.append((rng.standard_normal(D) ** 2).astype(np.float32))
    return rows


def test_bound_holds_on_router_rows():
    rng = np.random.default_rng(1)
    bad, worst = violations(router_rows(rng, 256))
    assert bad == 0
    # the bound is rigorous, not tight: the chain typically sits far inside
    assert worst < 0.5


def test_bound_holds_on_adversarial_rows():
    bad, worst = violations(adversarial_rows())
    assert bad == 0
    # steady rounding reaches a sizeable fraction of the bound
    assert worst > 0.2


def test_bound_with_bias_term():
    """A router bias is one more add after the chain: n = D + 1 terms."""
    rng = np.random.default_rng(2)
    for p in router_rows(rng, 64):
        b = np.float32(rng.standard_normal() * 0.5)
        ref = np.float32(chain(p) + b)
        S, B = cert(p)
        S += float(b)
        # the kernel adds |S + b| to S_abs for the bias add
        _, B0 = cert(p)
        sabs = (B0 - 1e-30) / U / (1.0 + 1e-3) * (1.0 - p.size * U)
        B = U * (sabs + abs(S)) * (1.0 + 1e-3) / (1.0 - (p.size + 1) * U) + 1e-30
        assert abs(float(ref) - S) <= B


def test_dropped_offset_term_fails():
    """Without L |O_c| a chunk's partial sums are bounded as if they started
    at zero: the steady-rounding row breaks it."""
    bad, _ = violations(adversarial_rows()[:1], drop_offset=True)
    assert bad == 1


def test_final_sum_bound_fails():
    """u |S| (the rounding of the final value alone) is no bound on a chain."""
    p = adversarial_rows()[0]
    S, _ = cert(p)
    assert abs(float(chain(p)) - S) > U * abs(S) * 10
