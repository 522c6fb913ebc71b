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


# ---------------------------------------------------------------------------
# With the layer's rmsnorm the reference's products are
#   p_i = fl(fl(w_i * fl(x_i * inv)) * W_i),  inv = fl(1 / fl(sqrt(fl(fl(ss / D) + 1e-6)))),
# ss the sequential fp32 sum of fl(x_i^2) (gpu.c:144-156).  The kernel sums
# q_i = fl(fl(x_i * w_i) * W_i) into T while the chain of ss runs elsewhere,
# and bounds |chain(p) - inv T| <= inv B_T with
#   B_T = u (A_q + 5.0001 n u Q) (1 + 1e-3) / (1 - n u) + 5.0001 u Q,
# Q = sum |q_i| (times 1 + 1e-3).  The selecting group then packs fp32
# (sf, bf) words and forms S = inv sf (+ bias), B = inv bf (+ the bias add's
# rounding).
# ---------------------------------------------------------------------------


def ref_inv(x):
    """The reference's rmsnorm scale (gpu.c:144-156), in fp32 throughout."""
    ss = chain((x * x).astype(np.float32))
    D = np.float32(x.size)
    return np.float32(np.float32(1.0) / np.sqrt(np.float32(np.float32(ss / D) + np.float32(1e-6))))


def q_parts(q, nch=64):
    """T, S_abs (the chunked partial-sum bound) and Q = sum |q| as the kernel forms them."""
    q = np.asarray(q, np.float32).astype(np.float64)
    L = q.size // nch
    l = np.cumsum(q.reshape(nch, L), axis=1)
    Tc = l[:, -1]
    A = np.abs(l.astype(np.float32)).sum(axis=1, dtype=np.float32).astype(np.float64)
    O = np.concatenate([[0.0], np.cumsum(Tc)[:-1]])
    return Tc.sum(), (L * np.abs(O) + A).sum(), np.abs(q).sum()


def norm_bound(sabs, Q, n, rounding_term=True):
    qa = Q * (1.0 + 1e-3)
    if not rounding_term:
        return U * sabs * (1.0 + 1e-3) / (1.0 - n * U) + 1e-30
    return (U * (sabs + 5.0001 * n * U * qa) * (1.0 + 1e-3) / (1.0 - n * U) +
            5.0001 * U * qa + 1e-30)


def f_up(v):
    f = np.float32(v)
    return f if float(f) >= v else np.nextafter(f, np.float32(np.inf))


def norm_case(x, w, W, bias=None, rounding_term=True):
    """(reference logit, S, B) for one expert column W."""
    inv = ref_inv(x)
    xn = (w * (x * inv)).astype(np.float32)
    ref = chain((xn * W).astype(np.float32))
    if bias is not None:
        ref = np.float32(ref + np.float32(bias))
    T, sabs, Q = q_parts(((x * w).astype(np.float32) * W).astype(np.float32))
    BT = norm_bound(sabs, Q, x.size, rounding_term)
    sf = np.float32(T)
    bf = f_up(BT + abs(T - float(sf)))
    S = float(inv) * float(sf)
    B = float(inv) * float(bf)
    if bias is not None:
        S += float(bias)
        B += U * (abs(S) + B) * (1.0 + 1e-6) + 1e-30
    return float(ref), S, B


def adversarial_norm_row(seed, D=256):
    """W chosen so that every p_i - inv q_i is positive while the partial
    sums stay near zero: the products' roundings add up, the chain's own
    error stays small."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(D).astype(np.float32)
    w = (1 + 0.25 * rng.standard_normal(D)).astype(np.float32)
    inv = ref_inv(x)
    xn = (w * (x * inv)).astype(np.float32)
    xw = (x * w).astype(np.float32)
    W = np.zeros(D, np.float32)
    s = 0.0
    for i in range(D):
        want = -1.0 if s > 0 else 1.0
        Wi = np.float32(want * np.sign(xw[i]) / abs(float(xw[i])))
        for kk in range(256):
            cand = np.float32(want * np.sign(xw[i]) * (1.0 + kk * 2.0 ** -18) / abs(float(xw[i])))
            if float(np.float32(xn[i] * cand)) - float(inv) * float(np.float32(xw[i] * cand)) > 0:
                Wi = cand
                break
        W[i] = Wi
        s += float(np.float32(xw[i] * Wi))
    return x, w, W


def test_norm_factored_bound_on_router_rows():
    rng = np.random.default_rng(7)
    D = 2048
    worst = 0.0
    for r in range(8):
        x = rng.standard_normal(D).astype(np.float32)
        w = (1 + 0.25 * rng.standard_normal(D)).astype(np.float32)
        for e in range(16):
            W = (0.02 * rng.standard_normal(D)).astype(np.float32)
            ref, S, B = norm_case(x, w, W)
            assert abs(ref - S) <= B
            worst = max(worst, abs(ref - S) / B)
            b = np.float32(0.5 * rng.standard_normal())
            ref, S, B = norm_case(x, w, W, bias=b)
            assert abs(ref - S) <= B
    assert worst < 0.5


def test_norm_factored_bound_on_adversarial_rows():
    worst = 0.0
    for seed in range(5):
        x, w, W = adversarial_norm_row(seed)
        ref, S, B = norm_case(x, w, W)
        assert abs(ref - S) <= B
        worst = max(worst, abs(ref - S) / B)
    assert worst > 0.05  # the rows do stress the rounding term


def test_dropped_rounding_term_fails():
    """Without the 5.0001 u Q terms (p_i taken as inv q_i exactly) the
    adversarial rows break the bound."""
    bad = 0
    for seed in range(5):
        x, w, W = adversarial_norm_row(seed)
        ref, S, B = norm_case(x, w, W, rounding_term=False)
        bad += abs(ref - S) > B
    assert bad >= 2
