"""The rounding bound behind the certified CFG expert selection (ds-ocr_amd/csrc/dsh_cert.h), checked
on the CPU against ds_linear's own order (the oracle's or_linear_f32, pinned bit for bit to the
reference's ds_linear, ds_kernels.c:639-652, by tests/test_oracle_ref.py) and ds_moe_top_k
(or_moe_top_k, ds_kernels.c:193-243).

A numpy model of the decode path's scores (R-row partials, each a sequential f32 sum of rounded
products, which the bound allows: any order with at most R roundings per term; the partials of four
contiguous ranges summed sequentially, then ((r0 + r1) + r2) + r3) gives the centre c and the prefix
sizes; cert_radius restates cert_radius_partials operation by operation in f32. The reference's
score must lie within c +- eps for every expert, over random routers and inputs and over inputs built
to make ds_linear's chain err the most (every product of one sign, products of 0.1, a dominant
coordinate). The check is sensitive: the same data break a bound with the prefix term dropped (the
running-error part) and the plain 2 gamma_{H+1} ||w|| ||x|| bound is shown to be far looser. Where the
intervals certify a selection, it is ds_moe_top_k's, in rank order."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "oracle"))

F = np.float32
U = F(2.0 ** -24)


def model_scores(W, x, R):
    """c, r[4], lam[4], nb[4] of route_reduce + route_init for router W [E][H] and input x."""
    E, H = W.shape
    NB = H // R
    prod = (W * x[None, :]).astype(F).reshape(E, NB, R)
    q = np.zeros((E, NB), F)
    for j in range(R):
        q = (q + prod[:, :, j]).astype(F)
    P = (NB + 3) // 4
    r = np.zeros((4, E), F)
    lam = np.zeros((4, E), F)
    nb = [max(0, min(P, NB - v * P)) for v in range(4)]
    for v in range(4):
        acc = np.zeros(E, F)
        lm = np.zeros(E, F)
        for b in range(v * P, v * P + nb[v]):
            lm = (lm + np.abs(acc)).astype(F)
            acc = (acc + q[:, b]).astype(F)
        r[v], lam[v] = acc, lm
    c = (((r[0] + r[1]).astype(F) + r[2]).astype(F) + r[3]).astype(F)
    return c, r, lam, nb


def cert_radius(r, lam, nb, R, H, wn, xn, drop_prefix=False):
    """cert_radius_partials (dsh_cert.h) in f32, one operation at a time."""
    g10 = F(1.0) + F(2.0 ** -10)
    A = (wn * xn * (F(1.0) + F(2.0 ** -20))).astype(F)
    O2 = (r[0] + r[1]).astype(F)
    O3 = (O2 + r[2]).astype(F)
    c = (O3 + r[3]).astype(F)
    lsum = ((lam[0] + lam[1]).astype(F) + (lam[2] + lam[3]).astype(F)).astype(F)
    rsum = ((lsum + (np.abs(r[0]) + np.abs(r[1])).astype(F)).astype(F) + (np.abs(r[2]) + np.abs(r[3])).astype(F)).astype(F)
    eC = (F(R) * U * g10 * A + U * rsum + U * ((np.abs(O2) + np.abs(O3)).astype(F) + np.abs(c)).astype(F)).astype(F)
    S1 = (F(R) * ((F(nb[1]) * np.abs(r[0]) + F(nb[2]) * np.abs(O2)).astype(F) + F(nb[3]) * np.abs(O3) + lsum)).astype(F)
    if drop_prefix:
        S1 = np.zeros_like(S1)
    nbt = F(sum(nb))
    run = (S1 + F(R) * nbt * eC + F(R) * A + F(H) * U * A).astype(F)
    return ((eC + U * A + U * g10 * run) * (F(1.0) + F(2.0 ** -16))).astype(F)


def norm_up(v):
    n = np.sqrt(np.sum(np.asarray(v, np.float64) ** 2, axis=-1))
    return np.nextafter(n.astype(F), F(np.inf))


def ref_scores(B, W, x):
    E, H = W.shape
    y = np.empty(E, F)
    B.oracle().or_linear_f32(y, np.ascontiguousarray(x, F), np.ascontiguousarray(W, F), H, E)
    return y


def check_case(B, W, x, R):
    E, H = W.shape
    c, r, lam, nb = model_scores(W, x, R)
    eps = cert_radius(r, lam, nb, R, H, norm_up(W), norm_up(x) * F(1.0 + 2.0 ** -10))
    s = ref_scores(B, W, x)
    err = np.abs(s.astype(np.float64) - c.astype(np.float64))
    assert np.all(err <= eps), (np.max(err / eps), np.argmax(err / eps))
    return c, eps, s, err


def certified_selection(c, eps, K):
    """cert_check's decision: (True, selection) when the intervals separate the ranks."""
    E = len(c)
    order = sorted(range(E), key=lambda e: (-float(c[e]), e))
    sel = order[:K]
    cd, ed = c.astype(np.float64), eps.astype(np.float64)
    lo = [cd[e] - ed[e] for e in sel]
    hi = [cd[e] + ed[e] for e in sel]
    ok = all(lo[i] > hi[i + 1] for i in range(K - 1))
    rest = [cd[e] + ed[e] for e in range(E) if e not in sel]
    ok = ok and (not rest or lo[K - 1] > max(rest))
    return ok, sel


@pytest.mark.parametrize("H,R", [(1280, 8), (256, 8), (2048, 16)])
def test_bound_holds_random(B, H, R):
    rng = np.random.default_rng(H + R)
    E, worst = 64, 0.0
    for trial in range(40):
        W = (rng.standard_normal((E, H)) * 0.02).astype(F)
        x = rng.standard_normal(H).astype(F)
        _, eps, _, err = check_case(B, W, x, R)
        worst = max(worst, float(np.max(err / eps)))
    print(f"H={H} R={R}: largest error / bound {worst:.3f}")


def test_bound_holds_adversarial_and_is_needed(B):
    """Inputs that make ds_linear's chain err the most: all products positive (prefix sums grow
    linearly, the case the running bound is widest for), products equal to 0.1f, one dominant input
    coordinate, and a router row that cancels. The bound holds on every one; with the prefix term
    dropped it fails on some (so the check sees that term)."""
    rng = np.random.default_rng(7)
    H, R, E = 1280, 8, 64
    cases = []
    W = np.abs(rng.standard_normal((E, H)) * 0.02).astype(F)
    cases.append((W, np.abs(rng.standard_normal(H)).astype(F) + F(0.5)))
    cases.append((np.full((E, H), 0.1, F) * (1 + np.arange(E, dtype=F)[:, None] * F(1e-3)), np.ones(H, F)))
    x = rng.standard_normal(H).astype(F)
    x[3] = F(1000.0)
    cases.append(((rng.standard_normal((E, H)) * 0.02).astype(F), x))
    Wc = (rng.standard_normal((E, H)) * 0.02).astype(F)
    Wc[:, 1::2] = -Wc[:, 0::2]
    cases.append((Wc, np.ones(H, F)))
    broken = 0
    for W, x in cases:
        c, r, lam, nb = model_scores(W, x, R)
        wn, xn = norm_up(W), norm_up(x) * F(1.0 + 2.0 ** -10)
        eps = cert_radius(r, lam, nb, R, H, wn, xn)
        weak = cert_radius(r, lam, nb, R, H, wn, xn, drop_prefix=True)
        s = ref_scores(B, W, x)
        err = np.abs(s.astype(np.float64) - c.astype(np.float64))
        print(f"case: largest error / bound {np.max(err / eps):.3f}, / weakened bound {np.max(err / weak):.3f}")
        assert np.all(err <= eps)
        broken += int(np.any(err > weak))
    assert broken >= 1


def test_bound_is_much_tighter_than_gamma(B):
    """On config-2-like data the radius is about 60x below 2 gamma_{H+1} ||w|| ||x||, the bound the
    prefill used before, which sent about a third of the tokens to the exact recomputation."""
    rng = np.random.default_rng(11)
    H, R, E = 1280, 8, 64
    W = (rng.standard_normal((E, H)) * 0.02).astype(F)
    x = rng.standard_normal(H).astype(F)
    c, r, lam, nb = model_scores(W, x, R)
    eps = cert_radius(r, lam, nb, R, H, norm_up(W), norm_up(x))
    gam = 2.0 * (H + 1) * 2.0 ** -24 / (1 - (H + 1) * 2.0 ** -24)
    old = gam * norm_up(W).astype(np.float64) * float(norm_up(x))
    ratio = float(np.median(old / eps))
    print(f"median 2 gamma_(H+1) ||w|| ||x|| / eps = {ratio:.1f}")
    assert ratio > 20


def test_certified_selection_is_the_references(B):
    """Over random layers, every selection the intervals certify is ds_moe_top_k's on the reference
    scores, in rank order; near ties planted between two router rows are never certified."""
    rng = np.random.default_rng(3)
    H, R, E, K = 1280, 8, 64, 6
    n_cert = 0
    for trial in range(200):
        W = (rng.standard_normal((E, H)) * 0.02).astype(F)
        x = rng.standard_normal(H).astype(F)
        if trial % 4 == 0:  # plant a near tie between the two best experts
            c0 = W @ x
            a, b = np.argsort(-c0)[:2]
            W[b] = W[a]
            W[b, 5] = np.nextafter(W[a, 5], F(np.inf))
        c, eps, s, _ = check_case(B, W, x, R)
        ok, sel = certified_selection(c, eps, K)
        ri = np.empty(K, np.int32)
        rw = np.empty(K, F)
        B.oracle().or_moe_top_k(ri, rw, s, E, K)
        if trial % 4 == 0:
            assert not ok
        if ok:
            n_cert += 1
            assert list(ri) == sel, (trial, list(ri), sel)
    print(f"certified {n_cert}/200 selections")
    assert n_cert >= 140
