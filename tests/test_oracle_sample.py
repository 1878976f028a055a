"""Pins the oracle's greedy token choice (or_lm_sample_greedy, ds_moe_decoder.c:1036-1095 and
:1105-1237) against formulations that do not share its structure: with no penalty and no ban it is
the plain argmax; with the penalty it is a maximum over penalised candidate logits (first occurrence
in history order on ties) instead of the reference's in-order scan; a banned choice gives the first
maximum of the full logits (the pinned matvec order) after per-occurrence penalties and bans,
computed here with numpy."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "oracle"))
import bindings as B  # noqa: E402

H, V = 256, 1500


def setup(seed):
    W = B.normal_bf16(V * H, seed, 0.02)
    x = B.normal_f32(H, seed + 1)
    return W, x


def sample(O, W, x, hist, rp, ngram, T=1):
    h = np.ascontiguousarray(hist, np.int32) if len(hist) else None
    used = C.c_int(-1)
    t = O.or_lm_sample_greedy(x, W, H, V, h, len(hist), rp, ngram, T, C.byref(used))
    return t, used.value


def dots(O, W, x, toks):
    return np.array([O.or_bf16_dot_row(x, W, H, int(t)) for t in toks], np.float32)


def pen(v, rp):
    v = np.float32(v)
    return np.float32(v / np.float32(rp)) if v > 0 else np.float32(v * np.float32(rp))


@pytest.mark.parametrize("T", [1, 3, 8])
def test_no_rules_is_the_argmax(T):
    O = B.oracle()
    for seed in range(5):
        W, x = setup(4000 + 10 * seed)
        hist = np.random.default_rng(seed).integers(0, V, 20)
        t, used = sample(O, W, x, hist, 1.0, 0, T)
        assert t == O.or_argmax_bf16(x, W, H, V, T, None) and used == 0


def near_tie(seed):
    """W, x and rows A = 0 (the argmax) and B = 1 with A's and B's exact dot products equal (B swaps
    two of A's elements whose x values are equal) but the argmax's AVX-512 order ranking A first
    while ds_bf16_dot_row's sequential order ranks B higher: the one case where the reference's
    fast-path penalty changes the token (the penalty itself preserves order)."""
    O = B.oracle()
    rng = np.random.default_rng(seed)
    W, x = setup(seed)
    W = W.reshape(V, H).copy()
    base = np.where(rng.random(H) < 0.5, 0x3D4D, 0x3D0F).astype(np.uint16)  # bf16 0.05, 0.035
    for _ in range(4000):
        k1, k2 = rng.choice(H, 2, replace=False)
        if base[k1] == base[k2]:
            continue
        xx = x.copy()
        xx[k2] = xx[k1]
        a = base | np.where(xx < 0, 0x8000, 0).astype(np.uint16)
        b = a.copy()
        b[k1], b[k2] = a[k2], a[k1]
        W4 = np.stack([a, b, W[2], W[3]])
        lg = np.empty(4, np.float32)
        O.or_argmax_logits_avx512(lg, xx, np.ascontiguousarray(W4), H, 4, 1)
        da = O.or_bf16_dot_row(xx, a, H, 0)
        db = O.or_bf16_dot_row(xx, b, H, 0)
        if lg[0] >= lg[1] and db > da:
            W[0], W[1] = a, b
            return np.ascontiguousarray(W).reshape(-1), xx
    raise AssertionError("no near tie found")


def test_penalty_switches_on_a_near_tie():
    O = B.oracle()
    for seed in (4700, 4710):
        W, x = near_tie(seed)
        assert O.or_argmax_bf16(x, W, H, V, 1, None) == 0
        t, used = sample(O, W, x, [7, 1, 0, 9], 1.2, 0)
        assert (t, used) == (1, 0)  # B's penalised dot beats A's penalised dot
        t2, _ = sample(O, W, x, [7, 9], 1.2, 0)
        assert t2 == 0  # B not in the history: no candidate


def test_penalty_is_a_max_over_candidates():
    O = B.oracle()
    rng = np.random.default_rng(7)
    changed = 0
    for seed in range(12):
        W, x = setup(4100 + 10 * seed)
        best0 = O.or_argmax_bf16(x, W, H, V, 1, None)
        lg = np.empty(V, np.float32)
        O.or_argmax_logits_avx512(lg, x, W, H, V, 1)
        top = np.argsort(-lg)[:40]
        hist = rng.choice(top, 30)
        if seed % 2:
            hist = np.concatenate([hist, [best0], [-3, V + 2]])  # the argmax itself, invalid ids
        rng.shuffle(hist)
        rp = 1.0 + 0.5 * rng.random()
        t, used = sample(O, W, x, hist, rp, 0)
        assert used == 0
        b0 = O.or_bf16_dot_row(x, W, H, best0)
        bv = pen(b0, rp) if best0 in hist else np.float32(b0)
        cand = [(i, int(tk)) for i, tk in enumerate(hist) if 0 <= tk < V and tk != best0]
        vals = np.array([pen(v, rp) for v in dots(O, W, x, [tk for _, tk in cand])], np.float32)
        k = int(np.argmax(vals))  # first maximum in history order
        expect = cand[k][1] if vals[k] > bv else best0
        assert t == expect, seed
        changed += t != best0
    assert changed == 0  # the penalty is monotone: away from near ties it keeps the argmax


def test_banned_choice_takes_the_full_path():
    O = B.oracle()
    rng = np.random.default_rng(11)
    for seed in range(6):
        W, x = setup(4300 + 10 * seed)
        best0 = O.or_argmax_bf16(x, W, H, V, 1, None)
        a, b = rng.integers(0, V, 2)
        hist = np.array(list(rng.integers(0, V, 5)) + [a, b, best0] + list(rng.integers(0, V, 4)) + [best0, a, b],
                        np.int32)
        rp = 1.25 if seed % 2 else 1.0
        t, used = sample(O, W, x, hist, rp, 3)
        assert used == 1
        lg = np.empty(V, np.float32)
        O.or_bf16_matvec_avx512(lg, x, W, H, V, 1)
        if rp > 1:
            for tk in hist:  # once per occurrence
                lg[tk] = pen(lg[tk], rp)
        for i in range(len(hist) - 2):
            if hist[i] == hist[-2] and hist[i + 1] == hist[-1]:
                lg[hist[i + 2]] = np.float32(-1e30)
        assert lg[best0] == np.float32(-1e30)
        assert t == int(np.argmax(lg))


def test_ngram_one_bans_every_history_token():
    O = B.oracle()
    W, x = setup(4500)
    best0 = O.or_argmax_bf16(x, W, H, V, 1, None)
    t, used = sample(O, W, x, [5, best0, 7], 1.0, 1)
    assert used == 1 and t not in (5, best0, 7)
    t2, used2 = sample(O, W, x, [5, 6, 7], 1.0, 1)
    assert used2 == 0 and t2 == best0
    t3, used3 = sample(O, W, x, [], 1.3, 2)
    assert used3 == 0 and t3 == best0
