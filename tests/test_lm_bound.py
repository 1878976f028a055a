"""The bound behind the LM head's int8 copy (ds-ocr_amd/csrc/k_lm.hip: k_lm_q8_build, k_lm_q8_argmax),
checked on the CPU over more than 10^6 rows against the reference's own logits.

For a bf16 row w, the int8 copy keeps q = rint(w / s) (s = max|w| / 127) with alpha = gamma_n ||w||_2 +
||w - s q||_2 and beta = s ||q||_1 (gamma_n for n = H/32 + 5 roundings); a step puts the input on the
grid 2^(e-14) (|x| < 2^e) as two 8-bit limbs and takes A = s 2^(e-14) (256 q.hi + q.lo), exact in
integers, and B = alpha ||x||_2 + beta 2^(e-15) + 2^-22 |A|. The kernel prunes a row only when
A + B is below another row's A - B, which is sound when every row's logit in the reference's order,
L (ds_kernels_avx.c:162-228, 4-row groups; the oracle's or_argmax_logits_avx512, pinned to the
reference build by tests/test_oracle_ref.py), lies in [A - B, A + B]. This restates both steps in
numpy and checks that interval on random heads at H = 1280 and 2048, on inputs with one dominant
coordinate (over rows whose codes are exact), on all-positive products (the rounding of the exact
order grows fastest) and on rows with one large weight (coarse codes). The check sees each term:
without the quantization term the random rows break it, and without the grid term the
dominant-coordinate inputs do."""
import numpy as np
import pytest

F, D = np.float32, np.float64


def f32_up(d):
    f = d.astype(F)
    lo = f.astype(D) < d
    f[lo] = np.nextafter(f[lo], F(np.inf))
    return f


def q8_build(W16, H):
    """k_lm_q8_build: codes q and (s, alpha, beta) per row."""
    v = (W16.astype(np.uint32) << 16).view(F)
    amax = np.max(np.abs(v), axis=1)
    s = (amax / F(127.0)).astype(F)
    inv = np.where(amax > 0, (F(1.0) / np.where(s > 0, s, F(1.0))).astype(F), F(0.0)).astype(F)
    q = np.clip(np.rint((v * inv[:, None]).astype(F)), -127, 127).astype(np.int8)
    d = v.astype(D) - s.astype(D)[:, None] * q.astype(D)
    n = H // 32 + 5
    gam = n * 2.0 ** -24 / (1.0 - n * 2.0 ** -24)
    w2 = np.sum(v.astype(D) ** 2, axis=1)
    r2 = np.sum(d * d, axis=1)
    q1 = np.sum(np.abs(q.astype(D)), axis=1)
    alpha = f32_up((gam * np.sqrt(w2) + np.sqrt(r2)) * (1.0 + 1e-12))
    beta = f32_up(s.astype(D) * q1 * (1.0 + 1e-12))
    alpha_noq = f32_up(gam * np.sqrt(w2) * (1.0 + 1e-12))  # the quantization term dropped
    return q, s, alpha, beta, alpha_noq


def q8_step(x, q, s, alpha, beta, alpha_noq):
    """k_lm_q8_argmax's per-row A and B (and B with a term dropped, for the sensitivity checks)."""
    xmax = np.max(np.abs(x))
    e = int(np.frexp(xmax)[1])  # xmax < 2^e
    x2 = np.sqrt(np.sum(x.astype(D) ** 2) * (1.0 + 1e-12))
    X = np.rint(np.ldexp(x, 14 - e).astype(F)).astype(np.int64)
    assert np.all(np.abs(X) <= 1 << 14)
    lo = ((X & 0xFF) ^ 0x80) - 0x80
    hi = (X - lo) >> 8
    assert np.all((lo >= -128) & (lo <= 127) & (hi >= -64) & (hi <= 64))
    qd = q.astype(D)
    dlo, dhi = qd @ lo.astype(D), qd @ hi.astype(D)  # exact: |sum| < 2^25
    A = s.astype(D) * 2.0 ** (e - 14) * (256.0 * dhi + dlo)
    half = 2.0 ** (e - 15)
    B = alpha.astype(D) * x2 + beta.astype(D) * half + 2.0 ** -22 * np.abs(A)
    B_noq = alpha_noq.astype(D) * x2 + beta.astype(D) * half + 2.0 ** -22 * np.abs(A)
    B_nogrid = alpha.astype(D) * x2 + 2.0 ** -22 * np.abs(A)
    return A, B, B_noq, B_nogrid


def ref_logits(B, x, W16, H):
    R = W16.shape[0]
    assert R % 4 == 0  # every row in a 4-row group, as for the heads the kernel accepts
    lg = np.empty(R, F)
    B.oracle().or_argmax_logits_avx512(lg, np.ascontiguousarray(x, F), np.ascontiguousarray(W16), H, R, 1)
    return lg


def make_rows(rng, R, H, kind):
    """bf16 rows from random bits: sign, 7 mantissa bits and exponents over [2^-9, 2^-1) (a wider
    range of magnitudes than a trained head's); "positive": no signs; "spike": one weight of 0.9 per
    row (coarse codes for the rest); "exact": w = k 2^-10 with |k| <= 127 and a +-127 in every row,
    so the codes are exact (no quantization error; the input's grid carries the bound)."""
    if kind == "exact":
        k = rng.integers(-127, 128, size=(R, H)).astype(F)
        k[np.arange(R), rng.integers(0, H, R)] = F(127.0) * rng.choice([F(-1.0), F(1.0)], R)
        return ((k * F(2.0 ** -10)).view(np.uint32) >> 16).astype(np.uint16)
    bits = rng.integers(0, 1 << 16, size=(R, H), dtype=np.uint16)
    W16 = (bits & np.uint16(0x807F)) | ((np.uint16(118) + ((bits >> 7) & np.uint16(7))) << 7).astype(np.uint16)
    if kind == "positive":
        W16 &= np.uint16(0x7FFF)
    if kind == "spike":
        W16[np.arange(R), rng.integers(0, H, R)] = np.uint16(0x3F66)  # 0.8984375
    return W16


def make_input(rng, H, kind):
    x = rng.standard_normal(H).astype(F)
    if kind == "positive":
        x = (np.abs(x) + F(0.5)).astype(F)
    if kind == "dominant":
        x = (x * F(1e-3)).astype(F)
        x[int(rng.integers(0, H))] = F(1000.0)
    return x


CASES = [  # (H, kind, rows): 1,081,344 rows in all
    (1280, "random", 393216),
    (2048, "random", 393216),
    (2048, "dominant", 98304),
    (1280, "dominant", 65536),
    (2048, "positive", 65536),
    (2048, "spike", 65536),
]


@pytest.mark.parametrize("H,kind,rows", CASES)
def test_lm_q8_bound_holds(B, H, kind, rows):
    rng = np.random.default_rng(H * 7 + len(kind))
    worst, broken_noq, broken_nogrid, n = 0.0, 0, 0, 0
    batch = 16384
    for b0 in range(0, rows, batch):
        W16 = make_rows(rng, batch, H, "exact" if kind == "dominant" else kind)
        x = make_input(rng, H, kind)
        q, s, alpha, beta, alpha_noq = q8_build(W16, H)
        A, Bd, B_noq, B_nogrid = q8_step(x, q, s, alpha, beta, alpha_noq)
        L = ref_logits(B, x, W16, H).astype(D)
        err = np.abs(L - A)
        assert np.all(np.isfinite(L)) and np.all(err <= Bd), (b0, float(np.max(err / Bd)))
        worst = max(worst, float(np.max(err / Bd)))
        broken_noq += int(np.sum(err > B_noq))
        broken_nogrid += int(np.sum(err > B_nogrid))
        n += batch
    print(f"H={H} {kind}: {n} rows, largest |L - A| / B = {worst:.3f}; without the quantization term "
          f"{broken_noq} rows break it, without the grid term {broken_nogrid}")
    if kind == "random":
        assert broken_noq > 0
    if kind == "dominant":
        assert broken_nogrid > 0


@pytest.mark.parametrize("H", [1280, 2048])
def test_lm_gamma_count_is_reached(B, H):
    """The rounding term gamma_n with n = H/32 + 5 (H/32 fused multiply-adds per chain of the
    reference's two 16-lane accumulators, a0 + a1, 4 levels of the 16-lane tree) is nearly reached:
    each of the 32 chains starts at 1 and then adds products of 1.0078125 2^-24, just over half an ulp
    of the running sum, so every step rounds up by almost half an ulp; the tree's additions are exact.
    The reference's logit then errs by about 0.93 gamma_n sum|w x|, inside the bound, while a count
    of H/64 + 5 roundings would not cover it."""
    x = np.ones(H, F)
    row = np.full(H, 0x3381, np.uint16)  # 1.0078125 * 2^-24
    row[:32] = 0x3F80  # 1.0: the first product of each of the 32 chains
    W16 = np.tile(row, (4, 1))
    L = ref_logits(B, x, W16, H).astype(D)
    w = (W16[0].astype(np.uint32) << 16).view(F).astype(D)
    exact, mag = float(np.sum(w)), float(np.sum(np.abs(w)))  # exact in f64
    gam = lambda n: n * 2.0 ** -24 / (1.0 - n * 2.0 ** -24)
    err = float(np.max(np.abs(L - exact)))
    ratio = err / (gam(H // 32 + 5) * mag)
    print(f"H={H}: |L - sum w x| = {err:.3e} = {ratio:.3f} gamma_(H/32+5) sum|w x|")
    assert ratio <= 1.0
    assert err > gam(H // 64 + 5) * mag
