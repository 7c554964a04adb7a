"""CPU tests of the certified router's error bound (ssa_amd/csrc/route.hip, route_score_mfma_kernel
and cert_band).

The router's approximate score is one bf16 MFMA contraction: every fp32 operand x of
A = [q | c2 fl32(q*q) | c3 fl32(fl32(q*q)*q)] and B = [mu | var | m3] is split into bf16 parts
hi = bf16(x), lo = bf16(x - hi), and a.b is taken as hi.hi + hi.lo + lo.hi, the 3n exact products
summed in fp32. The select kernels trust |approx - exact| <= e with
    e = ecoef (1 + 2^-10) emag + 2^-100,   ecoef = 1.03 (3n + 16) 2^-23 + 2^-14,
    emag = sum_t |A_t| |B_t| + 2^-56 sum_t (|A_t| + |B_t|),
where exact is the router's exact score (fp64 sums, fp32 assembly; oracle.scores). Here the
MFMA arithmetic is emulated in NumPy (round-to-nearest-even bf16, sequential fp32 accumulation in
index order and in a shuffled order) and the bound is checked on random, badly scaled,
cancelling and adversarially aligned inputs; on the aligned case (every lo part near 2^-8, one
sign) the bound without the split term 2^-14 fails, so the test tells the two formulas apart.
"""
import numpy as np
import pytest

from oracle import ssa_oracle as O


def bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bfloat16 (ties to even), returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return r.astype(np.uint32).view(np.float32)


def split(x: np.ndarray):
    hi = bf16(x)
    lo = bf16((x - hi).astype(np.float32))
    return hi, lo


def operands(q, mu, var, m3, c2, c3):
    """A rows (R, n) and B rows (C, n) of the contraction, in fp32 as the kernel stages them."""
    q2 = (q * q).astype(np.float32)
    a = [q, (np.float32(c2) * q2).astype(np.float32)]
    b = [mu, var]
    if m3 is not None:
        a.append((np.float32(c3) * (q2 * q).astype(np.float32)).astype(np.float32))
        b.append(m3)
    return a, b


def approx_scores(a, b, order):
    """fp32 sum of the 3n exact bf16 products per (row, candidate), added in `order`."""
    A = np.concatenate(a, axis=1)
    Bm = np.concatenate(b, axis=1)
    ah, al = split(A)
    bh, bl = split(Bm)
    # exact products (bf16 x bf16 fits fp32), three per head dim
    prods = np.concatenate([ah[:, None, :].astype(np.float64) * bh[None, :, :],
                            ah[:, None, :].astype(np.float64) * bl[None, :, :],
                            al[:, None, :].astype(np.float64) * bh[None, :, :]],
                           axis=2).astype(np.float32)
    return np.cumsum(prods[:, :, order], axis=2, dtype=np.float32)[:, :, -1]


def bound(a, b, n, split_term=True):
    na = [np.sqrt((x.astype(np.float64) ** 2).sum(1)) for x in a]
    nb = [np.sqrt((x.astype(np.float64) ** 2).sum(1)) for x in b]
    emag = sum(x[:, None] * y[None, :] for x, y in zip(na, nb))
    emag = emag + 2.0 ** -56 * sum(x[:, None] + y[None, :] for x, y in zip(na, nb))
    ecoef = 1.03 * (3 * n + 16) * 2.0 ** -23 + (2.0 ** -14 if split_term else 0.0)
    return ecoef * (1 + 2.0 ** -10) * emag + 2.0 ** -100


def cases():
    rng = np.random.default_rng(7)
    d = 64
    out = []
    for scale in (1e-3, 1.0, 1e3):
        q = (rng.standard_normal((16, d)) * scale).astype(np.float32)
        mu = (rng.standard_normal((48, d)) * scale).astype(np.float32)
        var = (rng.uniform(0.0, 2.0, (48, d)) * scale * scale).astype(np.float32)
        out.append((f"normal_{scale:g}", q, mu, var, None))
    # cancellation: mu orthogonal to q up to rounding, large norms
    q = rng.standard_normal((16, d)).astype(np.float32) * 100
    mu = rng.standard_normal((48, d)).astype(np.float32) * 100
    qn = q[0] / np.linalg.norm(q[0])
    mu = (mu - (mu @ qn)[:, None] * qn[None, :]).astype(np.float32)
    var = rng.uniform(0.0, 1e-3, (48, d)).astype(np.float32)
    out.append(("cancel", q, mu, var, None))
    # every element carries a full 24-bit mantissa (large lo parts) and mixed signs
    q = (rng.choice([-1, 1], (16, d)) * (1 + rng.integers(1, 2 ** 23, (16, d)) * 2.0 ** -23))
    mu = (rng.choice([-1, 1], (48, d)) * (1 + rng.integers(1, 2 ** 23, (48, d)) * 2.0 ** -23))
    out.append(("full_mantissa", q.astype(np.float32), mu.astype(np.float32),
                rng.uniform(0.5, 1.5, (48, d)).astype(np.float32), None))
    # edgeworth term, and tiny values whose lo parts fall below the bf16 normal range
    q = rng.standard_normal((16, d)).astype(np.float32)
    mu = rng.standard_normal((48, d)).astype(np.float32)
    m3 = rng.standard_normal((48, d)).astype(np.float32)
    out.append(("edgeworth", q, mu, rng.uniform(0.5, 1.5, (48, d)).astype(np.float32), m3))
    q = (rng.standard_normal((16, d)) * 2.0 ** -60).astype(np.float32)
    out.append(("tiny", q, mu, rng.uniform(0.5, 1.5, (48, d)).astype(np.float32), None))
    # aligned operands whose lo parts are all near 2^-8 (hi = 1): the dropped lo.lo products add
    # up to 2^-16 |a||b| with one sign, at a head dim (8) where the fp32 summation term is small
    x = np.float32(1 + 2.0 ** -8 - 2.0 ** -20)
    q = np.full((16, 8), x, np.float32) * rng.uniform(1, 1 + 2.0 ** -20, (16, 1)).astype(np.float32)
    mu = np.full((48, 8), x, np.float32)
    out.append(("aligned_lo", q.astype(np.float32), mu, np.zeros((48, 8), np.float32), None))
    return out


@pytest.mark.parametrize("name,q,mu,var,m3", cases(), ids=[c[0] for c in cases()])
def test_bf16_split_scores_within_the_certificate_bound(name, q, mu, var, m3):
    c2 = 1.0
    c3 = 2.0 / 3.0 if m3 is not None else 0.0
    a, b = operands(q, mu, var, m3, c2, c3)
    n = sum(x.shape[1] for x in a)
    exact = O.scores(q[None, None], mu[None, None], var[None, None], c2,
                     None if m3 is None else m3[None, None], c3)[0, 0].astype(np.float64)
    e = bound(a, b, n)
    rng = np.random.default_rng(3)
    for order in (np.arange(3 * n), rng.permutation(3 * n)):
        err = np.abs(approx_scores(a, b, order).astype(np.float64) - exact)
        assert (err <= e).all(), (name, float((err / e).max()))


def test_fp32_bound_is_too_tight_for_the_split():
    """Without the split term the bound fails: the test distinguishes the two formulas."""
    worst = 0.0
    for name, q, mu, var, m3 in [c for c in cases() if c[0] == "aligned_lo"]:
        a, b = operands(q, mu, var, m3, 1.0, 0.0)
        n = sum(x.shape[1] for x in a)
        exact = O.scores(q[None, None], mu[None, None], var[None, None], 1.0)[0, 0]
        err = np.abs(approx_scores(a, b, np.arange(3 * n)).astype(np.float64) - exact)
        worst = max(worst, float((err / bound(a, b, n, split_term=False)).max()))
    assert worst > 1.0
