"""CPU pins of the treecode oracle (oracle.ssa_oracle.tree_build / tree_descend), the
restatement of ssa/treecode.py. The reference holds no tests or fixtures for this module; its own
validation (treecode.py:141-200) checks the admissible invariant and that the beam's recall climbs
to the flat full-scan ceiling, which the tests below restate, beside closed forms and the
reduction of a beam that holds every node to the flat top_c of the leaf bounds."""
import math

import numpy as np
import pytest

from oracle import ssa_oracle as O


def _clustered(rng, B, H, nb, block, d, spread=3.0, within=0.2):
    return (rng.standard_normal((B, H, nb, 1, d)) * spread
            + within * rng.standard_normal((B, H, nb, block, d))).reshape(B, H, nb * block, d)


def _slack(k, levels, F, block, q):
    """min over levels and nodes of bound(q) - the largest key score below the node
    (ssa/treecode.py:141-157), per head: q (BH, d)."""
    B, H, n, d = k.shape
    BH, nb = B * H, n // block
    kf = k.reshape(BH, n, d).astype(np.float64)
    worst = math.inf
    for bh in range(BH):
        qv = q[bh].astype(np.float64)
        leafmax = (kf[bh, :nb * block] @ qv).reshape(nb, block).max(-1)
        qn = math.sqrt(qv @ qv)
        for l, lvl in enumerate(levels):
            bound = lvl["mu"][bh].astype(np.float64) @ qv + qn * lvl["R"][bh].astype(np.float64)
            span = F ** l
            nl = bound.shape[0]
            lm = np.concatenate([leafmax, np.full(nl * span - nb, -np.inf)])
            truemax = lm.reshape(nl, span).max(-1)
            worst = min(worst, float((bound - truemax).min()))
    return worst


@pytest.mark.parametrize("kind", ["random", "clustered"])
def test_tree_bound_is_admissible(kind):
    """treecode.py:141-157 (the P1 check of its main): every node's <q, mu> + |q| R bounds the
    largest key score below it; dropping R (a plausible slip) breaks it."""
    rng = np.random.default_rng(0)
    B, H, n, d, block, F = 1, 2, 4096, 32, 64, 8
    k = (rng.standard_normal((B, H, n, d)) if kind == "random"
         else _clustered(rng, B, H, n // block, block, d)).astype(np.float32)
    levels = O.tree_build(k, block, F, top_cap=1)
    assert [lv["mu"].shape[1] for lv in levels] == [64, 8, 1]
    for t in range(8):
        q = rng.standard_normal((B * H, d)).astype(np.float32)
        assert _slack(k, levels, F, block, q) >= -1e-4
    flat = [dict(lv, R=np.zeros_like(lv["R"])) for lv in levels]
    assert _slack(k, flat, F, block, rng.standard_normal((B * H, d)).astype(np.float32)) < -1e-2


def test_tree_statistics_closed_forms():
    """Leaves: a block of keys +-a e_0 has mean 0, variance a^2 on dim 0 and R = a; a constant
    block has its value as mean, variance 0, R = 0. Parent of the two: the mean of the means,
    mean(var + mu^2) - mean^2, R = max(|mu_c - mean| + R_c), lo = 0."""
    d, block, a, c = 8, 4, 3.0, 2.0
    k = np.zeros((1, 1, 2 * block, d), np.float32)
    k[0, 0, 0:2, 0], k[0, 0, 2:4, 0] = a, -a
    k[0, 0, 4:8, :] = c
    lv = O.tree_build(k, block, F=2, top_cap=1)
    assert len(lv) == 2
    leaf, top = lv
    np.testing.assert_array_equal(leaf["mu"][0, 0], np.zeros(d))
    np.testing.assert_array_equal(leaf["var"][0, 0], np.eye(d)[0] * a * a)
    assert leaf["R"][0, 0] == a
    np.testing.assert_array_equal(leaf["mu"][0, 1], np.full(d, c))
    np.testing.assert_array_equal(leaf["var"][0, 1], np.zeros(d))
    assert leaf["R"][0, 1] == 0.0
    np.testing.assert_array_equal(leaf["lo"], [0, block])
    m = np.full(d, c / 2)
    np.testing.assert_allclose(top["mu"][0, 0], m)
    np.testing.assert_allclose(top["var"][0, 0], (np.eye(d)[0] * a * a + np.full(d, c * c)) / 2 - m * m)
    half = math.sqrt(d) * c / 2  # |mu_c - mean| for either child
    np.testing.assert_allclose(top["R"][0, 0], max(half + a, half + 0.0), rtol=1e-6)
    assert top["lo"][0] == 0


@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_full_width_beam_is_the_flat_leaf_top_c(beta):
    """With W at least the node count of every level the beam keeps every node, so the descent
    returns the flat top_c of the leaf bounds by (score desc, block asc)."""
    rng = np.random.default_rng(3)
    B, H, nb, block, d, F, top_c = 1, 2, 40, 16, 16, 4, 6
    k = _clustered(rng, B, H, nb, block, d, spread=1.0, within=0.5).astype(np.float32)
    levels = O.tree_build(k, block, F, top_cap=3)
    q = rng.standard_normal((B * H, 5, d)).astype(np.float32)
    sel = O.tree_descend(levels, F, q, W=64, top_c=top_c, beta=beta)
    leaf = levels[0]
    for bh in range(B * H):
        for qi in range(5):
            q64 = q[bh, qi].astype(np.float64)
            s = (leaf["mu"][bh].astype(np.float64) @ q64
                 + math.sqrt(q64 @ q64) * leaf["R"][bh].astype(np.float64))
            if beta:
                s = s + 0.5 * beta * (leaf["var"][bh].astype(np.float64) @ (q64 * q64))
            s32 = s.astype(np.float32)
            order = sorted(range(nb), key=lambda j: (-float(s32[j]), j))[:top_c]
            assert sel[bh, qi].tolist() == order


def test_causal_mask_keeps_leaves_at_or_before_q_pos():
    rng = np.random.default_rng(5)
    B, H, nb, block, d, F = 1, 1, 64, 16, 16, 4
    k = rng.standard_normal((B, H, nb * block, d)).astype(np.float32)
    levels = O.tree_build(k, block, F, top_cap=4)
    Q = 32
    q = rng.standard_normal((1, Q, d)).astype(np.float32)
    pos = rng.integers(0, nb * block, size=(1, Q))
    sel = O.tree_descend(levels, F, q, W=8, top_c=8, q_pos=pos)
    for qi in range(Q):
        got = [j for j in sel[0, qi] if j >= 0]
        assert got and all(j * block <= pos[0, qi] for j in got)
        # as many as exist: every leaf at or before q_pos when there are fewer than top_c
        assert len(got) == min(8, pos[0, qi] // block + 1)


def test_beam_recall_climbs_to_the_flat_ceiling():
    """treecode.py:160-200 (the P2 check of its main, smaller): corrupted-cue queries; the fraction
    whose true best block lands in the selection grows with W and reaches the flat full-scan
    ceiling of the leaf bounds."""
    rng = np.random.default_rng(1)
    B, H, nb, block, d, F, top_c = 1, 2, 128, 64, 32, 8, 4
    n = nb * block
    k = _clustered(rng, B, H, nb, block, d, within=0.3).astype(np.float32)
    levels = O.tree_build(k, block, F, top_cap=8)
    kf = k.reshape(B * H, n, d).astype(np.float64)
    T = 60
    t = rng.integers(0, n, size=(B * H, T))
    q = (kf[np.arange(B * H)[:, None], t] + 0.6 * rng.standard_normal((B * H, T, d))).astype(np.float32)
    true_block = np.stack([(kf[bh] @ q[bh].T.astype(np.float64)).argmax(0) // block
                           for bh in range(B * H)])
    leaf = levels[0]
    flat = 0
    for bh in range(B * H):
        q64 = q[bh].astype(np.float64)
        s = q64 @ leaf["mu"][bh].astype(np.float64).T + np.linalg.norm(q64, axis=1)[:, None] * leaf["R"][bh]
        top = np.argsort(-s, axis=1)[:, :top_c]
        flat += int((top == true_block[bh][:, None]).any(1).sum())
    rec = {}
    for W in (1, 4, 16):
        sel = O.tree_descend(levels, F, q, W=W, top_c=top_c)
        rec[W] = int((sel == true_block[:, :, None]).any(-1).sum()) / (B * H * T)
    ceiling = flat / (B * H * T)
    assert rec[1] <= rec[4] + 1e-9 <= rec[16] + 2e-9, rec
    assert rec[16] >= ceiling - 0.02, (rec, ceiling)
    assert ceiling > 0.5
