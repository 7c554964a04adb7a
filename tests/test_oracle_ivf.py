"""CPU pinning of the IVF router oracle (oracle.ssa_oracle.ivf_*), the faiss-free restatement of
ssa/ivf_kernel.py:63-119. faiss itself is absent here, so the checks are the mathematics: the
exhaustive search reduces to brute force, hand-built known answers, planted clusters, the list
invariants, and the reference's own agreement test (ssa/tests/test_ivf_kernel.py:67-88)."""
from __future__ import annotations

import numpy as np

from oracle import ssa_oracle as O


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def clustered_keys(n, d, block, seed):
    """ssa/tests/test_ivf_kernel.py:15-26 restated with NumPy: block means drawn from
    max(4, sqrt(nb)) centres, every key = its block's centre + 0.1 N(0, 1), fp16."""
    rng = np.random.default_rng(seed)
    nb = n // block
    nc = max(4, int(nb ** 0.5))
    centers = rng.standard_normal((nc, d)).astype(np.float32)
    assign = rng.integers(0, nc, nb)
    k = np.repeat(centers[assign], block, axis=0) + 0.1 * rng.standard_normal((n, d))
    return k.astype(np.float16).astype(np.float32).reshape(1, 1, n, d)


def test_exhaustive_search_is_bruteforce_topc():
    """All lists probed and search_k = nb: the selection is the top_c of <q̄_i, μ_j> over j <= i
    (fp64 ranking, rows without near-ties), OR the own block and one predecessor."""
    nb, d, top_c = 96, 32, 6
    qb, mu = _rand((nb, d), 1), _rand((nb, d), 2)
    cent, lists = O.ivf_build(mu, 8, 5)
    got = O.ivf_search(qb, mu, cent, lists, nprobe=8, search_k=nb, top_c=top_c, local=1)
    s = qb.astype(np.float64) @ mu.astype(np.float64).T
    checked = 0
    for i in range(nb):
        order = np.argsort(-s[i, :i + 1], kind="stable")
        if i + 1 > top_c and s[i, order[top_c - 1]] - s[i, order[top_c]] < 1e-5:
            continue
        want = set(order[:top_c].tolist()) | {max(0, i - 1), i}
        assert got[i] == sorted(want), i
        checked += 1
    assert checked > nb - 5


def test_search_cut_precedes_causal_filter():
    """Known answer: faiss returns the search_k best blocks overall, THEN the future ones are
    dropped (ssa/ivf_kernel.py:82-85). Query block 1 whose two best blocks (2, 3) are both in the
    future keeps no routed block, only its local window; filtering first would pick block 0."""
    mu = np.zeros((4, 32), dtype=np.float32)
    mu[:, 0] = [1.0, 2.0, 4.0, 3.0]
    qb = np.zeros((4, 32), dtype=np.float32)
    qb[:, 0] = 1.0
    cent, lists = O.ivf_build(mu, 1, 0)
    got = O.ivf_search(qb, mu, cent, lists, nprobe=1, search_k=2, top_c=1, local=0)
    assert got[1] == [1]
    assert got[3] == [2, 3]                          # block 2 ranks first and is causal
    assert got[2] == [2]
    wider = O.ivf_search(qb, mu, cent, lists, nprobe=1, search_k=4, top_c=1, local=0)
    assert wider[1] == [1]                           # block 1 itself (score 2) is the first hit
    assert O.ivf_search(qb, mu, cent, lists, nprobe=1, search_k=4, top_c=2, local=0)[1] == [0, 1]


def test_full_budget_selects_every_causal_block():
    nb, d = 40, 64
    sel, _, _ = O.ivf_route(_rand((1, 1, nb, d), 3), _rand((1, 1, nb, d), 4), top_c=nb,
                            local=nb, nprobe=nb, search_k=nb)
    for i in range(nb):
        assert sel[0, 0, i] == list(range(i + 1))


def test_planted_clusters_recovered():
    """Well-separated directions laid out in contiguous runs of blocks: the initial centroids
    (mu[c * nb / nlist]) hit every cluster once and spherical k-means keeps the partition."""
    k, per, d = 6, 20, 32
    dirs = np.linalg.qr(np.random.default_rng(5).standard_normal((d, k)))[0].T * 3.0
    mu = (np.repeat(dirs, per, axis=0) +
          0.01 * np.random.default_rng(6).standard_normal((k * per, d))).astype(np.float32)
    cent, lists = O.ivf_build(mu, k, 10)
    assert [l.tolist() for l in lists] == [list(range(c * per, (c + 1) * per)) for c in range(k)]
    for c in range(k):
        unit = dirs[c] / np.linalg.norm(dirs[c])
        assert float(cent[c] @ unit) > 0.999


def test_lists_partition_and_assignment():
    nb, d, nlist = 200, 64, 14
    mu = _rand((nb, d), 7)
    cent, lists = O.ivf_build(mu, nlist, 10)
    allm = np.concatenate(lists)
    assert sorted(allm.tolist()) == list(range(nb))
    s = mu.astype(np.float64) @ cent.astype(np.float64).T
    for c, l in enumerate(lists):
        assert (np.diff(l) > 0).all()
        for j in l:
            assert s[j].argmax() == c or s[j].max() - s[j, c] < 1e-5
    # a centroid with members is its members' normalised mean direction (one more round of the
    # update leaves the assignment's centroids within rounding)
    for c, l in enumerate(lists):
        if len(l):
            m = mu[l].astype(np.float64).sum(0)
            assert np.allclose(cent[c], m / np.linalg.norm(m), atol=0.2)


def test_agreement_with_flat_router_on_clustered_geometry():
    """ssa/tests/test_ivf_kernel.py:67-88 restated on the oracle: IVF (nprobe 8) vs the flat
    block_route selection, mean Jaccard over rows i >= top_c at least 0.6."""
    block, top_c = 128, 8
    n = 64 * block
    nb = n // block
    q = clustered_keys(n, 64, block, 1)
    k = clustered_keys(n, 64, block, 2)
    sel, _, _ = O.ivf_route(O.qmean(q, block), O.qmean(k, block), top_c=top_c, local=1, nprobe=8)
    kv_num, kv_idx = O.route_flat(q, k, block, top_c=top_c, local=1)
    jac = []
    for i in range(top_c, nb):
        a = set(sel[0, 0, i])
        b = set(kv_idx[0, 0, i, :kv_num[0, 0, i]].tolist())
        jac.append(len(a & b) / max(1, len(a | b)))
    assert np.mean(jac) >= 0.6, np.mean(jac)


def test_planted_slip_fails_bruteforce():
    """A plausible slip -- ranking by the float64 score but with ties to the HIGHER index -- is
    caught: with duplicated block means the tie order decides the selection."""
    nb, d = 16, 32
    mu = np.repeat(_rand((8, d), 8), 2, axis=0)      # blocks 2t and 2t+1 identical
    qb = _rand((nb, d), 9)
    cent, lists = O.ivf_build(mu, 4, 3)
    got = O.ivf_search(qb, mu, cent, lists, nprobe=4, search_k=nb, top_c=1, local=0)
    for i in range(1, nb, 2):
        s = O._dot_seq(qb[i:i + 1], mu[:i + 1])[0]
        best = int(np.flatnonzero(s == s.max())[0])   # lowest index among the tied best
        assert got[i] == sorted({best, i})
