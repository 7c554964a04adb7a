"""CPU pins of the cascade oracle (oracle.ssa_oracle.CascadeOracle and its helpers), the
restatement of ssa/cascade_router.py. faiss (the reference's index) is absent and the reference
holds no fixtures for this module; its own tests (ssa/tests/test_cascade_router.py,
ssa/tests/test_ccc_certificates.py) are restated here on the oracle: exhaustive selection equals
the brute-force sub-block max-pool, chunking invariance, causal / own-block / unique lists,
certificate soundness against the exact top-k of the routing metric (with a built index, on
clustered and random keys), admissible and exact radii, monotone escalation, the outlier channel
catching a hidden norm spike, and a starved probe failing closed. Closed forms pin the group
means, the Lloyd update and the outlier order."""
import numpy as np
import pytest

from oracle import ssa_oracle as O

BLOCK, SUB = 128, 32


def _qkv(n, d=64, seed=0):
    rng = np.random.default_rng(seed)
    f = lambda: rng.standard_normal((n, d)).astype(np.float16).astype(np.float32)
    return f(), f(), f()


def _clustered(n, d=64, seed=0, spread=0.1):
    """ssa/tests/test_ccc_certificates.py:15-32: keys around sqrt(n/32) centres per 32-key
    sub-block, query blocks around random centres."""
    rng = np.random.default_rng(seed)
    nb4 = n // SUB
    nc = max(8, int(nb4 ** 0.5))
    centers = rng.standard_normal((nc, d))
    k = np.repeat(centers[rng.integers(0, nc, nb4)], SUB, 0) + spread * rng.standard_normal((n, d))
    nbq = n // BLOCK
    q = np.repeat(centers[rng.integers(0, nc, nbq)], BLOCK, 0) + 0.2 * rng.standard_normal((n, d))
    return q.astype(np.float16).astype(np.float32), k.astype(np.float16).astype(np.float32)


def _random(n, d=64, seed=0):
    q, k, _ = _qkv(n, d, seed)
    return q, k


def _bruteforce(q, k, top_c, local, sub=SUB):
    """test_cascade_router.py:21-39 in float64: block score = max over sub-blocks <q_bar, mu_sub>,
    strictly-past top_c, OR the own block and `local` predecessors."""
    n, d = q.shape
    nb, spb = n // BLOCK, BLOCK // sub
    qb = q.astype(np.float64).reshape(nb, BLOCK, d).mean(1)
    mus = k.astype(np.float64).reshape(nb * spb, sub, d).mean(1)
    s = (qb @ mus.T).reshape(nb, nb, spb).max(-1)
    out = []
    for i in range(nb):
        past = np.arange(i)
        top = past[np.argsort(-s[i, :i], kind="stable")[:top_c]]
        out.append(set(top.tolist()) | {j for j in range(i - local, i + 1) if j >= 0})
    return out


def test_group_means_and_outliers_closed_form():
    """Group means of hand-built rows; the outlier order is the squared distance to the own
    group mean, ties to the lower row, with parents and positions offset by the chunk base."""
    x = np.zeros((8, 32), np.float32)
    x[:4, 0] = [1, 2, 3, 6]          # group 0 mean 3: distances^2 4, 1, 0, 9
    x[4:, 1] = [5, 5, 5, 5]          # group 1 constant: all 0
    mu = O.ccc_group_means(x, 4)
    np.testing.assert_array_equal(mu[0], np.eye(32)[0] * 3)
    np.testing.assert_array_equal(mu[1], np.eye(32)[1] * 5)
    v, par, pos = O.ccc_outliers(x, mu, 4, 3, base=256, block=128)
    assert pos.tolist() == [259, 256, 257] and par.tolist() == [2, 2, 2]
    np.testing.assert_array_equal(v[0], x[3])
    v, par, pos = O.ccc_outliers(x, mu, 4, 6, base=0, block=2)
    assert pos.tolist() == [3, 0, 1, 2, 4, 5]          # zero distances: lower rows first
    assert par.tolist() == [1, 0, 0, 1, 2, 2]


def test_kmeans_closed_form():
    """Two tight, well-separated clusters: a cold start from rows 0 and n/2 converges in one
    round to the exact cluster means; a warm start keeps them; lists and radii follow."""
    rng = np.random.default_rng(0)
    a = (np.eye(32)[0] * 10 + 0.01 * rng.standard_normal((6, 32))).astype(np.float32)
    b = (np.eye(32)[1] * 10 + 0.01 * rng.standard_normal((6, 32))).astype(np.float32)
    X = np.concatenate([a, b])
    C = O.ccc_kmeans(X, 2, iters=3)
    np.testing.assert_allclose(C[0], a.astype(np.float64).mean(0), rtol=1e-6)
    np.testing.assert_allclose(C[1], b.astype(np.float64).mean(0), rtol=1e-6)
    np.testing.assert_array_equal(O.ccc_kmeans(X, 2, iters=2, C0=C), C)
    asg = O.ccc_assign(X, C)
    assert asg.tolist() == [0] * 6 + [1] * 6
    R = O.ccc_radii(X, C, asg, np.zeros(2, np.float32))
    want = [np.linalg.norm(a - C[0], axis=1).max(), np.linalg.norm(b - C[1], axis=1).max()]
    np.testing.assert_allclose(R, want, rtol=1e-6)


def test_exhaustive_equals_bruteforce():
    """test_cascade_router.py:80-98: one chunk, every sub-mean staged, search_k over all of
    them, no outliers -> the brute-force sub-block max-pool selection."""
    n, top_c, local = 24 * BLOCK, 3, 1
    nb = n // BLOCK
    q, k, _ = _qkv(n, seed=3)
    cc = O.CascadeOracle(64, top_c=top_c, local=local, chunk_blocks=nb, search_k=nb * 4,
                         outlier_cap=0)
    cc.append(k)
    kn, kv, _, _ = cc.route(q, 0, search_k=nb * 4)
    ref = _bruteforce(q, k, top_c, local)
    for i in range(nb):
        assert set(kv[i]) == ref[i], (i, kv[i], sorted(ref[i]))
        assert kn[i] == len(kv[i])


def test_chunking_invariance():
    """test_cascade_router.py:101-130: the same keys appended as one chunk or as 2-block chunks
    (flat committed scan + staged) give identical selections."""
    n, top_c = 16 * BLOCK, 4
    nb = n // BLOCK
    sk = nb * (BLOCK // SUB)
    q, k, _ = _qkv(n, seed=5)

    def run(chunk_blocks):
        cc = O.CascadeOracle(64, top_c=top_c, local=1, chunk_blocks=chunk_blocks, search_k=sk,
                             outlier_cap=0)
        out = []
        cb = chunk_blocks * BLOCK
        for t in range(0, n, cb):
            cc.append(k[t:t + cb])
            out += cc.route(q[t:t + cb], t, search_k=sk)[1]
        return out

    assert run(nb) == run(2)


def test_selection_causal_owns_block_unique():
    """test_cascade_router.py:58-77."""
    n = 12 * BLOCK
    nb = n // BLOCK
    q, k, _ = _qkv(n)
    cc = O.CascadeOracle(64, top_c=2, local=1, chunk_blocks=4, n_hint=n)
    kv = []
    for t in range(0, n, 4 * BLOCK):
        cc.append(k[t:t + 4 * BLOCK])
        kv += cc.route(q[t:t + 4 * BLOCK], t)[1]
    assert np.mean([len(x) for x in kv]) < (nb + 1) / 2
    for i, ids in enumerate(kv):
        assert ids and max(ids) <= i and i in ids and len(set(ids)) == len(ids)


def _build_cascade(k, q, top_c=6, local=1, nprobe=3, chunk_blocks=8, force_build=96, **kw):
    """test_ccc_certificates.py:40-54: append and route chunk by chunk with a small build
    threshold so that the index builds; returns the cascade ready for the last chunk."""
    n = k.shape[0]
    cc = O.CascadeOracle(64, top_c=top_c, local=local, nprobe=nprobe, chunk_blocks=chunk_blocks,
                         n_hint=n, **kw)
    cc.build_threshold = force_build
    cb = chunk_blocks * BLOCK
    chunks = list(range(0, n, cb))
    for t in chunks[:-1]:
        cc.append(k[t:t + cb])
        cc.route(q[t:t + cb], t)
    return cc, chunks[-1]


def _exact_topc(cc, qr, qb_start):
    """test_ccc_certificates.py:57-77: the exact top-k routing blocks of each query block over
    every past sub-mean (committed and staged), strictly before the query block."""
    s = O._dot_seq(qr, cc.means).astype(np.float64)
    par = np.arange(cc.n_sub) // cc.spb
    out = []
    for j in range(qr.shape[0]):
        qblk = qb_start + j
        blk = np.full(par.max() + 1, -np.inf)
        np.maximum.at(blk, par[par < qblk], s[j][par < qblk])
        order = np.argsort(-blk, kind="stable")[:min(cc.top_c, qblk)]
        out.append({int(b) for b in order if blk[b] > -np.inf})
    return out


@pytest.mark.parametrize("geom", ["clustered", "random"])
def test_certificate_soundness(geom):
    """test_ccc_certificates.py:80-101: every certified query block's list holds the exact top-k
    routing blocks (zero violations), with a real index; some rows certify."""
    n = 96 * BLOCK
    q, k = _clustered(n, seed=1) if geom == "clustered" else _random(n, seed=1)
    cc, last = _build_cascade(k, q)
    assert cc.C is not None, "the index must be built"
    cc.append(k[last:])
    kn, kv, cert, _ = cc.route(q[last:], last, certify=True)
    qr = O.ccc_group_means(q[last:], BLOCK)
    exact = _exact_topc(cc, qr, last // BLOCK)
    viol = sum(1 for j in range(len(exact)) if cert[j] and not exact[j] <= set(kv[j]))
    assert viol == 0, f"{geom}: {viol} certified rows missed a top-k block"
    if geom == "clustered":
        assert cert.any()


def test_certificate_without_radii_is_unsound():
    """A plausible slip: bounding unprobed cells by <q, c> alone (radii dropped) certifies rows
    whose list misses an exact top-k block, on the clustered geometry."""
    n = 96 * BLOCK
    viol = 0
    for seed in range(1, 5):
        q, k = _clustered(n, seed=seed)
        cc, last = _build_cascade(k, q, nprobe=1, max_escalations=0)
        cc.append(k[last:])
        cc._commit()
        cc.Rc = np.zeros_like(cc.Rc)
        _, kv, cert, _ = cc.route(q[last:], last, certify=True)
        exact = _exact_topc(cc, O.ccc_group_means(q[last:], BLOCK), last // BLOCK)
        viol += sum(1 for j in range(len(exact)) if cert[j] and not exact[j] <= set(kv[j]))
    assert viol > 0


def test_radius_admissible():
    """test_ccc_certificates.py:104-117: incremental radii bound every member's distance."""
    n = 200 * BLOCK
    q, k = _clustered(n, seed=2)
    cc, last = _build_cascade(k, q, chunk_blocks=8)
    cc.append(k[last:])
    cc._commit()
    X = cc.means[:cc.committed]
    a = O.ccc_assign(X, cc.C)
    true_R = O.ccc_radii(X, cc.C, a, np.zeros(cc.nlist, np.float32))
    assert (cc.Rc + 1e-4 >= true_R).all()
    np.testing.assert_array_equal(a, cc.assign)


@pytest.mark.parametrize("geom", ["clustered", "random"])
def test_escalation_monotone(geom):
    """test_ccc_certificates.py:120-132: more escalation rounds never shrink the certified set;
    on random keys (where two probed lists rarely certify) the escalated rounds certify more."""
    n = 96 * BLOCK
    q, k = _clustered(n, seed=4) if geom == "clustered" else _random(n, seed=4)
    rates = []
    for me in (0, 1, 2):
        cc, last = _build_cascade(k, q, nprobe=2, max_escalations=me)
        cc.append(k[last:])
        rates.append(float(cc.route(q[last:], last, certify=True)[2].mean()))
    assert rates[0] <= rates[1] + 1e-6 <= rates[2] + 1e-6, rates
    if geom == "random":
        assert rates[2] > rates[0], rates


def test_outlier_catches_norm_spike():
    """test_ccc_certificates.py:135-160: one hidden high-norm key (12 u) in block 5, the last
    query block pointing at u: at top_c 2 the sub-block routing alone mostly misses block 5 (its
    sub-mean carries 12 u / 32 among 252 noisy sub-means), the outlier channel always catches it."""
    n = 64 * BLOCK
    missed = 0
    for seed in range(7, 18):
        rng = np.random.default_rng(seed)
        q = rng.standard_normal((n, 64)).astype(np.float16).astype(np.float32)
        k = rng.standard_normal((n, 64)).astype(np.float16).astype(np.float32)
        u = rng.standard_normal(64)
        u = (u / np.linalg.norm(u)).astype(np.float16).astype(np.float32)
        q[n - BLOCK:] = u
        k[5 * BLOCK + 17] = (12.0 * u).astype(np.float16).astype(np.float32)

        def selects(cap):
            cc = O.CascadeOracle(64, top_c=2, local=0, chunk_blocks=n // BLOCK, outlier_cap=cap,
                                 search_k=64)
            cc.append(k)
            return 5 in cc.route(q, 0, search_k=64)[1][-1]

        missed += not selects(0)
        assert selects(4), seed
    assert missed >= 8, missed


def test_starved_probe_fails_closed():
    """test_cascade_router.py:150-178: fixed one-hot centroids, 4 members per cell, nprobe 1,
    search_k 16: the search returns fewer than search_k members (its last score reported as
    -inf), the lists hold only real past blocks and the certificate fails (budget not full)."""
    d, nlist, per = 32, 8, 4
    C = np.eye(nlist, d, dtype=np.float32)
    rng = np.random.default_rng(0)
    X = (np.repeat(C, per, 0) + 0.01 * rng.standard_normal((nlist * per, d))).astype(np.float32)
    cc = O.CascadeOracle(d, top_c=8, local=1, nprobe=1, nlist=nlist, max_escalations=0,
                         search_k=16, kmeans=lambda X, iters=6: C)
    cc.means, cc.committed = X, X.shape[0]
    cc._build_index()
    assert [len(m) for m in cc.lists()] == [per] * nlist
    qc = (rng.standard_normal((BLOCK, d)) + 4 * C[0]).astype(np.float32)
    kn, kv, cert, _ = cc.route(qc, cc.n_sub * SUB, certify=True)
    nb_global = cc.n_sub * SUB // BLOCK + 1
    assert all(0 <= b < nb_global for b in kv[0])
    assert not cert[0]


def test_rebuild_preserves_index():
    """test_ccc_certificates.py:163-177: a warm rebuild keeps every committed mean in the lists
    and makes the radii exact."""
    n = 400 * BLOCK
    q, k = _clustered(n, seed=8)
    cc = _build_cascade(k, q, chunk_blocks=8)[0]
    before = cc.committed
    cc._build_index()
    assert sum(len(m) for m in cc.lists()) == before
    X = cc.means[:cc.committed]
    a = O.ccc_assign(X, cc.C)
    np.testing.assert_array_equal(O.ccc_radii(X, cc.C, a, np.zeros(cc.nlist, np.float32)), cc.Rc)
