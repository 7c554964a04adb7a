"""GPU parity of the certified causal cascade (ssa_ccc_* through ssa_amd.cascade_router) against
the CPU oracle (oracle.ssa_oracle.CascadeOracle, pinned in tests/test_oracle_ccc.py).

Bar: bit-exact. Group means, outlier keys, Lloyd centroids, assignments and lists equal the
oracle's; radii within 1 ulp (an fp64 square root rounded to fp32); and streamed end to end
(flat regime, first build, incremental adds, warm rebuilds, escalation rounds, outliers), every
chunk's kv_num, kv_idx, certificate and round count equal the oracle's. Plus the reference's own
mechanics tests (ssa/tests/test_cascade_router.py) on the HIP path: full budget equals dense,
decode step equals the prefill row, causal / own / unique lists, a starved probe failing closed."""
import numpy as np
import pytest
import torch

from oracle import ssa_oracle as O
from ssa_amd import _lib
from ssa_amd import cascade_router as C
from tests.test_oracle_ccc import BLOCK, SUB, _clustered, _qkv, _random

pytestmark = pytest.mark.gpu


def dev16(x, cuda, dtype=torch.float16):
    return torch.from_numpy(np.ascontiguousarray(x)).to(cuda).to(dtype)


def ulps(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    return int(np.abs(a - b).max()) if a.size else 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [64, 96])
def test_stage_means_and_outliers(cuda, dtype, d):
    rng = np.random.default_rng(d)
    m = 64 * SUB
    x = rng.standard_normal((m, d)).astype(np.float32)
    x[777] *= 9.0
    xt = dev16(x, cuda, dtype)
    xh = xt.float().cpu().numpy()
    cc = C.CausalCascade(d, outlier_rate=0.02)
    cc.append(xt)
    mu = O.ccc_group_means(xh, SUB)
    np.testing.assert_array_equal(cc.means[:cc.n_sub].cpu().numpy(), mu)
    v, par, pos = O.ccc_outliers(xh, mu, SUB, int(0.02 * m), 0, BLOCK)
    assert cc.n_out == len(pos) and pos[0] == 777
    np.testing.assert_array_equal(cc.O[:cc.n_out].cpu().numpy(), v)
    np.testing.assert_array_equal(cc.O_parent[:cc.n_out].cpu().numpy(), par)
    np.testing.assert_array_equal(cc.O_pos[:cc.n_out].cpu().numpy(), pos)
    # block means of queries (a partial tail block dropped), through a strided view
    big = dev16(np.concatenate([x, x], 1), cuda, dtype)[:m - 5, :d]
    qb = C._group_means(big, BLOCK)
    np.testing.assert_array_equal(qb.cpu().numpy(), O.ccc_group_means(xh[:m - 5], BLOCK))


@pytest.mark.parametrize("nlist", [19, 4, 64])
def test_kmeans_and_index_build(cuda, nlist):
    """Cold and warm Lloyd rounds, the index's lists and radii, and the incremental add."""
    q, k = _clustered(160 * BLOCK, seed=3)
    X = O.ccc_group_means(k, SUB)
    n0 = 400
    cc = C.CausalCascade(64, nlist=nlist, n_hint=len(X) * SUB)
    cc.means = torch.from_numpy(X).to(cuda)
    cc.n_sub = cc.committed = n0
    cc._build_index()
    Ch = O.ccc_kmeans(X[:n0], nlist, 6)
    np.testing.assert_array_equal(cc.centroids.cpu().numpy(), Ch)
    a = O.ccc_assign(X[:n0], Ch)
    np.testing.assert_array_equal(cc.cell_of.cpu().numpy(), a)
    R = O.ccc_radii(X[:n0], Ch, a, np.zeros(nlist, np.float32))
    assert ulps(cc.Rc.cpu().numpy(), R) <= 1
    np.testing.assert_array_equal(cc._assign(cc.means[:n0]).cpu().numpy(), a)
    # incremental add: assignment of the new means, radii only rise
    cc.n_sub = len(X)
    cc.committed_at_rebuild = len(X)          # keep this add from triggering a rebuild
    cc._commit()
    a2 = O.ccc_assign(X[n0:], Ch)
    np.testing.assert_array_equal(cc.cell_of.cpu().numpy(), np.concatenate([a, a2]))
    R2 = O.ccc_radii(X[n0:], Ch, a2, R)
    assert ulps(cc.Rc.cpu().numpy(), R2) <= 1
    # warm rebuild
    cc._rebuild()
    Cw = O.ccc_kmeans(X, nlist, 6, C0=Ch)
    np.testing.assert_array_equal(cc.centroids.cpu().numpy(), Cw)


def _stream(cuda, q, k, chunk_blocks, certify, force_build=None, hint=True, **cfg):
    """The GPU cascade and the oracle side by side over the chunks; every route compared."""
    n = k.shape[0]
    nh = n if hint else None
    gpu = C.CausalCascade(64, chunk_blocks=chunk_blocks, n_hint=nh, **cfg)
    ora = O.CascadeOracle(64, chunk_blocks=chunk_blocks, n_hint=nh, **cfg)
    if force_build is not None:
        gpu.build_threshold = ora.build_threshold = force_build
    qt, kt = dev16(q, cuda), dev16(k, cuda)
    cb = chunk_blocks * BLOCK
    seen = {"rounds": 0, "cert": 0, "rows": 0, "built": False}
    for t in range(0, n, cb):
        gpu.append(kt[t:t + cb])
        ora.append(k[t:t + cb])
        kn, ki, cert, st = gpu.route(qt[t:t + cb], t, certify=certify)
        okn, okv, ocert, orounds = ora.route(q[t:t + cb], t, certify=certify)
        kn, ki = kn.cpu().numpy(), ki.cpu().numpy()
        assert gpu.committed == ora.committed and gpu.n_out == len(ora.O_pos)
        np.testing.assert_array_equal(kn, okn, err_msg=f"chunk at {t}")
        for j in range(len(kn)):
            assert ki[j, :kn[j]].tolist() == okv[j], (t, j)
            assert (ki[j, kn[j]:] == 0).all()
        if certify:
            np.testing.assert_array_equal(cert.cpu().numpy(), ocert, err_msg=f"chunk at {t}")
            np.testing.assert_array_equal(st["rounds"].cpu().numpy(), orounds)
            seen["rounds"] = max(seen["rounds"], int(orounds.max()))
            seen["cert"] += int(ocert.sum())
        seen["rows"] += len(kn)
        seen["built"] |= ora.C is not None
    if ora.C is not None:
        np.testing.assert_array_equal(gpu.centroids.cpu().numpy(), ora.C)
        assert ulps(gpu.Rc.cpu().numpy(), ora.Rc) <= 1
    return seen


def test_stream_flat_regime(cuda):
    """Flat committed scan + staged chunks + outliers, no index."""
    q, k, _ = _qkv(24 * BLOCK, seed=2)
    s = _stream(cuda, q, k, 4, True, top_c=3, local=1, outlier_rate=5e-3)
    assert not s["built"] and s["cert"] > 0


@pytest.mark.parametrize("geom,nprobe,extra", [
    ("clustered", 3, {}), ("random", 2, {}), ("random", 1, {"cert_margin": 0.05}),
    ("clustered", 3, {"retrain_every": 3}), ("random", 2, {"max_escalations": 0})])
def test_stream_index_regime(cuda, geom, nprobe, extra):
    """First build mid-stream, incremental adds, warm rebuilds, certificates and escalation."""
    n = 200 * BLOCK
    q, k = _clustered(n, seed=5) if geom == "clustered" else _random(n, seed=5)
    s = _stream(cuda, q, k, 8, True, force_build=96, top_c=6, nprobe=nprobe, **extra)
    assert s["built"]
    if geom == "random" and extra.get("max_escalations", 2):
        assert s["rounds"] >= 1


@pytest.mark.parametrize("nlist,geom", [(181, "clustered"), (150, "random")])
def test_stream_many_cells(cuda, nlist, geom):
    """More than 64 cells: the probed lists are found by threads of several waves (a missing
    workgroup barrier between writing them and reading their sizes once let a route read stale
    list ids at 1M tokens)."""
    n = 400 * BLOCK
    q, k = _clustered(n, seed=6) if geom == "clustered" else _random(n, seed=6)
    s = _stream(cuda, q, k, 16, True, force_build=512, nlist=nlist, top_c=8, nprobe=4)
    assert s["built"]


def test_stream_without_size_hint(cuda):
    """No n_hint (as the reference's own tests construct it): the sub-mean, outlier and index
    buffers grow as chunks arrive (the index is rebuilt larger with the same centroids and the
    incremental radii carried over), and nlist is fixed at the first build from the committed
    count."""
    n = 200 * BLOCK
    q, k = _clustered(n, seed=13)
    s = _stream(cuda, q, k, 8, True, force_build=96, hint=False, top_c=6, nprobe=3)
    assert s["built"]


def test_stream_long_scans(cuda):
    """More than 2048 candidates per search (several passes of the streaming top-k): a flat scan
    over 2304 committed sub-means, then a 4-list index whose probed lists hold ~3000."""
    n = 96 * 1024
    q, k, _ = _qkv(n, seed=9)
    _stream(cuda, q, k, 192, False, top_c=8, search_k=64)
    _stream(cuda, q, k, 96, True, force_build=1024, nlist=4, top_c=8, nprobe=4, search_k=256,
            max_escalations=1)


def test_stream_with_projection(cuda):
    """proj = a (d, d_r) matrix (ssa/cascade_router.py:51-61): keys and query-block means routed in
    the d_r-dimensional space. The oracle gets the projected keys and query summaries the class
    forms (the same per-chunk GEMMs), so every selection, certificate and round must agree."""
    n, d_r, cb_blocks = 64 * BLOCK, 32, 8
    q, k = _clustered(n, seed=12)
    rng = np.random.default_rng(12)
    Wp = torch.from_numpy((rng.standard_normal((64, d_r)) / 8).astype(np.float32)).to(cuda)
    gpu = C.CausalCascade(64, proj=Wp, chunk_blocks=cb_blocks, n_hint=n, top_c=6, nprobe=2)
    ora = O.CascadeOracle(d_r, chunk_blocks=cb_blocks, n_hint=n, top_c=6, nprobe=2)
    assert gpu.dr == d_r and gpu.nlist == ora.nlist
    gpu.build_threshold = ora.build_threshold = 48
    qt, kt = dev16(q, cuda), dev16(k, cuda)
    cb = cb_blocks * BLOCK
    for t in range(0, n, cb):
        gpu.append(kt[t:t + cb])
        ora.append((kt[t:t + cb].float() @ Wp).cpu().numpy())
        kn, ki, cert, st = gpu.route(qt[t:t + cb], t, certify=True)
        qr = (C._group_means(qt[t:t + cb], BLOCK) @ Wp).cpu().numpy()
        okn, okv, ocert, orounds = ora.route_rows(qr, t // BLOCK, True)
        kn, ki = kn.cpu().numpy(), ki.cpu().numpy()
        np.testing.assert_array_equal(kn, okn, err_msg=f"chunk at {t}")
        for j in range(len(kn)):
            assert ki[j, :kn[j]].tolist() == okv[j], (t, j)
        np.testing.assert_array_equal(cert.cpu().numpy(), ocert)
        np.testing.assert_array_equal(st["rounds"].cpu().numpy(), orounds)
    assert ora.C is not None


def test_ccc_full_budget_matches_dense(cuda):
    """test_cascade_router.py:42-55."""
    from ssa_amd.ssa_kernel import dense
    n = 16 * BLOCK
    nb = n // BLOCK
    q, k, v = (dev16(x, cuda).view(1, 1, n, 64) for x in _qkv(n))
    out, kv_num, kv_idx, _ = C.ccc_prefill(q, k, v, top_c=nb, local=nb, nprobe=nb,
                                           search_k=nb * 4, chunk_blocks=nb)
    assert (kv_num[0, 0].cpu() == torch.arange(1, nb + 1, dtype=torch.int32)).all()
    ref = dense(q.float(), k.float(), v.float())
    assert (out.float() - ref).abs().max().item() < 2e-2


def test_ccc_selection_causal_owns_block_unique(cuda):
    """test_cascade_router.py:58-77."""
    n = 12 * BLOCK
    nb = n // BLOCK
    q, k, v = (dev16(x, cuda).view(1, 1, n, 64) for x in _qkv(n))
    _, kv_num, kv_idx, _ = C.ccc_prefill(q, k, v, top_c=2, local=1, chunk_blocks=4)
    kn, ki = kv_num[0, 0].cpu(), kv_idx[0, 0].cpu()
    assert (kn >= 1).all() and kn.float().mean().item() < (nb + 1) / 2
    for i in range(nb):
        ids = ki[i, :int(kn[i])].tolist()
        assert max(ids) <= i and i in ids and len(set(ids)) == len(ids)


def test_ccc_decode_step_matches_prefill_row(cuda):
    """test_cascade_router.py:133-147: the last query row attended over the last query block's
    list equals the prefill output row."""
    from ssa_amd.ivf_decode import decode_attend
    n = 12 * BLOCK
    nb = n // BLOCK
    q, k, v = (dev16(x, cuda).view(1, 1, n, 64) for x in _qkv(n, seed=7))
    out, kv_num, kv_idx, _ = C.ccc_prefill(q, k, v, top_c=4, local=1, chunk_blocks=nb,
                                           search_k=nb * 4)
    blocks = kv_idx[0, 0, nb - 1, :int(kv_num[0, 0, nb - 1])].tolist()
    row = decode_attend(q[0, 0, n - 1], k[0, 0], v[0, 0], blocks, pos=n - 1, block=BLOCK)
    assert (row.float() - out[0, 0, n - 1].float()).abs().max().item() < 2e-2
    # CausalCascade.step over the same cache routes the query alone
    cc = C.CausalCascade(64, top_c=4, local=1, chunk_blocks=nb, search_k=nb * 4)
    cc.append(k[0, 0])
    got = cc.step(q[0, 0, n - 1], None, None, k[0, 0], v[0, 0], n - 1)
    ora = O.CascadeOracle(64, top_c=4, local=1, chunk_blocks=nb, search_k=nb * 4)
    ora.append(k[0, 0].float().cpu().numpy())
    sel = ora.route_rows(q[0, 0, n - 1:].float().cpu().numpy(), nb - 1)[1][0]
    want = decode_attend(q[0, 0, n - 1], k[0, 0], v[0, 0], sel, pos=n - 1, block=BLOCK)
    assert torch.equal(got, want)


def test_starved_probe_fails_closed(cuda):
    """test_cascade_router.py:150-178 on the HIP path (the oracle decides the same)."""
    d, nlist, per = 32, 8, 4
    Cm = np.eye(nlist, d, dtype=np.float32)
    rng = np.random.default_rng(0)
    X = (np.repeat(Cm, per, 0) + 0.01 * rng.standard_normal((nlist * per, d))).astype(np.float32)
    cc = C.CausalCascade(d, block=128, sub=32, top_c=8, local=1, nprobe=1, nlist=nlist,
                         max_escalations=0, search_k=16)
    cc._kmeans = lambda X, iters=6: torch.from_numpy(Cm).to(cuda)
    cc.means = torch.from_numpy(X).to(cuda)
    cc.n_sub = cc.committed = X.shape[0]
    cc._build_index()
    qc = (rng.standard_normal((BLOCK, d)) + 4 * Cm[0]).astype(np.float32)
    kv_num, kv_idx, cert, _ = cc.route(torch.from_numpy(qc).to(cuda), cc.n_sub * cc.sub,
                                       certify=True)
    nb_global = cc.n_sub * cc.sub // cc.block + 1
    assert (kv_idx >= 0).all() and (kv_idx < nb_global).all()
    assert not bool(cert[0])
    ora = O.CascadeOracle(d, top_c=8, local=1, nprobe=1, nlist=nlist, max_escalations=0,
                          search_k=16, kmeans=lambda X, iters=6: Cm)
    ora.means, ora.committed = X, X.shape[0]
    ora._build_index()
    okn, okv, ocert, _ = ora.route(qc, ora.n_sub * SUB, certify=True)
    assert kv_idx[0, :int(kv_num[0])].tolist() == okv[0] and not ocert[0]


def test_errors(cuda):
    with pytest.raises(ValueError):
        C.CausalCascade(48)
    cc = C.CausalCascade(64)
    with pytest.raises(ValueError):
        cc.append(torch.zeros(100, 64, device=cuda, dtype=torch.float16))
    with pytest.raises(RuntimeError):
        C.sub_block_means(torch.zeros(64, 64))
    x = torch.randn(4 * BLOCK, 64, device=cuda)
    means = torch.empty(16, 64, device=cuda)
    with pytest.raises(_lib.SSAError):        # outlier quota above 2048
        _lib.call("ssa_ccc_stage", x.data_ptr(), 0, 4 * BLOCK, 64, 64, SUB, means.data_ptr(),
                  4096, 0, BLOCK, None, None, None, None, 0, _lib.stream_of(x))
    kv = torch.empty(8, device=cuda, dtype=torch.int32)
    with pytest.raises(_lib.SSAError):        # routing dim not a multiple of 32
        _lib.call("ssa_ccc_route", x.data_ptr(), 1, 1, 48, None, 0, 0, 4, None, 0, 0, None, None,
                  0, 8, 1, 4, 32, 32, 4, 4, 2, 0, 0.0, kv.data_ptr(), kv.data_ptr(), 8,
                  kv.data_ptr(), kv.data_ptr(), None, 0, _lib.stream_of(x))


def test_escalation_needs_workspace(cuda):
    """With an index, certificates and escalation rounds, ssa_ccc_route keeps each round's best
    committed keys in the caller's workspace; without one it refuses the call."""
    d, nlist, per = 32, 8, 4
    Cm = np.eye(nlist, d, dtype=np.float32)
    cc = C.CausalCascade(d, block=128, sub=32, top_c=8, local=1, nprobe=1, nlist=nlist,
                         search_k=16)
    cc._kmeans = lambda X, iters=6: torch.from_numpy(Cm).to(cuda)
    cc.means = torch.from_numpy(np.repeat(Cm, per, 0)).to(cuda)
    cc.n_sub = cc.committed = nlist * per
    cc._build_index()
    qr = torch.randn(1, d, device=cuda)
    out = torch.zeros(16, device=cuda, dtype=torch.int32)
    ix = cc.index
    args = [qr.data_ptr(), 1, cc.n_sub // 4, d, cc.means.data_ptr(), cc.committed, cc.n_sub, 4,
            ix.buf.data_ptr(), ix.n_cap, ix.nlist, None, None, 0, 8, 1, 4, 16, 16, 1, 4, 2, 1,
            0.0, out.data_ptr(), out.data_ptr(), 16, out.data_ptr(), out.data_ptr()]
    with pytest.raises(_lib.SSAError):        # no workspace
        _lib.call("ssa_ccc_route", *args, None, 0, _lib.stream_of(qr))
    ws = torch.empty(32, device=cuda, dtype=torch.int64)
    with pytest.raises(_lib.SSAError):        # 1 x 8 x 32 bytes needed (16 doubled twice, cap 32)
        _lib.call("ssa_ccc_route", *args, ws.data_ptr(), 8 * 31, _lib.stream_of(qr))


def test_index_add_in_place_and_overflow(cuda):
    """Incremental adds write a list's new members after its current ones while they fit the
    capacity its last layout gave it (roundup64(2 size) + 64 slots), and lay every list out again
    when one would overflow; either way list c holds its members ascending from slot off[c] (a
    multiple of 64), their means in 64-member tiles stored transposed (d, 64)."""
    d, nlist, per = 32, 8, 4
    Cm = np.eye(nlist, d, dtype=np.float32)
    rng = np.random.default_rng(1)
    X = np.concatenate([np.repeat(Cm, per, 0),                      # the build: 4 per list
                        Cm[rng.integers(0, nlist, 40)],             # fits every capacity (128)
                        np.repeat(Cm[:1], 300, 0)])                 # overflows list 0
    X = (X + 0.01 * rng.standard_normal(X.shape)).astype(np.float32)
    cc = C.CausalCascade(d, block=128, sub=32, nlist=nlist, n_hint=4096 * 32)
    cc._kmeans = lambda X, iters=6: torch.from_numpy(Cm).to(cuda)
    cc.means = torch.from_numpy(X).to(cuda)
    cc.n_sub = cc.committed = nlist * per
    cc._build_index()

    def layout(n):
        ix = cc.index
        buf = ix.buf.cpu().numpy()
        r = lambda x: (x + 255) // 256 * 256
        mcap = 2 * ix.n_cap + 128 * nlist
        o_count = 2 * r(nlist * d * 4) + r(nlist * 4) + r(ix.n_cap * 4)
        o_off = o_count + r(nlist * 4)
        o_ids = o_off + r((nlist + 1) * 4)
        o_mu = o_ids + r(mcap * 4)
        count = buf[o_count:o_count + 4 * nlist].view(np.int32)
        off = buf[o_off:o_off + 4 * (nlist + 1)].view(np.int32)
        ids = buf[o_ids:o_ids + 4 * mcap].view(np.int32)
        mu = buf[o_mu:o_mu + 4 * mcap * d].view(np.float32)
        a = O.ccc_assign(X[:n], Cm)
        np.testing.assert_array_equal(cc.cell_of.cpu().numpy(), a)
        for c in range(nlist):
            want = np.flatnonzero(a == c)
            assert count[c] == len(want) and off[c] % 64 == 0 and off[c + 1] - off[c] >= len(want)
            np.testing.assert_array_equal(ids[off[c]:off[c] + len(want)], want)
            for k, j in enumerate(want):
                t0 = off[c] + k - k % 64
                np.testing.assert_array_equal(mu[t0 * d + np.arange(d) * 64 + k % 64], X[j])
        return off[1:] - off[:-1]

    caps = [layout(nlist * per)]
    for n in (nlist * per + 40, len(X)):
        cc.n_sub = n
        cc.committed_at_rebuild = n               # keep the adds from triggering a rebuild
        cc._commit()
        caps.append(layout(n))
    assert (caps[1] == caps[0]).all()             # the first add wrote in place
    assert caps[2][0] > caps[0][0]                # the second laid the lists out again
