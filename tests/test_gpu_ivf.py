"""GPU parity of the IVF router (ssa_ivf_build / ssa_ivf_route through ssa_amd.ivf_kernel).

Bar: the index (centroids, list sizes, offsets, member ids) and every routed selection are
bit-exact against the oracle (oracle.ssa_oracle.ivf_*) run on the same block means; plus the
reference's own IVF tests (ssa/tests/test_ivf_kernel.py:29-88) restated on the HIP path."""
import numpy as np
import pytest
import torch

from oracle import ssa_oracle as O
from ssa_amd import _lib
from ssa_amd import ivf_kernel as I
from ssa_amd import ssa_kernel as K
from tests.test_oracle_ivf import clustered_keys

pytestmark = pytest.mark.gpu


def np_of(t):
    return t.detach().cpu().numpy()


def _means(BH, nb, d, seed, cuda, clustered=False):
    rng = np.random.default_rng(seed)
    if clustered:
        nc = max(4, int(nb ** 0.5))
        c = rng.standard_normal((nc, d)).astype(np.float32)
        x = c[rng.integers(0, nc, (BH, nb))] + 0.2 * rng.standard_normal((BH, nb, d))
    else:
        x = rng.standard_normal((BH, nb, d))
    return torch.tensor(x.astype(np.float32), device=cuda)


BUILD_CASES = [  # (BH, nb, d, nlist, niter)
    (2, 300, 64, None, 10),
    (1, 64, 32, 8, 0),
    (3, 1000, 128, 31, 10),
    (1, 40, 64, 40, 4),
    (2, 513, 256, 5, 6),
    (3, 1, 64, 1, 10),                   # one block per head
]


@pytest.mark.parametrize("case", BUILD_CASES, ids=[str(c) for c in BUILD_CASES])
def test_ivf_build_matches_oracle(cuda, case):
    BH, nb, d, nlist, niter = case
    mu = _means(BH, nb, d, 11 + nb, cuda, clustered=BH != 3)
    index = I.build_ivf(mu, nlist, niter=niter)
    torch.cuda.synchronize()
    nl = index.nlist
    cent, sizes, offs, ids = (np_of(index.centroids), np_of(index.list_sizes),
                              np_of(index.list_offsets), np_of(index.list_ids))
    m = np_of(mu)
    for h in range(BH):
        ocent, olists = O.ivf_build(m[h], nl, niter)
        assert np.array_equal(cent[h], ocent), h
        assert sizes[h].tolist() == [len(x) for x in olists]
        assert offs[h].tolist() == np.concatenate([[0], np.cumsum([len(x) for x in olists])]).tolist()
        assert ids[h].tolist() == np.concatenate(olists).tolist()


ROUTE_CASES = [  # (nb, d, nlist, nprobe, search_k, top_c, local)
    (300, 64, None, 1, 16, 8, 1),
    (300, 64, None, 4, None, 4, 2),
    (64, 32, 8, 8, 64, 64, 64),          # exhaustive: every causal block
    (200, 64, 12, 3, 40, 0, 1),          # top_c = 0: the local window only
    (257, 128, 16, 5, 1024, 300, 3),     # search_k above nb, top_c above search_k
    (4096, 64, 8, 8, 64, 16, 1),         # 4096 candidates: two passes through LDS
    (1, 64, 1, 4, 8, 8, 1),              # one block: the own block only
    (5, 32, 4, 2, 1, 1, 0),              # search_k 1, no local window
]


@pytest.mark.parametrize("case", ROUTE_CASES, ids=[str(c) for c in ROUTE_CASES])
def test_ivf_route_matches_oracle(cuda, case):
    nb, d, nlist, nprobe, search_k, top_c, local = case
    BH = 2 if nb < 1000 else 1
    mu = _means(BH, nb, d, 3 + nb, cuda, clustered=True)
    qb = _means(BH, nb, d, 5 + nb, cuda, clustered=True)
    index = I.build_ivf(mu, nlist, nprobe=nprobe)
    sk = min(2 * top_c, nb) if search_k is None else search_k
    kv_num, kv_idx = I.search(index, qb, top_c, local, nprobe, sk)
    torch.cuda.synchronize()
    kn, ki = np_of(kv_num), np_of(kv_idx)
    m, q = np_of(mu), np_of(qb)
    W = min(top_c + local + 1, nb)
    assert ki.shape == (BH, nb, W)
    for h in range(BH):
        cent, lists = O.ivf_build(m[h], index.nlist, 10)
        want = O.ivf_search(q[h], m[h], cent, lists, nprobe, sk, top_c, local)
        for i in range(nb):
            assert kn[h, i] == len(want[i]), (h, i)
            assert ki[h, i, :kn[h, i]].tolist() == want[i], (h, i)
            assert (ki[h, i, kn[h, i]:] == 0).all()


def test_ivf_grouped_query_heads_match_oracle(cuda):
    """Hq = 7 * Hkv: each key head's index serves its 7 query heads (query head h -> index head
    h // 7), every selection equal to the oracle search of that head's index."""
    B, Hkv, G, nb, d = 1, 2, 7, 300, 64
    mu = _means(B * Hkv, nb, d, 31, cuda, clustered=True)
    qb = _means(B * Hkv * G, nb, d, 32, cuda, clustered=True)
    index = I.build_ivf(mu, None, 4)
    kv_num, kv_idx = I.search(index, qb, 8, 1, 4, 16)
    torch.cuda.synchronize()
    assert kv_num.shape == (B * Hkv * G, nb)
    kn, ki, m, q = np_of(kv_num), np_of(kv_idx), np_of(mu), np_of(qb)
    for hk in range(B * Hkv):
        cent, lists = O.ivf_build(m[hk], index.nlist, 10)
        for g in range(G):
            h = hk * G + g
            want = O.ivf_search(q[h], m[hk], cent, lists, 4, 16, 8, 1)
            for i in range(nb):
                assert ki[h, i, :kn[h, i]].tolist() == want[i], (h, i)
    # the same through ivf_route on (B, Hq, n, d) / (B, Hkv, n, d) tensors
    n = 8 * K.BLOCK
    qt = torch.randn(1, 14, n, 64, device=cuda, dtype=torch.bfloat16)
    kt = torch.randn(1, 2, n, 64, device=cuda, dtype=torch.bfloat16)
    kn2, ki2 = I.ivf_route(qt, kt, top_c=2, local=1)
    assert kn2.shape == (1, 14, 8) and (kn2 >= 1).all()
    # full budget with grouped heads: every causal block, i.e. dense causal attention over the
    # key head of each query head
    vt = torch.randn_like(kt)
    out = I.ssa_flex_ivf(qt, kt, vt, top_c=8, local=8, nprobe=8, search_k=8)
    ref = K.dense(qt, kt.repeat_interleave(7, 1).contiguous(), vt.repeat_interleave(7, 1).contiguous())
    assert torch.allclose(out.float(), ref.float(), atol=2e-2)


def test_ivf_full_budget_matches_dense(cuda):
    """ssa/tests/test_ivf_kernel.py:29-42: exhaustive IVF (every causal block selectable) equals
    dense causal attention."""
    torch.manual_seed(0)
    n = 16 * K.BLOCK
    nb = n // K.BLOCK
    q = torch.randn(1, 1, n, 64, device=cuda, dtype=torch.float16)
    k, v = torch.randn_like(q), torch.randn_like(q)
    out_dense = K.dense(q, k, v)
    out_ivf = I.ssa_flex_ivf(q, k, v, top_c=nb, local=nb, nprobe=nb, search_k=nb)
    assert torch.allclose(out_ivf.float(), out_dense.float(), atol=2e-2)


def test_ivf_selection_is_causal_and_owns_its_block(cuda):
    """ssa/tests/test_ivf_kernel.py:45-64."""
    torch.manual_seed(0)
    n = 8 * K.BLOCK
    nb = n // K.BLOCK
    q = torch.randn(1, 1, n, 64, device=cuda, dtype=torch.float16)
    k = torch.randn_like(q)
    kv_num, kv_idx = I.ivf_route(q, k, top_c=2, local=1)
    assert (kv_num >= 1).all()
    assert kv_num.float().mean().item() < (nb + 1) / 2
    for i in range(nb):
        kn = int(kv_num[0, 0, i])
        ids = kv_idx[0, 0, i, :kn]
        assert (ids <= i).all()
        assert i in ids.tolist()
        assert len(set(ids.tolist())) == kn


def test_ivf_agreement_with_flat_router(cuda):
    """ssa/tests/test_ivf_kernel.py:67-88: on clustered geometry the IVF selection overlaps the
    flat block_route selection with mean Jaccard >= 0.6 (both on the HIP path)."""
    block, top_c = K.BLOCK, 8
    n = 64 * block
    nb = n // block
    q = torch.tensor(clustered_keys(n, 64, block, 1), device=cuda).half()
    k = torch.tensor(clustered_keys(n, 64, block, 2), device=cuda).half()
    kv_num, kv_idx = I.ivf_route(q, k, top_c=top_c, local=1, nprobe=8)
    _, _, sel = K.block_route(q, k, top_c=top_c, local=1)
    inter, rows = 0.0, 0
    for i in range(top_c, nb):
        a = set(kv_idx[0, 0, i, :int(kv_num[0, 0, i])].tolist())
        b = set(sel[0, 0, i].nonzero().flatten().tolist())
        inter += len(a & b) / max(1, len(a | b))
        rows += 1
    assert inter / rows >= 0.6, inter / rows


def test_ivf_block_means_match_summary(cuda):
    """block_means drops a partial tail block and equals the q̄ summary of the full blocks."""
    x = torch.randn(2, 3, 1000, 64, device=cuda, dtype=torch.bfloat16)
    bm = I.block_means(x, 128)
    assert bm.shape == (2, 3, 7, 64)
    assert torch.equal(bm, K.block_summary(x[:, :, :896].contiguous(), 128, "qmean"))
    assert torch.equal(I.block_means(x[0, 0], 128), bm[0, 0])


def test_ivf_route_rejects_oversized_search(cuda):
    mu = _means(1, 4096, 64, 1, cuda)
    index = I.build_ivf(mu)
    with pytest.raises(_lib.SSAError, match="exceeds 1024"):
        I.search(index, mu, top_c=8, local=1, search_k=2048)


def test_ivf_c5_scale_properties_and_sampled_rows(cuda):
    """The C5 router shape (49,152 key blocks, d 64, nlist 221, nprobe 4, search_k 128, top_c 64,
    local 1): every list and every row checked for the contract's invariants on the device, and
    sampled members / rows bit-exact against the oracle's assignment and search run on the
    device's own centroids and lists."""
    nb, d, top_c, local, nprobe, sk = 49152, 64, 64, 1, 4, 128
    mu = _means(1, nb, d, 21, cuda, clustered=True)
    qb = _means(1, nb, d, 22, cuda, clustered=True)
    index = I.build_ivf(mu, None, nprobe)
    kv_num, kv_idx = I.search(index, qb, top_c, local, nprobe, sk)
    torch.cuda.synchronize()
    nl = index.nlist
    assert nl == 221
    sizes, offs, ids = index.list_sizes[0], index.list_offsets[0], index.list_ids[0]
    # the lists partition the blocks, each ascending
    assert int(sizes.sum()) == nb and int(offs[-1]) == nb
    assert torch.equal(torch.sort(ids.long()).values, torch.arange(nb, device=cuda))
    lid = torch.repeat_interleave(torch.arange(nl, device=cuda), sizes.long())
    step = ids[1:].long() - ids[:-1].long()
    assert bool(((step > 0) | (lid[1:] != lid[:-1])).all())
    # every row: own block kept, causal, ascending and unique, padded with 0
    W = kv_idx.shape[-1]
    kn, ki = kv_num[0].long(), kv_idx[0].long()
    rows = torch.arange(nb, device=cuda)
    pos = torch.arange(W, device=cuda)[None, :]
    live = pos < kn[:, None]
    assert bool((kn >= 1).all()) and bool((kn <= W).all())
    assert bool(((ki <= rows[:, None]) | ~live).all())
    assert bool(((ki == rows[:, None]) & live).any(1).all())
    inc = (ki[:, 1:] > ki[:, :-1]) | ~live[:, 1:]
    assert bool(inc.all())
    assert bool(((ki == 0) | live).all())
    # sampled members at their argmax centroid (oracle keys on the device centroids)
    cent = np_of(index.centroids[0])
    m, q = np_of(mu[0]), np_of(qb[0])
    ids_h, offs_h = np_of(ids), np_of(offs)
    member_list = np.repeat(np.arange(nl), np_of(sizes))
    rng = np.random.default_rng(5)
    pick = rng.choice(nb, 256, replace=False)
    keys = O.ivf_keys(O._dot_seq(m[ids_h[pick]], cent), np.arange(nl)[None, :])
    assert (keys.argmax(1) == member_list[pick]).all()
    # sampled rows against the oracle's search over the device index
    lists = [ids_h[offs_h[c]:offs_h[c + 1]].astype(np.int64) for c in range(nl)]
    kn_h, ki_h = np_of(kv_num[0]), np_of(kv_idx[0])
    for i in list(rng.choice(nb, 24, replace=False)) + [0, 1, 65, nb - 1]:
        ck = O.ivf_keys(O._dot_seq(q[i:i + 1], cent)[0], np.arange(nl))
        probes = np.argsort(ck)[::-1][:nprobe]
        cand = np.concatenate([lists[c] for c in probes])
        fine = O._dot_seq(q[i:i + 1], m[cand])[0]
        top = cand[np.argsort(O.ivf_keys(fine, cand))[::-1][:sk]]
        hits = top[top <= i][:top_c]
        want = sorted(set(hits.tolist()) | set(range(max(0, i - local), i + 1)))
        assert ki_h[i, :kn_h[i]].tolist() == want, i
