"""GPU parity of the treecode router (ssa_tree_build / ssa_tree_descend through ssa_amd.treecode)
against the CPU oracle (oracle.ssa_oracle.tree_build / tree_descend, pinned in
tests/test_oracle_tree.py). Bars: the tree's float32 statistics within 1 ulp of the oracle's
(both sum in float64 and round once; only the summation order differs); descents equal to the
oracle's on the GPU's own tree values (every selection, every level's ties by the lower node)."""

import numpy as np
import pytest
import torch

from oracle import ssa_oracle as O
from ssa_amd import ssa_kernel as K
from ssa_amd import treecode as T
from ssa_amd import workloads as WL
from tests.test_oracle_tree import _clustered

pytestmark = pytest.mark.gpu


def ulps(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    return int(np.abs(a - b).max())


def host_levels(levels):
    return [dict(mu=lv.mu.cpu().numpy(), var=lv.var.cpu().numpy(), R=lv.R.cpu().numpy(),
                 lo=lv.lo.cpu().numpy()) for lv in levels]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("F,top_cap,nb", [(8, 8, 200), (2, 1, 37), (16, 4, 64)])
def test_tree_build_matches_oracle(cuda, dtype, F, top_cap, nb):
    rng = np.random.default_rng(11)
    B, H, block, d = 1, 3, 64, 64
    k = _clustered(rng, B, H, nb, block, d, spread=1.5, within=0.4).astype(np.float32)
    k = np.concatenate([k, rng.standard_normal((B, H, 17, d)).astype(np.float32)], axis=2)
    k = WL.round_to(k, dtype)  # a partial tail block, dropped as n // block drops it
    levels, _ = T.build_tree(WL.to_device(k, dtype, cuda), block, F, top_cap)
    ref = O.tree_build(k, block, F, top_cap)
    assert len(levels) == len(ref)
    for lv, rv in zip(host_levels(levels), ref):
        for name in ("mu", "var", "R"):
            assert lv[name].shape == rv[name].shape
            assert ulps(lv[name], rv[name]) <= 1, (name, ulps(lv[name], rv[name]))
        np.testing.assert_array_equal(lv["lo"], rv["lo"])


@pytest.mark.parametrize("d", [4, 48, 256, 512])
def test_tree_build_head_dims(cuda, d):
    """Head dims on both leaf kernels: the vector one (d / 4 or d / 8 a power of two: 4, 256,
    512) and the scalar one (48)."""
    rng = np.random.default_rng(d)
    k = WL.round_to(rng.standard_normal((1, 2, 40 * 32, d)).astype(np.float32), torch.bfloat16)
    levels, _ = T.build_tree(WL.to_device(k, torch.bfloat16, cuda), 32, 4, 2)
    ref = O.tree_build(k, 32, 4, 2)
    for lv, rv in zip(host_levels(levels), ref):
        for name in ("mu", "var", "R"):
            assert ulps(lv[name], rv[name]) <= 1, (name, ulps(lv[name], rv[name]))


def test_tree_build_strided_view_equals_contiguous(cuda):
    """k given as a transposed (B, n, H, d) -> (B, H, n, d) view builds the same tree."""
    rng = np.random.default_rng(2)
    x = torch.from_numpy(rng.standard_normal((1, 4096, 2, 64)).astype(np.float32)).to(cuda)
    a, _ = T.build_tree(x.transpose(1, 2), 128, 8, 8)
    b, _ = T.build_tree(x.transpose(1, 2).contiguous(), 128, 8, 8)
    for la, lb in zip(a, b):  # (the buffer's alignment padding is never written)
        for name in ("mu", "var", "R", "lo"):
            assert torch.equal(getattr(la, name), getattr(lb, name))


@pytest.mark.parametrize("W,F,top_c,beta,causal", [
    (1, 8, 4, 0.0, False), (4, 8, 4, 0.0, False), (16, 8, 8, 0.0, False), (16, 8, 8, 1.0, True),
    (64, 16, 64, 2.0, True), (8, 2, 3, 0.0, True), (32, 4, 16, 0.5, False)])
def test_descend_matches_oracle(cuda, W, F, top_c, beta, causal):
    rng = np.random.default_rng(7)
    B, H, nb, block, d = 1, 2, 300, 32, 64
    k = _clustered(rng, B, H, nb, block, d, spread=2.0, within=0.3).astype(np.float32)
    levels, _ = T.build_tree(torch.from_numpy(k).to(cuda), block, F, 8)
    Q = 96
    n = nb * block
    idx = rng.integers(0, n, size=(B * H, Q))
    kf = k.reshape(B * H, n, d)
    q = (kf[np.arange(B * H)[:, None], idx] + 0.5 * rng.standard_normal((B * H, Q, d))).astype(np.float32)
    q_pos = rng.integers(0, n, size=(B * H, Q)) if causal else None
    sel = T.descend_beam(levels, F, torch.from_numpy(q).to(cuda), W, top_c,
                         None if q_pos is None else torch.from_numpy(q_pos).to(cuda), beta)
    ref = O.tree_descend(host_levels(levels), F, q, W, top_c, q_pos, beta)
    got = sel.cpu().numpy()
    assert got.shape == ref.shape == (B * H, Q, min(top_c, W))
    mism = int((got != ref).any(-1).sum())
    assert mism == 0, f"{mism} of {B * H * Q} queries differ"
    if causal:
        assert ((got < 0) | (got * block <= q_pos[:, :, None])).all()


def test_descend_single_level_and_errors(cuda):
    """nb <= top_cap: the leaves are the top level, scanned whole; W above the leaf count returns
    every leaf (then -1). A tree built with another F is refused."""
    rng = np.random.default_rng(4)
    k = rng.standard_normal((1, 1, 6 * 16, 32)).astype(np.float32)
    levels, F = T.build_tree(torch.from_numpy(k).to(cuda), 16, 4, 8)
    assert len(levels) == 1
    q = rng.standard_normal((1, 3, 32)).astype(np.float32)
    sel = T.descend_beam(levels, F, torch.from_numpy(q).to(cuda), 8, 8).cpu().numpy()
    ref = O.tree_descend(host_levels(levels), F, q, 8, 8)
    np.testing.assert_array_equal(sel, ref)
    assert (sel[:, :, 6:] == -1).all() and (np.sort(sel[:, :, :6], -1) == np.arange(6)).all()
    with pytest.raises(ValueError):
        T.descend_beam(levels, 8, torch.from_numpy(q).to(cuda), 8, 8)


def test_tree_route_contract_and_attention(cuda):
    """tree_route: ascending lists of blocks <= i holding the local window, then the
    block-sparse attention over them matches the oracle's masked softmax on sampled blocks."""
    rng = np.random.default_rng(9)
    B, Hq, Hkv, nb, block, d = 1, 4, 2, 64, 64, 64
    n = nb * block
    k = _clustered(rng, B, Hkv, nb, block, d, spread=1.0, within=0.5).astype(np.float32)
    q = rng.standard_normal((B, Hq, n, d)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, n, d)).astype(np.float32)
    q, k, v = (WL.round_to(x, torch.bfloat16) for x in (q, k, v))
    qt, kt, vt = (WL.to_device(x, torch.bfloat16, cuda) for x in (q, k, v))
    kv_num, kv_idx = T.tree_route(qt, kt, block, top_c=8, local=1, W=16)
    num, idx = kv_num.cpu().numpy(), kv_idx.cpu().numpy()
    assert idx.shape == (B, Hq, nb, 8 + 2)
    for h in range(Hq):
        for i in range(nb):
            lst = idx[0, h, i, :num[0, h, i]].tolist()
            assert lst == sorted(set(lst)) and all(0 <= j <= i for j in lst)
            assert i in lst and (i == 0 or i - 1 in lst)
            assert num[0, h, i] <= min(i + 1, 10)
    out = K.sparse_attention(qt, kt, vt, kv_num, kv_idx, block)
    qb = [0, 5, nb // 2, nb - 1]
    ref = O.sparse_attention(q, k, v, num, idx, block, qblocks=qb, heads=[0, 3])
    o = out.float().cpu().numpy()
    for h in (0, 3):
        for i in qb:
            sl = slice(i * block, (i + 1) * block)
            assert np.abs(o[0, h, sl] - ref[0, h, sl]).max() < 2e-2


@pytest.mark.parametrize("tc,local,nb", [(8, 1, 40), (16, 3, 9), (1, 0, 5), (64, 2, 300)])
def test_tree_pack(cuda, tc, local, nb):
    """ssa_tree_pack (tree_route's compact lists): each row's leaves (-1 = none, duplicates
    allowed) OR blocks i - local .. i, distinct and ascending, pad 0."""
    from ssa_amd import _lib
    rng = np.random.default_rng(tc * 7 + nb)
    rows = 3 * nb
    i = np.arange(rows) % nb
    sel = rng.integers(-1, nb, size=(rows, tc))
    sel = np.where(sel > i[:, None], -1, sel).astype(np.int32)   # leaves at or before block i
    sel[::5, :2] = sel[::5, :1]                                   # a duplicated leaf
    W = tc + local + 1
    st = torch.from_numpy(sel).to(cuda)
    kv_num = torch.full((rows,), -7, device=cuda, dtype=torch.int32)
    kv_idx = torch.full((rows, W), -7, device=cuda, dtype=torch.int32)
    _lib.call("ssa_tree_pack", st.data_ptr(), rows, nb, tc, local, kv_num.data_ptr(),
              kv_idx.data_ptr(), W, _lib.stream_of(st))
    kn, ki = kv_num.cpu().numpy(), kv_idx.cpu().numpy()
    for r in range(rows):
        want = sorted({int(x) for x in sel[r] if x >= 0} |
                      {int(i[r]) - L for L in range(local + 1) if i[r] - L >= 0})
        assert kn[r] == len(want) and ki[r, :kn[r]].tolist() == want, r
        assert (ki[r, kn[r]:] == 0).all()
    with pytest.raises(_lib.SSAError):
        _lib.call("ssa_tree_pack", st.data_ptr(), rows, nb, tc, local, kv_num.data_ptr(),
                  kv_idx.data_ptr(), W - 1 if nb > local else tc, _lib.stream_of(st))
