"""CPU tests pinning the oracle (oracle/ssa_oracle.py) before it is trusted as the checker.

* against the reference's own outputs (tests/golden/, written by tests/golden/make_golden.py
  from the reference run in float32/float64): selections of block_route_budget / block_route /
  _selection_mask, the FlexAttention output of ssa_flex, the analytic attention path;
* against mathematics: closed-form block statistics, brute-force ranking on tiny rows, full
  budget == dense causal softmax, the needle known-answer test, the reference's invariants.
"""
import math
from types import SimpleNamespace

import numpy as np
import pytest

from oracle import ssa_oracle as O
from ssa_amd import workloads as WL
from tests import golden_util as GU

ROUTE_CASES = {
    # fixture: (config, variant, mode, kwargs)
    "c1_budget": ("C1", "segmented", "budget", dict(top_c=8, local=1, beta=2.0)),
    "c1_frac": ("C1", "segmented", "budget", dict(budget_frac=0.25, local=1, beta=2.0)),
    "c1_flat": ("C1", "segmented", "flat", dict(top_c=8, local=1)),
    "c2_budget": ("C2", "segmented", "budget", dict(top_c=32, local=2, beta=2.0)),
    "c2_edgeworth": ("C2", "segmented", "budget", dict(top_c=32, local=2, beta=2.0, edgeworth=True)),
    "c3_budget_seg": ("C3", "segmented", "budget", dict(top_c=64, local=2, beta=2.0)),
    "c3_budget_lit": ("C3", "literal", "budget", dict(top_c=64, local=2, beta=2.0)),
    "c1_sub16": ("C1", "segmented", "budget", dict(top_c=8, local=1, beta=2.0, sub=16)),
    "c2_sub16": ("C2", "segmented", "budget", dict(top_c=32, local=2, beta=2.0, sub=16)),
    "c1_proj": ("C1", "segmented", "budget", dict(top_c=8, local=1, proj_seed=31)),
    "c2_proj_pair": ("C2", "segmented", "budget", dict(top_c=32, local=2, proj_pair_seed=41)),
}


def resolve_kw(cfg, kw, pair_as="tuple"):
    """Case kwargs -> call kwargs: projection seeds become the seeded matrices (a (W_q, W_k)
    tuple for the oracle, an object with W_q / W_k attributes like the reference accepts)."""
    kw = dict(kw)
    if "proj_seed" in kw:
        kw["proj"] = WL.proj_matrix(kw.pop("proj_seed"), cfg.d)
    if "proj_pair_seed" in kw:
        s0 = kw.pop("proj_pair_seed")
        wq, wk = WL.proj_matrix(s0, cfg.d), WL.proj_matrix(s0 + 1, cfg.d)
        kw["proj"] = (wq, wk) if pair_as == "tuple" else SimpleNamespace(W_q=wq, W_k=wk)
    return kw


def oracle_route(p, mode, kw):
    cfg = p["cfg"]
    kw = resolve_kw(cfg, kw)
    if mode == "flat":
        return O.route_flat(p["q"], p["k"], cfg.block, **kw)
    return O.route_budget(p["q"], p["k"], cfg.block, **kw)


def certificate_inputs(p, mode, kw):
    cfg = p["cfg"]
    qb = O.qmean(p["q"], cfg.block)
    if mode == "flat":
        mu, var, _ = O.block_stats(p["k"], cfg.block, "unbiased")
        return O.exact_scores64(qb, mu, var, 0.5)
    kw = resolve_kw(cfg, kw)
    sub = kw.get("sub") or cfg.block
    mu, var, m3 = O.block_stats(p["k"], sub, "pop")
    if kw.get("proj") is not None:  # exact score of the unrounded projections
        wq, wk = kw["proj"] if isinstance(kw["proj"], tuple) else (kw["proj"], kw["proj"])
        G = cfg.Hq // cfg.Hkv
        kh = np.arange(cfg.Hq) // G
        qp, mp = qb.astype(np.float64) @ wq, (mu.astype(np.float64) @ wk)[:, kh]
        qa, ma = np.abs(qb.astype(np.float64)) @ np.abs(wq), (np.abs(mu.astype(np.float64)) @ np.abs(wk))[:, kh]
        r64 = np.einsum("bhid,bhcd->bhic", qp, mp)
        mag = np.einsum("bhid,bhcd->bhic", qa, ma)
    else:
        beta = kw.get("beta", 2.0)
        r64, mag = O.exact_scores64(qb, mu, var, 0.5 * beta, m3 if kw.get("edgeworth") else None,
                                    beta ** 2 / 6.0)
    pool = cfg.block // sub
    return O.pool_max(r64, pool), O.pool_max(mag, pool)


def certificate_d(cfg, kw):
    """Length of the float32 dot products behind a case's scores (projections add d')."""
    return cfg.d + (16 if ("proj_seed" in kw or "proj_pair_seed" in kw) else 0)


@pytest.mark.parametrize("case", list(ROUTE_CASES))
def test_oracle_selection_matches_reference(case):
    cfg_name, variant, mode, kw = ROUTE_CASES[case]
    g = GU.load(case)
    p = WL.make(cfg_name, variant)
    assert GU.sha(p["q"], p["k"]) == str(g["inputs_sha256"]), "generator drifted from the fixture"
    kv_num, kv_idx = oracle_route(p, mode, dict(kw))
    r64, mag = certificate_inputs(p, mode, kw)
    n, n_eq, n_cert, bad = GU.compare_selections(kv_num, kv_idx, g["kv_num"], g["kv_idx"], r64, mag,
                                                 d=certificate_d(p["cfg"], kw))
    print(f"{case}: {n} rows, {n_eq} identical, {n_cert} certified float32 near-ties")
    assert not bad, bad[:5]
    # the certificate must be rare: these inputs are not adversarial
    assert n_cert <= max(2, n // 1000), (n_cert, n)


def test_oracle_decode_selection_matches_reference():
    g = GU.load("c4_query")
    p = WL.make("C4", n=65536 + 128)
    assert GU.sha(p["q"], p["k"]) == str(g["inputs_sha256"])
    cfg = p["cfg"]
    for a, pos in enumerate(g["positions"].tolist()):
        rows = p["q"][:, :, pos:pos + 1]
        kv_num, kv_idx = O.route_query(rows, p["k"], cfg.block, pos, top_c=cfg.top_c,
                                       local=cfg.local, beta=cfg.beta, kv_len=pos + 1)
        mu, var, _ = O.block_stats(p["k"][:, :, :pos + 1], cfg.block, "pop")
        r64, mag = O.exact_scores64(rows, mu, var, 0.5 * cfg.beta)
        n, n_eq, n_cert, bad = GU.compare_selections(kv_num[:, :, 0], kv_idx[:, :, 0],
                                                     g["kv_num"][a][None], g["kv_idx"][a][None],
                                                     r64[:, :, 0], mag[:, :, 0])
        assert not bad and n_eq + n_cert == n, (pos, bad)


def test_oracle_attention_matches_reference_flex_output():
    """ssa_flex (FlexAttention, float32, CPU) on C1 vs the oracle's exact masked softmax over
    the oracle's block_route selection: within the float32 tolerance 1e-5."""
    g = GU.load("c1_flex_out")
    p = WL.make("C1")
    assert GU.sha(p["q"], p["k"], p["v"]) == str(g["inputs_sha256"])
    kv_num, kv_idx = O.route_flat(p["q"], p["k"], 64, top_c=8, local=1)
    out = O.sparse_attention(p["q"], p["k"], p["v"], kv_num, kv_idx, 64)
    err = np.abs(out - g["out"]).max()
    assert err < 1e-5, err


def test_oracle_analytic_path_matches_reference():
    """Per-query routing + masked softmax (ssa_attention_forward impl='analytic', float64,
    GQA 2:1, n=300 not a block multiple) and the q_len=1 decode row."""
    g = GU.load("analytic_gqa")
    rng = np.random.default_rng(11)
    q = rng.standard_normal((1, 4, 300, 64))
    k = rng.standard_normal((1, 2, 300, 64))
    v = rng.standard_normal((1, 2, 300, 64))
    assert GU.sha(q, k, v) == str(g["inputs_sha256"])
    kv_num, kv_idx = O.route_query(q, k, 64, 0, top_c=None, budget_frac=0.5, local=1, beta=2.0)
    out = O.attend_rows(q, k, v, kv_num, kv_idx, 0, 64, scale=0.125)
    ref = g["out"].transpose(0, 2, 1, 3)
    # the reference takes its softmax in float32 even for float64 inputs (gemma_ssa.py:239),
    # so it carries float32 rounding of the weights (~1e-7); a selection difference would be O(0.1)
    assert np.abs(out - ref).max() < 2e-6
    assert np.abs(out[:, :, -1] - g["out_last"][:, 0]).max() < 2e-6


def test_oracle_analytic_edgeworth_matches_reference():
    """The per-query router with the edgeworth term (ssa/gemma_ssa.py:101-102) on skewed keys:
    the oracle's routing + masked softmax equals the reference's float64 analytic output, and
    dropping the term (a plausible slip) fails the same fixture."""
    g = GU.load("analytic_gqa_edgeworth")
    q, k, v = GU.analytic_inputs(12, skew=0.7)
    assert GU.sha(q, k, v) == str(g["inputs_sha256"])
    ref = g["out"].transpose(0, 2, 1, 3)
    outs = {}
    for edge in (True, False):
        kv_num, kv_idx = O.route_query(q, k, 64, 0, top_c=None, budget_frac=0.5, local=1,
                                       beta=2.0, edgeworth=edge)
        outs[edge] = O.attend_rows(q, k, v, kv_num, kv_idx, 0, 64, scale=0.125)
    assert np.abs(outs[True] - ref).max() < 2e-6
    assert np.abs(outs[True][:, :, -1] - g["out_last"][:, 0]).max() < 2e-6
    assert np.abs(outs[False] - ref).max() > 1e-2


def test_oracle_c5_geometry_prefix_matches_reference():
    """block_route_budget at C5's geometry (fp16, block 256, top_c 64, local 1, beta 2) on the
    2,097,152-token prefix (8192 query blocks): the oracle's selections equal the reference's
    float32 selections except on certified float32 near-ties."""
    g = GU.load("c5_prefix")
    p = WL.make_c5_prefix()
    cfg = p["cfg"]
    assert GU.sha(p["q"], p["k"]) == str(g["inputs_sha256"])
    onum, oidx = O.route_budget(p["q"], p["k"], cfg.block, top_c=cfg.top_c, local=cfg.local,
                                beta=cfg.beta)
    qb = O.qmean(p["q"], cfg.block)
    mu, var, _ = O.block_stats(p["k"], cfg.block, "pop")
    r64, mag = O.exact_scores64(qb, mu, var, 0.5 * cfg.beta)
    n, n_eq, n_cert, bad = GU.compare_selections(onum, oidx, g["kv_num"], g["kv_idx"], r64, mag)
    print(f"c5_prefix: {n} rows, {n_eq} identical, {n_cert} certified near-ties")
    assert not bad, bad[:3]
    assert n_eq >= n - 8


def test_oracle_decode_router_full_1m_cache_matches_reference():
    """_selection_mask at q_len = 1 over the full 1,048,576-token C4 cache (plus the appended
    tokens) at three decode steps, the last completing a block: the oracle's per-query router
    equals the reference's float32 selection on every head (or differs on a certified
    near-tie)."""
    g = GU.load("c4_query_1m")
    p = WL.make_decode(steps=GU.C4_1M_STEPS)
    cfg, n = p["cfg"], p["n_cache"]
    assert GU.sha(p["q"], p["k"]) == str(g["inputs_sha256"])
    # every block complete at the checked steps is complete in the first n + 128 tokens
    mu, var, _ = O.block_stats(p["k"][:, :, :n + 128], cfg.block, "pop")
    steps = g["steps"].tolist()
    assert max(steps) < 128
    # the summary shortcut equals the per-position restatement (checked on the first step)
    t0 = steps[0]
    a0 = O.route_query(p["q"][:, :, t0:t0 + 1], p["k"], cfg.block, n + t0, top_c=cfg.top_c,
                       local=cfg.local, beta=cfg.beta, kv_len=n + t0 + 1)
    b0 = O.route_query_summaries(p["q"][:, :, t0:t0 + 1], mu, var, cfg.block, n + t0,
                                 top_c=cfg.top_c, local=cfg.local, beta=cfg.beta)
    assert all((x == y).all() for x, y in zip(a0, b0))
    for a, t in enumerate(steps):
        pos = n + t
        qrow = p["q"][:, :, t:t + 1]
        onum, oidx = O.route_query_summaries(qrow, mu, var, cfg.block, pos, top_c=cfg.top_c,
                                             local=cfg.local, beta=cfg.beta)
        r64, mag = O.exact_scores64(qrow, mu, var, 0.5 * cfg.beta)
        n_, n_eq, n_cert, bad = GU.compare_selections(onum[:, :, 0], oidx[:, :, 0],
                                                      g["kv_num"][a][None], g["kv_idx"][a][None],
                                                      r64[:, :, 0], mag[:, :, 0])
        assert not bad, (t, bad)
        assert int(onum.max()) <= cfg.top_c + cfg.local + 1


# ---- mathematics -------------------------------------------------------------------------------

def test_block_stats_closed_form():
    x = np.zeros((1, 1, 10, 8), dtype=np.float32)
    x[0, 0, :, 0] = np.arange(10)             # block of 4: 0..3 -> mean 1.5, pop var 1.25
    x[0, 0, :, 1] = 2.0                       # constant column -> var 0
    mu, var, m3 = O.block_stats(x, 4, "pop")
    assert mu.shape == (1, 1, 3, 8)
    assert mu[0, 0, 0, 0] == 1.5 and var[0, 0, 0, 0] == 1.25 and m3[0, 0, 0, 0] == 0.0
    assert var[0, 0, 0, 1] == 0.0 and mu[0, 0, 1, 1] == 2.0
    # last block holds rows 8, 9 only (n=10): mean 8.5, pop var 0.25
    assert mu[0, 0, 2, 0] == 8.5 and var[0, 0, 2, 0] == 0.25
    _, uvar, _ = O.block_stats(x, 4, "unbiased")
    assert uvar[0, 0, 0, 0] == np.float32(5.0 / 3.0)
    # n_real excludes pad rows: rows >= 9 dropped -> block 2 = {8}
    mu2, var2, _ = O.block_stats(x, 4, "pop", n_real=9)
    assert mu2[0, 0, 2, 0] == 8.0 and var2[0, 0, 2, 0] == 0.0
    # skew of {0, 0, 0, 4}: mean 1, m3 = (3*(-1)^3 + 27)/4 = 6
    y = np.zeros((1, 1, 4, 8), dtype=np.float32)
    y[0, 0, 3, 0] = 4.0
    assert O.block_stats(y, 4, "pop")[2][0, 0, 0, 0] == 6.0
    # query mean counts pad rows as zeros
    assert O.qmean(x, 4)[0, 0, 2, 0] == np.float32((8 + 9) / 4)


def test_scores_closed_form():
    rows = np.array([[[[1.0, 2.0]]]], dtype=np.float32)           # (1,1,1,2)
    mu = np.array([[[[3.0, -1.0], [0.5, 0.5]]]], dtype=np.float32)
    var = np.array([[[[2.0, 1.0], [0.0, 4.0]]]], dtype=np.float32)
    r = O.scores(rows, mu, var, coef2=1.0)
    # <q,mu> + 1.0*<q^2,var>: (3-2) + (2+4) = 7 ; (0.5+1) + (0+16) = 17.5
    assert r[0, 0, 0].tolist() == [7.0, 17.5]
    m3 = np.array([[[[1.0, 0.0], [0.0, -1.0]]]], dtype=np.float32)
    r3 = O.scores(rows, mu, var, 1.0, m3, coef3=2.0 / 3.0)
    assert np.allclose(r3[0, 0, 0], [7.0 + 2.0 / 3.0, 17.5 - 16.0 / 3.0], atol=1e-5)


def test_select_matches_bruteforce_ranking():
    """select_rows against an independent O(n^2) rank count, with forced exact ties."""
    rng = np.random.default_rng(5)
    for trial in range(40):
        nbk = int(rng.integers(2, 24))
        r = rng.integers(-3, 4, size=(1, 1, nbk, nbk)).astype(np.float32)   # many exact ties
        top_c = int(rng.integers(0, 6))
        local = int(rng.integers(0, 3))
        mode = ["budget", "flat"][trial % 2]
        got = O.select_rows(r, mode, top_c, 0.0, local)
        for i in range(nbk):
            cmax = i if mode == "budget" else i + 1
            k = min(top_c, cmax)
            row = r[0, 0, i, :cmax]
            rank = [sum(1 for y in range(cmax) if row[y] > row[x] or (row[y] == row[x] and y < x))
                    for x in range(cmax)]
            pick = {x for x in range(cmax) if rank[x] < k}
            pick |= set(range(max(0, i - local), i + 1))
            assert got[0, 0, i] == sorted(pick), (trial, i)


def test_budget_keep_is_float32_ceil():
    # ceil(fl32(0.1) * 10) = ceil(1.0000000149 rounded to fp32 = 1.0) = 1, not 2
    assert O._keep_budget(0.1, 10) == 1
    assert O._keep_budget(0.25, 0) == 1
    assert O._keep_budget(0.3, 7) == 3      # fl32(0.3)*7 = 2.1000001 -> 3
    assert O._keep_budget(1.0, 37) == 37


def test_full_budget_equals_dense():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 4, 200, 16))
    k = rng.standard_normal((1, 2, 200, 16))
    v = rng.standard_normal((1, 2, 200, 16))
    kv_num, kv_idx = O.route_budget(q, k, 32, budget_frac=1.0, local=1, n_real=200)
    assert (kv_num[0, 0] == np.arange(1, 8)).all()
    out = O.sparse_attention(q, k, v, kv_num, kv_idx, 32, n=200)
    assert np.abs(out - O.dense_causal(q, k, v)).max() < 1e-12


def test_needle_known_answer():
    """test_gemma_ssa.py:100-121 restated: top_c=1, no local window, a key 12*u aligned with the
    probe query in block 1 -> per-query routing selects it and the probe output is its value."""
    rng = np.random.default_rng(0)
    d, n, block = 64, 128, 32
    q = rng.standard_normal((1, 1, n, d))
    k = rng.standard_normal((1, 1, n, d))
    v = rng.standard_normal((1, 1, n, d))
    u = rng.standard_normal(d)
    u /= np.linalg.norm(u)
    q[0, 0, n - 1] = u
    k[0, 0, 40] = 12.0 * u
    v[0, 0, 40] = np.arange(d) / d
    kv_num, kv_idx = O.route_query(q[:, :, -1:], k, block, n - 1, top_c=1, local=0, beta=2.0)
    assert 1 in kv_idx[0, 0, 0, :kv_num[0, 0, 0]].tolist()
    out = O.decode_attend(q[0, 0, -1], k[0, 0], v[0, 0], kv_idx[0, 0, 0, :kv_num[0, 0, 0]], n - 1,
                          block, scale=1.0)
    assert np.abs(out - v[0, 0, 40]).max() < 3e-3


def test_budget_router_invariants():
    """test_flex_swap.py:49-73 restated: causal, own block kept, counts monotone in budget."""
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 1, 32 * 128, 64)).astype(np.float32)
    k = rng.standard_normal((1, 1, 32 * 128, 64)).astype(np.float32)
    kv_num, kv_idx = O.route_budget(q, k, 128, budget_frac=0.25, local=1)
    for i in range(32):
        ids = kv_idx[0, 0, i, :kv_num[0, 0, i]].tolist()
        assert all(c <= i for c in ids) and i in ids
    counts = [int(O.route_budget(q, k, 128, budget_frac=f, local=0)[0].sum())
              for f in (1.0, 0.5, 0.25, 0.1)]
    assert counts[0] > counts[1] > counts[2] >= counts[3], counts


def test_decode_row_equals_prefill_row():
    """decode_attend over a query block's selection reproduces that block's last prefill row
    (test_ivf_decode.py:14-29 restated)."""
    rng = np.random.default_rng(3)
    n, block = 12 * 64, 64
    q = rng.standard_normal((1, 1, n, 64))
    k = rng.standard_normal((1, 1, n, 64))
    v = rng.standard_normal((1, 1, n, 64))
    kv_num, kv_idx = O.route_budget(q, k, block, top_c=4, local=1)
    pre = O.sparse_attention(q, k, v, kv_num, kv_idx, block, qblocks=[11])
    row = O.decode_attend(q[0, 0, n - 1], k[0, 0], v[0, 0], kv_idx[0, 0, 11, :kv_num[0, 0, 11]],
                          n - 1, block)
    assert np.abs(row - pre[0, 0, n - 1]).max() < 1e-12


def test_keys_order_and_special_values():
    r = np.array([-np.inf, -2.0, -0.0, 0.0, 1e-30, 3.0, np.inf, np.nan], dtype=np.float32)
    k = O.score_keys(r)
    assert (np.diff(k[:2].astype(np.int64)) > 0).all()
    assert k[2] == k[3]                                     # -0 == +0
    assert list(np.argsort(k[[0, 1, 3, 4, 5, 6, 7]], kind="stable")) == list(range(7))
    assert math.isnan(float(r[7])) and k[7] == np.uint32(0xFFFFFFFF)


def test_oracle_sub_identity_and_planted_subblock():
    """sub=None / sub=block are the default route; with centroid scores (beta = 0) sub=32 finds
    a planted coherent 32-key sub-block whose block mean is diluted 4x (the reference's
    test_cascade_router.py:147-167, which it skips; with beta = 2 the variance bonus of random
    sub-blocks, ~|q|^2, hides the variance-free needle)."""
    rng = np.random.default_rng(23)
    n, block = 8 * 128, 128
    q = rng.standard_normal((1, 1, n, 64)).astype(np.float32)
    k = rng.standard_normal((1, 1, n, 64)).astype(np.float32)
    a = O.route_budget(q, k, block, top_c=2, local=1)
    for sub in (None, block):
        b = O.route_budget(q, k, block, top_c=2, local=1, sub=sub)
        assert (a[0] == b[0]).all() and (a[1] == b[1]).all()
    u = rng.standard_normal(64)
    u = (u / np.linalg.norm(u)).astype(np.float32)
    q[0, 0, n - block:] = u
    k[0, 0, block:block + 32] = u
    qblk = (n - 1) // block
    num, idx = O.route_budget(q, k, block, top_c=1, local=0, sub=32, beta=0.0)
    assert idx[0, 0, qblk, :num[0, 0, qblk]].tolist() == [1, qblk]
    qb = O.qmean(q, block)
    mu, var, _ = O.block_stats(k, 32, "pop")
    r = O.scores(qb, mu, var, 0.0)
    # max-pooling by hand: the pooled score of block 1 is its best sub-block's score (~1), the
    # block-mean score is diluted to ~1/4
    assert O.pool_max(r, 4)[0, 0, qblk, 1] == r[0, 0, qblk, 4:8].max()
    mub, _, _ = O.block_stats(k, block, "pop")
    rb = O.scores(qb, mub, None, 0.0)
    assert r[0, 0, qblk, 4] > 0.99 and 0.15 < rb[0, 0, qblk, 1] < 0.35


def test_oracle_proj_identity_equals_centroid_routing():
    """proj = I reproduces beta = 0 exactly (test_share_route.py:27-37); a projection to d'
    columns equals routing on explicitly projected summaries."""
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 1, 8 * 128, 64)).astype(np.float32)
    k = rng.standard_normal((1, 1, 8 * 128, 64)).astype(np.float32)
    a = O.route_budget(q, k, 128, top_c=3, local=1, proj=np.eye(64, dtype=np.float32))
    b = O.route_budget(q, k, 128, top_c=3, local=1, beta=0.0)
    assert (a[0] == b[0]).all() and (a[1] == b[1]).all()
    w = WL.proj_matrix(5)
    qp = (q[0, 0].astype(np.float64) @ w)
    assert np.array_equal(O.project(q[0, 0], w), qp.astype(np.float32))


# ---- f3: ssa_swap.ssa_masked -------------------------------------------------------------------

def _masked_case(name):
    seed, (b, h, n, d), block, top_c, local = GU.MASKED_CASES[name]
    q, k, v, g = GU.masked_inputs(seed, b, h, n, d)
    ref = GU.load(name)
    assert GU.sha(q, k, v, g) == str(ref["inputs_sha256"])
    return q, k, v, g, block, top_c, local, ref


@pytest.mark.parametrize("name", list(GU.MASKED_CASES))
def test_oracle_masked_matches_reference(name):
    """Selection, forward and q/k/v gradients of ssa_masked (ssa/ssa_swap.py:32-56, the
    reference run in float32 with torch autograd) against the float64 oracle."""
    q, k, v, g, block, top_c, local, ref = _masked_case(name)
    sel = O.masked_route(q, k, block, top_c, local)
    out, _ = O.masked_forward(q, k, v, sel, block)
    dq, dk, dv = O.masked_grads(q, k, v, sel, g, block)
    for got, key in ((out, "out"), (dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert np.abs(got - ref[key]).max() < 1e-5, key


def test_oracle_masked_planted_mistakes_fail():
    """Each plausible slip in the routing statistics or geometry changes the output of the b16
    fixture far beyond the 1e-5 bar: biased variance, pad rows left out of the statistics,
    complete-block (rather than begun-block) candidates."""
    q, k, v, g, block, top_c, local, ref = _masked_case("swap_masked_b16")
    n = q.shape[2]
    kp = np.pad(k, ((0, 0), (0, 0), (0, -n % block), (0, 0)))
    variants = {
        "biased": (O.block_stats(kp, block, "pop"), "started"),
        "pad_excluded": (O.block_stats(k, block, "unbiased", n_real=n), "started"),
        "complete_blocks": (O.block_stats(kp, block, "unbiased"), "query"),
    }
    for nm, ((mu, var, _), mode) in variants.items():
        sel = O.select_rows(O.scores(q, mu, var, 0.5), mode, top_c, 0.0, local, 0, block)
        out, _ = O.masked_forward(q, k, v, sel, block)
        assert np.abs(out - ref["out"]).max() > 1e-2, nm


def test_masked_full_selection_equals_dense_and_autograd():
    """top_c >= number of blocks: every begun block is kept, so the masked forward is dense
    causal softmax, and its gradients equal torch autograd of dense causal attention (float64)."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    q, k, v, g = (rng.standard_normal((1, 2, 70, 16)) for _ in range(4))
    sel = O.masked_route(q.astype(np.float32), k.astype(np.float32), 16, 99, 0)
    assert [len(x) for x in sel[0, 0]] == [i // 16 + 1 for i in range(70)]
    out, lse = O.masked_forward(q, k, v, sel, 16)
    assert np.abs(out - O.dense_causal(q, k, v)).max() < 1e-12
    tq, tk, tv = (torch.from_numpy(x).requires_grad_(True) for x in (q, k, v))
    s = (tq @ tk.transpose(-1, -2)) * 0.25
    s = s.masked_fill(torch.ones(70, 70, dtype=torch.bool).triu(1), float("-inf"))
    assert np.abs(torch.logsumexp(s, -1).detach().numpy() - lse).max() < 1e-12
    (torch.softmax(s, -1) @ tv).backward(torch.from_numpy(g))
    dq, dk, dv = O.masked_grads(q, k, v, sel, g, 16)
    for got, t in ((dq, tq), (dk, tk), (dv, tv)):
        assert np.abs(got - t.grad.numpy()).max() < 1e-12


def test_masked_grads_finite_differences():
    """Gradients of sum(out * g) with the selection held fixed, by central differences on a
    sparse selection with GQA 2:1 (top_c=1, local=0)."""
    rng = np.random.default_rng(4)
    q = rng.standard_normal((1, 4, 40, 8))
    k, v = (rng.standard_normal((1, 2, 40, 8)) for _ in range(2))
    g = rng.standard_normal((1, 4, 40, 8))
    sel = O.masked_route(q.astype(np.float32), k.astype(np.float32), 8, 1, 0)
    assert max(len(x) for x in sel.ravel()) == 2 and min(len(x) for x in sel.ravel()) == 1
    dq, dk, dv = O.masked_grads(q, k, v, sel, g, 8)

    def loss(q_, k_, v_):
        return float((O.masked_forward(q_, k_, v_, sel, 8)[0] * g).sum())

    eps = 1e-6
    for arr, grad, which in ((q, dq, 0), (k, dk, 1), (v, dv, 2)):
        for idx in [(0, 1, 5, 3), (0, 1, 33, 0), (0, 0, 17, 7)]:
            plus, minus = [x.copy() for x in (q, k, v)], [x.copy() for x in (q, k, v)]
            plus[which][idx] += eps
            minus[which][idx] -= eps
            fd = (loss(*plus) - loss(*minus)) / (2 * eps)
            assert abs(fd - grad[idx]) < 1e-6 * max(1.0, abs(fd)), (which, idx, fd, grad[idx])
